// broadcast.hip -- a bias shared by every row of a batch, and its reverse rule (f32, f64).
//
// The reference adds a bias of the operand's own shape (examples/xor_tensor.cleave:44-49,
// one example at a time: matmul(x, w) + b1 with both 1 x n), because Ring<Tensor>::add
// needs equal shapes (stdlib/linalg/tensor.cleave:66-71).  A batch of rows needs the
// broadcast form out[i][j] = a[i][j] + b[j]; its reverse rule is db[j] = sum_i g[i][j],
// the cotangent summed over the broadcast dimension.
//
// Both are HBM-bound.  Threads own one 16-byte column chunk and walk a group of rows,
// so every wave reads and writes whole 1 KiB row segments; the bias chunk (or the
// column accumulator) stays in registers.  The column sums add each row group in
// ascending row order, then the group partials in ascending group order: a fixed
// order, so results are deterministic for a given shape.
#include "common.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kRowUnroll = 4;

// A 16-byte column chunk: 4 floats or 2 doubles.
template <class T>
struct Chunk {
    static constexpr int kN = 16 / sizeof(T);
    typedef T type __attribute__((ext_vector_type(kN)));
};
template <class T>
__device__ __forceinline__ typename Chunk<T>::type ldnt(const T* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const typename Chunk<T>::type*>(p));
}
template <class T>
__device__ __forceinline__ void stnt(T* p, typename Chunk<T>::type v) {
    __builtin_nontemporal_store(v, reinterpret_cast<typename Chunk<T>::type*>(p));
}

// Launch shape of both kernels: blockIdx.x = group * nseg + seg, where seg
// picks kThreads column chunks and group a run of rows_per_group rows.
struct Tiling {
    int64_t cv = 0;          // 16-byte column chunks per row (cols / elements per chunk)
    int64_t nseg = 0;        // column segments of kThreads chunks
    int64_t groups = 0;      // row groups
    int64_t rows_per_group = 0;
};

Tiling tiling_rows(int64_t rows, int64_t cols, int64_t rows_per_group, int per_chunk) {
    Tiling t;
    t.cv = cols / per_chunk;
    t.nseg = (t.cv + kThreads - 1) / kThreads;
    t.rows_per_group = rows_per_group < rows ? rows_per_group : rows;
    t.groups = (rows + t.rows_per_group - 1) / t.rows_per_group;
    return t;
}
// The bias add moves every element once, so short row groups (many blocks, as a
// one-shot map) keep the most bytes in flight: 8 rows per block measured
// 6.6 TB/s at 65536 x 4096 against 4.8 TB/s for 128.
Tiling tiling_bias(int64_t rows, int64_t cols, int per_chunk) { return tiling_rows(rows, cols, 8, per_chunk); }
// The column sums write one partial row per group, which the second stage
// reads back; about four blocks per CU in the first stage measured best
// (6.75 TB/s at 65536 x 4096, 256 groups).
Tiling tiling_sum(int64_t rows, int64_t cols, int per_chunk) {
    const int64_t nseg = (cols / per_chunk + kThreads - 1) / kThreads;
    int64_t groups = 4LL * ch::num_cus() / nseg;
    if (groups < 1) groups = 1;
    if (groups > rows) groups = rows;
    return tiling_rows(rows, cols, (rows + groups - 1) / groups, per_chunk);
}

template <class T>
__global__ __launch_bounds__(kThreads) void add_row_bias_kernel(const T* __restrict__ a, const T* __restrict__ bias,
                                                                T* __restrict__ out, int64_t rows, int64_t cols,
                                                                int64_t nseg, int64_t rpg) {
    typedef typename Chunk<T>::type V;
    const int64_t seg = blockIdx.x % nseg, group = blockIdx.x / nseg;
    const int64_t c = (seg * kThreads + threadIdx.x) * Chunk<T>::kN;
    if (c >= cols) return;
    const V b = *reinterpret_cast<const V*>(bias + c);
    const int64_t r0 = group * rpg;
    const int64_t r1 = r0 + rpg < rows ? r0 + rpg : rows;
    int64_t r = r0;
    for (; r + kRowUnroll <= r1; r += kRowUnroll) {
        V v[kRowUnroll];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) v[u] = ldnt(a + (r + u) * cols + c);
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) stnt(out + (r + u) * cols + c, v[u] + b);
    }
    for (; r < r1; ++r) stnt(out + r * cols + c, ldnt(a + r * cols + c) + b);
}

template <class T>
__global__ __launch_bounds__(kThreads) void sum_rows_stage1(const T* __restrict__ g, T* __restrict__ part,
                                                            int64_t rows, int64_t cols, int64_t nseg, int64_t rpg) {
    typedef typename Chunk<T>::type V;
    const int64_t seg = blockIdx.x % nseg, group = blockIdx.x / nseg;
    const int64_t c = (seg * kThreads + threadIdx.x) * Chunk<T>::kN;
    if (c >= cols) return;
    const int64_t r0 = group * rpg;
    const int64_t r1 = r0 + rpg < rows ? r0 + rpg : rows;
    V acc = ldnt(g + r0 * cols + c);
    int64_t r = r0 + 1;
    for (; r + kRowUnroll <= r1; r += kRowUnroll) {
        V v[kRowUnroll];
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) v[u] = ldnt(g + (r + u) * cols + c);
#pragma unroll
        for (int u = 0; u < kRowUnroll; ++u) acc = acc + v[u];
    }
    for (; r < r1; ++r) acc = acc + ldnt(g + r * cols + c);
    *reinterpret_cast<V*>(part + group * cols + c) = acc;
}

// out[j] = the sum of part[0..groups)[j].  Eight threads share a column:
// thread s left-folds groups [s*G/8, (s+1)*G/8) with eight loads in flight,
// then thread 0 folds the eight partials in order s = 0..7, so the result is
// deterministic.  A block covers 32 columns; the 32 threads of a half-wave
// that share s read 128 contiguous bytes of a partial row.  At 65536 x 4096
// this stage takes 5.4 us (sixteen threads per column: the same); one thread
// per column, folding all 256 groups itself, left 16 blocks and took 12.4 us.
constexpr int kGroupUnroll = 8;
constexpr int kStage2Split = 8, kStage2Cols = kThreads / kStage2Split;
template <class T>
__global__ __launch_bounds__(kThreads) void sum_rows_stage2(const T* __restrict__ part, T* __restrict__ out,
                                                            int64_t groups, int64_t cols) {
    __shared__ T red[kStage2Split][kStage2Cols];
    const int jj = threadIdx.x % kStage2Cols, s = threadIdx.x / kStage2Cols;
    const int64_t j = (int64_t)blockIdx.x * kStage2Cols + jj;
    const int64_t q0 = groups * s / kStage2Split, q1 = groups * (s + 1) / kStage2Split;
    T acc = T(0);
    if (j < cols && q0 < q1) {
        acc = part[q0 * cols + j];
        int64_t q = q0 + 1;
        for (; q + kGroupUnroll <= q1; q += kGroupUnroll) {
            T v[kGroupUnroll];
#pragma unroll
            for (int u = 0; u < kGroupUnroll; ++u) v[u] = part[(q + u) * cols + j];
#pragma unroll
            for (int u = 0; u < kGroupUnroll; ++u) acc = acc + v[u];
        }
        for (; q < q1; ++q) acc = acc + part[q * cols + j];
    }
    red[s][jj] = acc;
    __syncthreads();
    if (s == 0 && j < cols) {
        // fold the non-empty chunks in order (a chunk is empty only when
        // groups < 8; the last one never is)
        int t = 0;
        while (groups * (t + 1) / kStage2Split == groups * t / kStage2Split) ++t;
        T r = red[t][jj];
        for (++t; t < kStage2Split; ++t)
            if (groups * (t + 1) / kStage2Split > groups * t / kStage2Split) r = r + red[t][jj];
        out[j] = r;
    }
}

// Scalar forms for widths that are not a multiple of 4 or unaligned pointers.
template <class T>
__global__ void add_row_bias_scalar(const T* a, const T* bias, T* out, int64_t rows, int64_t cols) {
    const int64_t n = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = a[i] + bias[i % cols];
}
template <class T>
__global__ void sum_rows_scalar(const T* g, T* out, int64_t rows, int64_t cols) {
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < cols; j += (int64_t)gridDim.x * blockDim.x) {
        T acc = g[j];
        for (int64_t r = 1; r < rows; ++r) acc = acc + g[r * cols + j];
        out[j] = acc;
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

unsigned blocks_for(int64_t n) {
    int64_t b = (n + kThreads - 1) / kThreads;
    if (b > 65536) b = 65536;
    return (unsigned)(b < 1 ? 1 : b);
}

template <class T>
int32_t run_add_row_bias(const char* fn, const T* a, int64_t alen, const T* bias, int64_t blen, T* out,
                         int64_t outlen, int32_t rows, int32_t cols) {
    constexpr int V = Chunk<T>::kN;
    CH_REQUIRE(rows >= 0 && cols >= 0, "%s: negative shape (%d x %d)", fn, rows, cols);
    CH_REQUIRE(alen == (int64_t)rows * cols && outlen == alen, "%s: a/out lengths (%lld, %lld) != rows*cols %lld",
               fn, (long long)alen, (long long)outlen, (long long)rows * cols);
    CH_REQUIRE(blen == cols, "%s: bias length %lld != cols %d", fn, (long long)blen, cols);
    if (alen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(a && bias && out, "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, a, alen * sizeof(T));
    CH_DEVICE(fn, bias, blen * sizeof(T));
    CH_DEVICE(fn, out, outlen * sizeof(T));
    if (cols % V == 0 && aligned16(a) && aligned16(bias) && aligned16(out)) {
        const Tiling t = tiling_bias(rows, cols, V);
        add_row_bias_kernel<T><<<(unsigned)(t.nseg * t.groups), kThreads, 0, ch::stream()>>>(
            a, bias, out, rows, cols, t.nseg, t.rows_per_group);
    } else {
        add_row_bias_scalar<T><<<blocks_for(alen), kThreads, 0, ch::stream()>>>(a, bias, out, rows, cols);
    }
    CH_LAUNCHED(fn);
    return CLEAVE_HIP_OK;
}

template <class T>
int32_t run_sum_rows(const char* fn, const T* g, int64_t glen, T* out, int64_t outlen, int32_t rows, int32_t cols) {
    constexpr int V = Chunk<T>::kN;
    CH_REQUIRE(rows >= 1 && cols >= 0, "%s: need at least one row (%d x %d)", fn, rows, cols);
    CH_REQUIRE(glen == (int64_t)rows * cols, "%s: g length %lld != rows*cols %lld", fn, (long long)glen,
               (long long)rows * cols);
    CH_REQUIRE(outlen == cols, "%s: out length %lld != cols %d", fn, (long long)outlen, cols);
    if (cols == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(g && out, "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, g, glen * sizeof(T));
    CH_DEVICE(fn, out, outlen * sizeof(T));
    if (cols % V == 0 && aligned16(g)) {
        const Tiling t = tiling_sum(rows, cols, V);
        T* part = (T*)ch::scratch(5, sizeof(T) * (size_t)(t.groups * cols));
        if (!part) return ch::fail(CLEAVE_HIP_ERR_OOM, "%s: scratch of %lld elements", fn, (long long)(t.groups * cols));
        sum_rows_stage1<T><<<(unsigned)(t.nseg * t.groups), kThreads, 0, ch::stream()>>>(g, part, rows, cols, t.nseg,
                                                                                          t.rows_per_group);
        CH_LAUNCHED(fn);
        sum_rows_stage2<T><<<(unsigned)((cols + kStage2Cols - 1) / kStage2Cols), kThreads, 0, ch::stream()>>>(
            part, out, t.groups, cols);
    } else {
        sum_rows_scalar<T><<<blocks_for(cols), kThreads, 0, ch::stream()>>>(g, out, rows, cols);
    }
    CH_LAUNCHED(fn);
    return CLEAVE_HIP_OK;
}

}  // namespace

extern "C" {

int32_t cleave_hip_add_row_bias_f32(const float* a, int64_t alen, const float* bias, int64_t blen, float* out,
                                    int64_t outlen, int32_t rows, int32_t cols) {
    return run_add_row_bias<float>("cleave_hip_add_row_bias_f32", a, alen, bias, blen, out, outlen, rows, cols);
}

int32_t cleave_hip_sum_rows_f32(const float* g, int64_t glen, float* out, int64_t outlen, int32_t rows,
                                int32_t cols) {
    return run_sum_rows<float>("cleave_hip_sum_rows_f32", g, glen, out, outlen, rows, cols);
}

int32_t cleave_hip_add_row_bias_f64(const double* a, int64_t alen, const double* bias, int64_t blen, double* out,
                                    int64_t outlen, int32_t rows, int32_t cols) {
    return run_add_row_bias<double>("cleave_hip_add_row_bias_f64", a, alen, bias, blen, out, outlen, rows, cols);
}

int32_t cleave_hip_sum_rows_f64(const double* g, int64_t glen, double* out, int64_t outlen, int32_t rows,
                                int32_t cols) {
    return run_sum_rows<double>("cleave_hip_sum_rows_f64", g, glen, out, outlen, rows, cols);
}

}  // extern "C"
