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

// ---- Broadcasting maps and their reverse rule ----------------------------
//
// out = a op b for operands whose shapes broadcast: the shapes are aligned at
// their last dimension, a missing leading dimension counts as 1, and a
// dimension of 1 stretches to the other operand's (numpy's rule).  The
// reference has none: its Ring<Tensor> maps need equal shapes
// (stdlib/linalg/tensor.cleave:66-71) and Activation<Tensor> is rank 1
// (stdlib/nn/nn.cleave:82).  Each output element is one IEEE operation on
// the two elements it maps to, so the results are bit-identical to the
// restated loop.
//
// The host collapses the shapes first: output dimensions of 1 drop out, and
// neighbours merge when both operands step through them alike (both
// contiguous across the pair, or both broadcast over it).  Equal shapes
// become one dimension and a row bias [rows, cols] with b's row stride 0.
// The kernel walks output rows (every collapsed dimension but the last) and
// the last dimension one 16-byte chunk per thread; an operand's stride in
// the last dimension is 1, or 0 when it is broadcast there, and whole
// vectors load when the last dimension is a multiple of the chunk and every
// base is 16-byte aligned.
//
// The reverse rule sums a cotangent of the output's shape over the
// dimensions that broadcasting stretched, down to an operand's shape.  Its
// dimensions collapse into runs that are kept or reduced: a leading reduced
// run over a kept one is the column sums above, a lone reduced run the
// library's Sum, a kept run over a long reduced one one wave per kept
// element (lanes stride the run, then a fixed-order tree), and any other
// pattern one thread per output element walking its reduced elements in
// row-major order.  Every path adds in an order fixed by the shape.

constexpr int kMaxRank = 8;

struct BDims {
    int rank;              // collapsed rank, >= 1
    int64_t n[kMaxRank];   // collapsed output dimensions
    int64_t sa[kMaxRank];  // a's element stride per collapsed dimension (0: broadcast)
    int64_t sb[kMaxRank];
};

struct BAdd { template <class T> __device__ T operator()(T a, T b) const { return a + b; } };
struct BSub { template <class T> __device__ T operator()(T a, T b) const { return a - b; } };
struct BMul { template <class T> __device__ T operator()(T a, T b) const { return a * b; } };
struct BDiv { template <class T> __device__ T operator()(T a, T b) const { return a / b; } };

// Offsets of output row `row` (a multi-index over the collapsed dimensions
// but the last) into a and b.
template <class I>
__device__ __forceinline__ void bcast_row_offsets(const BDims& d, I row, I& oa, I& ob) {
    oa = 0, ob = 0;
#pragma unroll
    for (int k = kMaxRank - 2; k >= 0; --k) {
        if (k < d.rank - 1) {
            const I nk = (I)d.n[k];
            const I q = row % nk;
            row /= nk;
            oa += q * (I)d.sa[k];
            ob += q * (I)d.sb[k];
        }
    }
}

// Rows of at least kRowChunks chunks: blocks take whole rows (grid-strided),
// compute the row's offsets once, and stride its chunks; operands read along
// the row and the output stream through non-temporal loads and stores, as in
// the same-shape maps.  Requires the VEC conditions.
constexpr int kRowChunks = 64;
template <class Op, class T, class I>
__global__ __launch_bounds__(kThreads) void bcast_rows_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                              T* __restrict__ out, BDims d, I rows, I chunks) {
    constexpr int V = Chunk<T>::kN;
    typedef typename Chunk<T>::type vec;
    const I inner = (I)d.n[d.rank - 1];
    const bool ia = d.sa[d.rank - 1] != 0, ib = d.sb[d.rank - 1] != 0;
    const Op op;
    for (I row = blockIdx.x; row < rows; row += gridDim.x) {
        I oa, ob;
        bcast_row_offsets(d, row, oa, ob);
        const T* pa = a + oa;
        const T* pb = b + ob;
        const vec sa = vec(pa[0]), sb = vec(pb[0]);
        T* o = out + row * inner;
        // four chunks per thread in flight: their loads, then their stores
        for (I c0 = threadIdx.x; c0 < chunks; c0 += 4 * kThreads) {
            vec va[4], vb[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const I c = c0 + u * kThreads;
                va[u] = sa, vb[u] = sb;
                if (c < chunks) {
                    if (ia) va[u] = ldnt(pa + c * V);
                    if (ib) vb[u] = ldnt(pb + c * V);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const I c = c0 + u * kThreads;
                if (c < chunks) {
                    vec r;
#pragma unroll
                    for (int t = 0; t < V; ++t) r[t] = op(va[u][t], vb[u][t]);
                    stnt(o + c * V, r);
                }
            }
        }
    }
}

// I: the index type, uint32_t when every operand has under 2^31 elements.
template <class Op, class T, bool VEC, class I>
__global__ __launch_bounds__(kThreads) void bcast_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                         T* __restrict__ out, BDims d, I rows, I chunks) {
    constexpr int V = Chunk<T>::kN;
    typedef typename Chunk<T>::type vec;
    const I inner = (I)d.n[d.rank - 1];
    const bool ia = d.sa[d.rank - 1] != 0, ib = d.sb[d.rank - 1] != 0;
    const I items = rows * chunks;
    const Op op;
    for (I it = (I)blockIdx.x * kThreads + threadIdx.x; it < items; it += (I)gridDim.x * kThreads) {
        I row = it / chunks;
        const I c0 = (it - row * chunks) * V;
        const I orow = row;
        I oa = 0, ob = 0;
#pragma unroll
        for (int k = kMaxRank - 2; k >= 0; --k) {
            if (k < d.rank - 1) {
                const I nk = (I)d.n[k];
                const I q = row % nk;
                row /= nk;
                oa += q * (I)d.sa[k];
                ob += q * (I)d.sb[k];
            }
        }
        T* o = out + orow * inner + c0;
        if constexpr (VEC) {
            vec va, vb, r;
            if (ia) va = *reinterpret_cast<const vec*>(a + oa + c0);
            else va = vec(a[oa]);
            if (ib) vb = *reinterpret_cast<const vec*>(b + ob + c0);
            else vb = vec(b[ob]);
#pragma unroll
            for (int t = 0; t < V; ++t) r[t] = op(va[t], vb[t]);
            *reinterpret_cast<vec*>(o) = r;
        } else {
#pragma unroll
            for (int t = 0; t < V; ++t)
                if (c0 + t < inner) o[t] = op(a[oa + (ia ? c0 + t : 0)], b[ob + (ib ? c0 + t : 0)]);
        }
    }
}

// Shape of a rank-r operand right-aligned into R dimensions (missing leading
// dimensions are 1); false when a dimension is negative.
bool align_shape(const int32_t* sh, int r, int R, int64_t* out) {
    for (int i = 0; i < R; ++i) {
        const int j = i - (R - r);
        out[i] = j < 0 ? 1 : sh[j];
        if (out[i] < 0) return false;
    }
    return true;
}

// Row-major element strides of shape d (rank R), 0 for dimensions of 1.
void bcast_strides(const int64_t* d, int R, int64_t* e) {
    int64_t st = 1;
    for (int i = R - 1; i >= 0; --i) {
        e[i] = d[i] == 1 ? 0 : st;
        st *= d[i];
    }
}

// Element count of shape d (rank R): 0 when a dimension is 0, -1 when the
// count exceeds int64 (no operand length matches it).
int64_t shape_prod(const int64_t* d, int R) {
    for (int i = 0; i < R; ++i)
        if (d[i] == 0) return 0;
    int64_t p = 1;
    for (int i = 0; i < R; ++i) {
        if (p > INT64_MAX / d[i]) return -1;
        p *= d[i];
    }
    return p;
}

// Checks that shapes (ash, ar) and (bsh, br) broadcast with the stated
// lengths and collapses them into *d.
int32_t plan_bcast(const char* fn, const int32_t* ash, int32_t ar, int64_t alen, const int32_t* bsh, int32_t br,
                   int64_t blen, int64_t outlen, BDims* d) {
    CH_REQUIRE(ar >= 0 && ar <= kMaxRank && br >= 0 && br <= kMaxRank, "%s: ranks %d and %d (each 0 .. %d)", fn,
               ar, br, kMaxRank);
    CH_REQUIRE((ar == 0 || ash) && (br == 0 || bsh), "%s: null shape array", fn);
    CH_REQUIRE(alen >= 0 && blen >= 0 && outlen >= 0, "%s: negative length (%lld, %lld, %lld)", fn,
               (long long)alen, (long long)blen, (long long)outlen);
    const int R = ar > br ? (ar > 0 ? ar : 1) : (br > 0 ? br : 1);
    int64_t da[kMaxRank], db[kMaxRank], n[kMaxRank], ea[kMaxRank], eb[kMaxRank];
    CH_REQUIRE(align_shape(ash, ar, R, da) && align_shape(bsh, br, R, db), "%s: negative dimension", fn);
    for (int i = 0; i < R; ++i) {
        CH_REQUIRE(da[i] == db[i] || da[i] == 1 || db[i] == 1,
                   "%s: shapes do not broadcast at aligned dimension %d (%lld against %lld)", fn, i,
                   (long long)da[i], (long long)db[i]);
        n[i] = da[i] == 1 ? db[i] : da[i];
    }
    CH_REQUIRE(shape_prod(da, R) == alen && shape_prod(db, R) == blen,
               "%s: lengths (%lld, %lld) do not match the shapes' (%lld, %lld)", fn, (long long)alen,
               (long long)blen, (long long)shape_prod(da, R), (long long)shape_prod(db, R));
    CH_REQUIRE(shape_prod(n, R) == outlen, "%s: out length %lld != the broadcast shape's %lld", fn,
               (long long)outlen, (long long)shape_prod(n, R));
    bcast_strides(da, R, ea);
    bcast_strides(db, R, eb);
    // inner to outer: drop output dimensions of 1, merge alike neighbours
    int r = 0;
    int64_t cn[kMaxRank], ca[kMaxRank], cb[kMaxRank];
    for (int i = R - 1; i >= 0; --i) {
        if (n[i] == 1) continue;
        if (r > 0 && ea[i] == ca[r - 1] * cn[r - 1] && eb[i] == cb[r - 1] * cn[r - 1]) {
            cn[r - 1] *= n[i];
        } else {
            cn[r] = n[i], ca[r] = ea[i], cb[r] = eb[i];
            ++r;
        }
    }
    if (r == 0) cn[0] = 1, ca[0] = 0, cb[0] = 0, r = 1;
    d->rank = r;
    for (int k = 0; k < r; ++k) {  // back to outer-to-inner order
        d->n[k] = cn[r - 1 - k];
        d->sa[k] = ca[r - 1 - k];
        d->sb[k] = cb[r - 1 - k];
    }
    for (int k = r; k < kMaxRank; ++k) d->n[k] = 1, d->sa[k] = 0, d->sb[k] = 0;
    return CLEAVE_HIP_OK;
}

template <class Op, class T>
int32_t run_bcast(const char* fn, const T* a, int64_t alen, const int32_t* ash, int32_t ar, const T* b, int64_t blen,
                  const int32_t* bsh, int32_t br, T* out, int64_t outlen) {
    constexpr int V = Chunk<T>::kN;
    BDims d;
    const int32_t st = plan_bcast(fn, ash, ar, alen, bsh, br, blen, outlen, &d);
    if (st != CLEAVE_HIP_OK) return st;
    if (outlen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(a && b && out, "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, a, alen * sizeof(T));
    CH_DEVICE(fn, b, blen * sizeof(T));
    CH_DEVICE(fn, out, outlen * sizeof(T));
    const int64_t inner = d.n[d.rank - 1], rows = outlen / inner, chunks = (inner + V - 1) / V;
    const bool vec = inner % V == 0 && aligned16(a) && aligned16(b) && aligned16(out);
    const bool narrow = outlen < (int64_t)1 << 31 && alen < (int64_t)1 << 31 && blen < (int64_t)1 << 31;
    if (vec && chunks >= kRowChunks) {
        const unsigned grid = (unsigned)(rows < 65536 * 8 ? rows : 65536 * 8);
        if (narrow)
            bcast_rows_kernel<Op, T, uint32_t><<<grid, kThreads, 0, ch::stream()>>>(a, b, out, d, (uint32_t)rows,
                                                                                   (uint32_t)chunks);
        else
            bcast_rows_kernel<Op, T, int64_t><<<grid, kThreads, 0, ch::stream()>>>(a, b, out, d, rows, chunks);
        CH_LAUNCHED(fn);
        return CLEAVE_HIP_OK;
    }
    const unsigned grid = blocks_for(rows * chunks);
    if (narrow) {
        if (vec)
            bcast_kernel<Op, T, true, uint32_t><<<grid, kThreads, 0, ch::stream()>>>(a, b, out, d, (uint32_t)rows,
                                                                                   (uint32_t)chunks);
        else
            bcast_kernel<Op, T, false, uint32_t><<<grid, kThreads, 0, ch::stream()>>>(a, b, out, d, (uint32_t)rows,
                                                                                    (uint32_t)chunks);
    } else {
        if (vec)
            bcast_kernel<Op, T, true, int64_t><<<grid, kThreads, 0, ch::stream()>>>(a, b, out, d, rows, chunks);
        else
            bcast_kernel<Op, T, false, int64_t><<<grid, kThreads, 0, ch::stream()>>>(a, b, out, d, rows, chunks);
    }
    CH_LAUNCHED(fn);
    return CLEAVE_HIP_OK;
}

struct RDims {
    int nk, nr;
    int64_t kn[kMaxRank], ks[kMaxRank];  // kept runs, outer to inner, and their strides in g
    int64_t rn[kMaxRank], rs[kMaxRank];  // reduced runs and their strides in g
    int64_t rtotal;                      // elements summed per output element
};

// out = 0 (a fill kernel rather than hipMemsetAsync, so that the call can be
// captured in a graph).
template <class T>
__global__ __launch_bounds__(kThreads) void zero_fill_kernel(T* __restrict__ out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreads)
        out[i] = T(0);
}

// One thread per output element: its reduced elements in row-major order.
template <class T>
__global__ __launch_bounds__(kThreads) void sum_to_shape_kernel(const T* __restrict__ g, T* __restrict__ out, RDims d,
                                                                int64_t nout) {
    for (int64_t o = (int64_t)blockIdx.x * kThreads + threadIdx.x; o < nout; o += (int64_t)gridDim.x * kThreads) {
        int64_t rem = o, base = 0;
#pragma unroll
        for (int k = kMaxRank - 1; k >= 0; --k) {
            if (k < d.nk) {
                const int64_t q = rem % d.kn[k];
                rem /= d.kn[k];
                base += q * d.ks[k];
            }
        }
        int64_t q[kMaxRank] = {};
        int64_t off = 0;
        T acc = 0;
        for (int64_t r = 0; r < d.rtotal; ++r) {
            acc += g[base + off];
#pragma unroll
            for (int k = kMaxRank - 1; k >= 0; --k) {
                if (k < d.nr) {
                    if (++q[k] < d.rn[k]) {
                        off += d.rs[k];
                        break;
                    }
                    off -= (d.rn[k] - 1) * d.rs[k];
                    q[k] = 0;
                }
            }
        }
        out[o] = acc;
    }
}

// One wave per row of g (rows x len, contiguous): lanes stride the row one
// 16-byte chunk at a time (VEC: len a multiple of the chunk and g aligned;
// else one element at a time), each lane adds its chunks in order and then
// the chunk's elements, and the 64 lane sums meet in a fixed xor tree.
template <class T, bool VEC>
__global__ __launch_bounds__(kThreads) void sum_segments_kernel(const T* __restrict__ g, T* __restrict__ out,
                                                                int64_t rows, int64_t len) {
    constexpr int V = Chunk<T>::kN;
    typedef typename Chunk<T>::type vec;
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * (kThreads / 64);
    for (int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); row < rows; row += waves) {
        const T* p = g + row * len;
        T acc = 0;
        if constexpr (VEC) {
            vec v = vec(0);
            for (int64_t c = lane; c < len / V; c += 64) v += ldnt(p + c * V);
#pragma unroll
            for (int t = 0; t < V; ++t) acc += v[t];
        } else {
            for (int64_t i = lane; i < len; i += 64) acc += p[i];
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
        if (lane == 0) out[row] = acc;
    }
}

template <class T>
int32_t run_sum_to_shape(const char* fn, const T* g, int64_t glen, const int32_t* gsh, int32_t gr, T* out,
                         int64_t outlen, const int32_t* osh, int32_t orank) {
    CH_REQUIRE(gr >= 0 && gr <= kMaxRank && orank >= 0 && orank <= gr, "%s: ranks %d (g) and %d (out): need "
               "0 <= out rank <= g rank <= %d", fn, gr, orank, kMaxRank);
    CH_REQUIRE((gr == 0 || gsh) && (orank == 0 || osh), "%s: null shape array", fn);
    CH_REQUIRE(glen >= 0 && outlen >= 0, "%s: negative length (%lld, %lld)", fn, (long long)glen,
               (long long)outlen);
    const int R = gr > 0 ? gr : 1;
    int64_t dg[kMaxRank], dout[kMaxRank], eg[kMaxRank];
    CH_REQUIRE(align_shape(gsh, gr, R, dg) && align_shape(osh, orank, R, dout), "%s: negative dimension", fn);
    for (int i = 0; i < R; ++i)
        CH_REQUIRE(dout[i] == dg[i] || dout[i] == 1, "%s: out dimension %lld does not broadcast to g's %lld "
                   "(aligned dimension %d)", fn, (long long)dout[i], (long long)dg[i], i);
    CH_REQUIRE(shape_prod(dg, R) == glen && shape_prod(dout, R) == outlen,
               "%s: lengths (%lld, %lld) do not match the shapes' (%lld, %lld)", fn, (long long)glen,
               (long long)outlen, (long long)shape_prod(dg, R), (long long)shape_prod(dout, R));
    if (outlen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(out && (g || glen == 0), "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    CH_DEVICE(fn, out, outlen * sizeof(T));
    if (glen == 0) {  // a reduced dimension of 0: sums over nothing
        zero_fill_kernel<T><<<blocks_for(outlen), kThreads, 0, ch::stream()>>>(out, outlen);
        CH_LAUNCHED(fn);
        return CLEAVE_HIP_OK;
    }
    CH_DEVICE(fn, g, glen * sizeof(T));
    // g's row-major strides; runs of kept (dout == dg) and reduced dimensions,
    // dimensions of 1 dropped, alike neighbours merged
    int64_t st = 1;
    for (int i = R - 1; i >= 0; --i) eg[i] = st, st *= dg[i];
    int nrun = 0;
    int64_t runn[kMaxRank], runs[kMaxRank];
    bool runk[kMaxRank];
    for (int i = 0; i < R; ++i) {
        if (dg[i] == 1) continue;
        const bool kept = dout[i] == dg[i];
        if (nrun > 0 && runk[nrun - 1] == kept && runs[nrun - 1] == eg[i] * dg[i]) {
            runn[nrun - 1] *= dg[i];
            runs[nrun - 1] = eg[i];
        } else {
            runn[nrun] = dg[i], runs[nrun] = eg[i], runk[nrun] = kept;
            ++nrun;
        }
    }
    int nk = 0, nr = 0;
    for (int i = 0; i < nrun; ++i) (runk[i] ? nk : nr)++;
    if (nr == 0) {  // nothing stretched: the cotangent itself
        CH_HIP(hipMemcpyAsync(out, g, (size_t)outlen * sizeof(T), hipMemcpyDeviceToDevice, ch::stream()));
        return CLEAVE_HIP_OK;
    }
    if (nk == 0 && nr == 1) {  // everything reduced: the library's Sum
        if constexpr (sizeof(T) == 4) return cleave_hip_reduce_sum_f32((const float*)g, glen, (float*)out);
        else return cleave_hip_reduce_sum_f64((const double*)g, glen, (double*)out);
    }
    if (nrun == 2 && !runk[0] && runk[1] && runn[0] <= INT32_MAX && runn[1] <= INT32_MAX)  // column sums
        return run_sum_rows<T>(fn, g, glen, out, outlen, (int32_t)runn[0], (int32_t)runn[1]);
    if (nrun == 2 && runk[0] && !runk[1] && runn[1] >= 256) {  // sums of contiguous rows
        const unsigned grid = blocks_for(runn[0] * 64);
        if (runn[1] % Chunk<T>::kN == 0 && aligned16(g))
            sum_segments_kernel<T, true><<<grid, kThreads, 0, ch::stream()>>>(g, out, runn[0], runn[1]);
        else
            sum_segments_kernel<T, false><<<grid, kThreads, 0, ch::stream()>>>(g, out, runn[0], runn[1]);
        CH_LAUNCHED(fn);
        return CLEAVE_HIP_OK;
    }
    RDims d{};
    d.rtotal = 1;
    for (int i = 0; i < nrun; ++i) {
        if (runk[i]) d.kn[d.nk] = runn[i], d.ks[d.nk] = runs[i], ++d.nk;
        else d.rn[d.nr] = runn[i], d.rs[d.nr] = runs[i], d.rtotal *= runn[i], ++d.nr;
    }
    sum_to_shape_kernel<T><<<blocks_for(outlen), kThreads, 0, ch::stream()>>>(g, out, d, outlen);
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

#define CH_BCAST(op, Op, T, sfx)                                                                                 \
    int32_t cleave_hip_##op##_bcast_##sfx(const T* a, int64_t alen, const int32_t* ashape, int32_t arank,          \
                                         const T* b, int64_t blen, const int32_t* bshape, int32_t brank, T* out, \
                                         int64_t outlen) {                                                      \
        return run_bcast<Op, T>("cleave_hip_" #op "_bcast_" #sfx, a, alen, ashape, arank, b, blen, bshape, brank, \
                                out, outlen);                                                                   \
    }
CH_BCAST(add, BAdd, float, f32)
CH_BCAST(sub, BSub, float, f32)
CH_BCAST(mul, BMul, float, f32)
CH_BCAST(div, BDiv, float, f32)
CH_BCAST(add, BAdd, double, f64)
CH_BCAST(sub, BSub, double, f64)
CH_BCAST(mul, BMul, double, f64)
CH_BCAST(div, BDiv, double, f64)
#undef CH_BCAST

int32_t cleave_hip_sum_to_shape_f32(const float* g, int64_t glen, const int32_t* gshape, int32_t grank, float* out,
                                    int64_t outlen, const int32_t* oshape, int32_t orank) {
    return run_sum_to_shape<float>("cleave_hip_sum_to_shape_f32", g, glen, gshape, grank, out, outlen, oshape, orank);
}

int32_t cleave_hip_sum_to_shape_f64(const double* g, int64_t glen, const int32_t* gshape, int32_t grank, double* out,
                                    int64_t outlen, const int32_t* oshape, int32_t orank) {
    return run_sum_to_shape<double>("cleave_hip_sum_to_shape_f64", g, glen, gshape, grank, out, outlen, oshape,
                                    orank);
}

}  // extern "C"
