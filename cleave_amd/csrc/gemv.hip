// gemv.hip -- matmul shapes with a dimension of 1: matrix-vector products and
// outer products (linalg.matmul of stdlib/linalg/matrix.cleave:27-61 at
// M = 1, N = 1 or K = 1).
//
// The reference's examples multiply by column vectors (examples/xor_tensor.cleave:
// 44-49: matmul(h, w2) with w2 of n x 1), and the reverse rule of such a
// product (stdlib/linalg/matrix.cleave:24) gives the other two shapes:
// d(h) = g w2^T is an outer product (K = 1) and d(w2) = h^T g a
// matrix-vector product over the batch.  On 32 x 32 matrix-core tiles these
// would waste 31/32 of the work and read the matrix with guarded loads; here
// they are HBM-bound streams over the one matrix operand:
//   row dots      y[i] = sum_k X[i][k] v[k]  (X with k contiguous)
//   weighted sums y[j] = sum_k v[k] X[k][j]  (X with j contiguous)
//   outer         C[i][j] = 0 + a[i] b[j]
// Every operand of such a product is a matrix X and a vector (a 1 x K or
// K x 1 operand is K contiguous values in either layout).  Sums run in a
// fixed order for a given shape (per-lane strided partials, then a fixed
// shuffle tree; or per-row-group partials, then groups in ascending order),
// so results are deterministic; the order differs from the reference's
// k-ascending loop by rounding only.  The outer product is bit-exact: the
// loop adds one product to a zero.
#include "common.hpp"

#include <algorithm>

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }

// 16 bytes of T as floats.  load: a cached load (a vector that every row
// reads again); load_nt: a non-temporal one, for a matrix streamed once and
// too large for the MALL (below).
template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
    static constexpr int N = 4;
    typedef float raw __attribute__((ext_vector_type(4)));
    __device__ static void unpack(raw r, float (&o)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = r[i];
    }
    __device__ static void load(const float* p, float (&o)[4]) { unpack(*reinterpret_cast<const raw*>(p), o); }
    __device__ static void load_nt(const float* p, float (&o)[4]) {
        unpack(__builtin_nontemporal_load(reinterpret_cast<const raw*>(p)), o);
    }
};
template <>
struct Vec16<uint16_t> {
    static constexpr int N = 8;
    typedef uint32_t raw __attribute__((ext_vector_type(4)));
    __device__ static void unpack(raw r, float (&o)[8]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = __uint_as_float(r[i] << 16);
            o[2 * i + 1] = __uint_as_float(r[i] & 0xFFFF0000u);
        }
    }
    __device__ static void load(const uint16_t* p, float (&o)[8]) { unpack(*reinterpret_cast<const raw*>(p), o); }
    __device__ static void load_nt(const uint16_t* p, float (&o)[8]) {
        unpack(__builtin_nontemporal_load(reinterpret_cast<const raw*>(p)), o);
    }
};

// A matrix read once streams with non-temporal loads when it is larger than
// the MI355X's 256 MiB MALL: on data read once, 16-byte loads stream about
// 7.3 TB/s with the hint against 6.2 without it (f32 65536 x 4096 . v 0.80 ->
// 0.88 of HBM).  A smaller one stays cached: across calls it is still in the
// MALL, and the hint then cost 5-38% (bf16 4096^2 . v 4.8 -> 6.6 us, f32
// 16384 x 4096 . v 37.8 -> 39.8).
constexpr int64_t kStreamBytes = 256LL << 20;
inline bool stream_nt(int64_t bytes) { return bytes > kStreamBytes; }

template <typename T, bool NT>
__device__ __forceinline__ void load_x(const T* p, float (&o)[Vec16<T>::N]) {
    if constexpr (NT) Vec16<T>::load_nt(p, o);
    else Vec16<T>::load(p, o);
}

// ---- row dots ---------------------------------------------------------------------
//
// y[r] = sum_k X[r][k] v[(r / rows_per_vec) * K + k] for r < rows.  A row is
// owned by `lpr` lanes (a power of two up to 64, sized to K), so a short row
// does not leave most of a wave idle; lane l of a row takes the 16-byte
// chunks l, l + lpr, ... (VEC) or the elements l, l + lpr, ... (scalar), four
// chunks in flight, and the row's lanes are then added by a shuffle tree.
template <typename T, bool VEC, bool NT>
__global__ __launch_bounds__(kThreads) void row_dots_kernel(const T* __restrict__ X, const T* __restrict__ v,
                                                            float* __restrict__ y, int64_t rows, int K,
                                                            int64_t rows_per_vec, int lpr) {
    constexpr int E = VEC ? Vec16<T>::N : 1;  // elements per load
    const int lane = threadIdx.x & 63;
    const int sub = lane & (lpr - 1);
    const int64_t rows_per_block = (int64_t)(kThreads / lpr);
    for (int64_t r0 = (int64_t)blockIdx.x * rows_per_block; r0 < rows; r0 += (int64_t)gridDim.x * rows_per_block) {
        const int64_t r = r0 + threadIdx.x / lpr;
        float acc = 0.0f;
        if (r < rows) {
            const T* x = X + r * (int64_t)K;
            const T* w = v + (r / rows_per_vec) * (int64_t)K;
            const int64_t step = (int64_t)lpr * E;
            int64_t k = (int64_t)sub * E;
            if constexpr (VEC) {
                for (; k + 3 * step < K; k += 4 * step) {
                    float a[4][E], b[4][E];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        load_x<T, NT>(x + k + u * step, a[u]);
                        Vec16<T>::load(w + k + u * step, b[u]);
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u)
#pragma unroll
                        for (int e = 0; e < E; ++e) acc = acc + a[u][e] * b[u][e];
                }
                for (; k < K; k += step) {
                    float a[E], b[E];
                    load_x<T, NT>(x + k, a);
                    Vec16<T>::load(w + k, b);
#pragma unroll
                    for (int e = 0; e < E; ++e) acc = acc + a[e] * b[e];
                }
            } else {
                for (; k < K; k += step) acc = acc + to_f32(x[k]) * to_f32(w[k]);
            }
        }
        // lanes sub = 0 .. lpr-1 of a row are consecutive; lpr is uniform
        for (int o = lpr >> 1; o > 0; o >>= 1) acc = acc + __shfl_xor(acc, o);
        if (r < rows && sub == 0) y[r] = acc;
    }
}

// Few long rows (a dot product, or fewer rows than the GPU has CUs): each
// row's k range is cut into `slices` pieces of `slice` elements (a multiple
// of the load width), one workgroup each.  A workgroup's lanes take strided
// chunks as above; its sum is the shuffle tree of each wave, then the four
// waves in order, into part[row][slice]; row_dots_fold adds a row's slices
// in order.
template <typename T, bool VEC, bool NT>
__global__ __launch_bounds__(kThreads) void row_dots_split_kernel(const T* __restrict__ X, const T* __restrict__ v,
                                                                  float* __restrict__ part, int K, int64_t rows_per_vec,
                                                                  int slices, int64_t slice) {
    constexpr int E = VEC ? Vec16<T>::N : 1;
    __shared__ float wsum[kThreads / 64];
    const int64_t r = blockIdx.y;
    const int s = blockIdx.x;
    const T* x = X + r * (int64_t)K;
    const T* w = v + (r / rows_per_vec) * (int64_t)K;
    const int64_t k0 = (int64_t)s * slice;
    const int64_t k1 = k0 + slice < K ? k0 + slice : K;
    constexpr int64_t step = (int64_t)kThreads * E;
    float acc = 0.0f;
    int64_t k = k0 + (int64_t)threadIdx.x * E;
    if constexpr (VEC) {
        for (; k + 3 * step < k1; k += 4 * step) {
            float a[4][E], b[4][E];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                load_x<T, NT>(x + k + u * step, a[u]);
                Vec16<T>::load(w + k + u * step, b[u]);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int e = 0; e < E; ++e) acc = acc + a[u][e] * b[u][e];
        }
        for (; k < k1; k += step) {
            float a[E], b[E];
            load_x<T, NT>(x + k, a);
            Vec16<T>::load(w + k, b);
#pragma unroll
            for (int e = 0; e < E; ++e) acc = acc + a[e] * b[e];
        }
    } else {
        for (; k < k1; k += step) acc = acc + to_f32(x[k]) * to_f32(w[k]);
    }
    for (int o = 32; o > 0; o >>= 1) acc = acc + __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = wsum[0];
#pragma unroll
        for (int i = 1; i < kThreads / 64; ++i) t = t + wsum[i];
        part[r * slices + s] = t;
    }
}

__global__ __launch_bounds__(kThreads) void row_dots_fold(const float* __restrict__ part, float* __restrict__ y,
                                                          int64_t rows, int slices) {
    const int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (r >= rows) return;
    const float* p = part + r * slices;
    float acc = p[0];
    for (int s = 1; s < slices; ++s) acc = acc + p[s];
    y[r] = acc;
}

// ---- weighted column sums -----------------------------------------------------------
//
// y[b][j] = sum_k v[b][k] X[b][k][j] (X of K x cols per product).  Stage 1: a
// thread owns one 16-byte column chunk (VEC) or one column and walks a group
// of rows in ascending order, into part[b][group][j]; stage 2 adds the
// groups in ascending order.  The column sums of broadcast.hip use the same
// tiling.
template <typename T, bool VEC, bool NT>
__global__ __launch_bounds__(kThreads) void wsum_stage1(const T* __restrict__ X, const T* __restrict__ v,
                                                        float* __restrict__ part, int K, int64_t cols, int64_t nseg,
                                                        int64_t groups, int64_t rpg) {
    constexpr int E = VEC ? Vec16<T>::N : 1;
    const int64_t b = blockIdx.y;
    const int64_t seg = blockIdx.x % nseg, group = blockIdx.x / nseg;
    const int64_t c = (seg * kThreads + threadIdx.x) * E;
    if (c >= cols) return;
    X += b * (int64_t)K * cols;
    v += b * (int64_t)K;
    const int64_t r0 = group * rpg;
    const int64_t r1 = r0 + rpg < K ? r0 + rpg : K;
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = 0.0f;
    const bool whole = c + E <= cols;
    int64_t r = r0;
    if constexpr (VEC) {
        if (whole) {
            // four rows' loads in flight, added in row order
            for (; r + 4 <= r1; r += 4) {
                float a[4][E], w[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    w[u] = to_f32(v[r + u]);
                    load_x<T, NT>(X + (r + u) * cols + c, a[u]);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[e] = acc[e] + w[u] * a[u][e];
            }
            for (; r < r1; ++r) {
                float a[E];
                const float w = to_f32(v[r]);
                load_x<T, NT>(X + r * cols + c, a);
#pragma unroll
                for (int e = 0; e < E; ++e) acc[e] = acc[e] + w * a[e];
            }
        }
    }
    for (; r < r1; ++r) {
        const float w = to_f32(v[r]);
        const T* x = X + r * cols + c;
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (c + e < cols) acc[e] = acc[e] + w * to_f32(x[e]);
    }
    float* p = part + (b * groups + group) * cols + c;
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (c + e < cols) p[e] = acc[e];
}

constexpr int kWsumSplit = 8, kWsumCols = kThreads / kWsumSplit;
__global__ __launch_bounds__(kThreads) void wsum_stage2(const float* __restrict__ part, float* __restrict__ y,
                                                        int64_t cols, int64_t groups) {
    // kWsumSplit threads per column, each adding a contiguous eighth of the
    // groups (eight loads in flight), then the eighths in order.  With one
    // thread per column, a column's 256 groups took 32 dependent rounds of
    // loads on 16 workgroups (12.6 us of a 171 us f32 v^T X at 65536 x 4096);
    // split, the product measured 164 us (bf16 103 -> 89, f32 100000 x 1000
    // 110 -> 73).
    __shared__ float red[kWsumSplit][kWsumCols];
    const int64_t b = blockIdx.y;
    const int jj = threadIdx.x % kWsumCols, sp = threadIdx.x / kWsumCols;
    const int64_t j = (int64_t)blockIdx.x * kWsumCols + jj;
    const int64_t q0 = groups * sp / kWsumSplit, q1 = groups * (sp + 1) / kWsumSplit;
    const float* p = part + b * groups * cols + j;
    float acc = 0.0f;
    if (j < cols && q0 < q1) {
        acc = p[q0 * cols];
        int64_t g = q0 + 1;
        for (; g + 8 <= q1; g += 8) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = p[(g + u) * cols];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = acc + t[u];
        }
        for (; g < q1; ++g) acc = acc + p[g * cols];
    }
    red[sp][jj] = acc;
    __syncthreads();
    if (sp == 0 && j < cols) {
        // the non-empty eighths in order (one is empty only when groups < 8;
        // the last never is)
        int t = 0;
        while (groups * (t + 1) / kWsumSplit == groups * t / kWsumSplit) ++t;
        float r = red[t][jj];
        for (++t; t < kWsumSplit; ++t)
            if (groups * (t + 1) / kWsumSplit > groups * t / kWsumSplit) r = r + red[t][jj];
        y[b * cols + j] = r;
    }
}

// ---- outer product ------------------------------------------------------------------
//
// C[b][i][j] = 0 + a[b][i] b[b][j]: one workgroup per row (grid-strided), four
// columns per thread.  0 + p is p except that a -0 product becomes +0, as in
// the reference's C = 0; C += a*b.

// Four consecutive values as floats: one 16-byte (f32) or 8-byte (bf16) load;
// p must be aligned to that size.
__device__ __forceinline__ void load4(const float* p, float (&o)[4]) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 r = *reinterpret_cast<const f4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = r[i];
}
__device__ __forceinline__ void load4(const uint16_t* p, float (&o)[4]) {
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    const u2 r = *reinterpret_cast<const u2*>(p);
    o[0] = __uint_as_float(r[0] << 16);
    o[1] = __uint_as_float(r[0] & 0xFFFF0000u);
    o[2] = __uint_as_float(r[1] << 16);
    o[3] = __uint_as_float(r[1] & 0xFFFF0000u);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void outer_kernel(const T* __restrict__ a, const T* __restrict__ bv,
                                                         float* __restrict__ C, int M, int N, int64_t rows,
                                                         bool vec_out) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const int64_t b = row / M;
        const float ai = to_f32(a[row]);  // a of product b holds M values: a[b*M + i]
        const T* bb = bv + b * (int64_t)N;
        float* c = C + row * (int64_t)N;
        for (int j = threadIdx.x * 4; j < N; j += kThreads * 4) {
            f4 o;
            if (vec_out && j + 4 <= N) {
                float bj[4];
                load4(bb + j, bj);
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = 0.0f + ai * bj[e];
                __builtin_nontemporal_store(o, reinterpret_cast<f4*>(c + j));
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = j + e < N ? 0.0f + ai * to_f32(bb[j + e]) : 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (j + e < N) c[j + e] = o[e];
            }
        }
    }
}

// ---- skinny products: one output dimension of at most 32 --------------------------
//
// Y[r][s] = sum_k X(r, k) V(s, k) for r < R, s < S <= 32, with X(r, k) =
// X[r*xs_r + k*xs_k] and V(s, k) = V[s*vs_s + k*vs_k]: X is the operand along
// the long output dimension, stored k-contiguous (xs_k == 1) or r-contiguous,
// and V the small one, in either layout.  On 128 x 128 tiles these products
// wasted most of every MFMA; with VALU fmas (each X value meeting its S values
// of V) they were bound by the fmas and the LDS reads of V from about 10
// vectors on (65536 x 32 x 4096 f32: 706 us, 0.19 of HBM; here 248 us).
//
// A wave owns RB blocks of MR rows and all MR columns over one group of k: the
// MFMA's A operand is X, its B operand V, which each lane loads straight from
// memory (V is small and stays in L2).  Columns past S and rows past R read
// clamped addresses; the MFMA keeps rows and columns apart, so what they
// compute is never stored.  k past K reads as zero in both operands.  One
// group per wave writes Y; several write their blocks to part[b][group][rb] in
// accumulator order and skinny_mfma_fold adds the groups in ascending order.
// The sums run in an order fixed by the shape.
//
// Instruction per type and MR (lane l; q = the lane's k quarter or half):
//   f32, 32: v_mfma_f32_32x32x2f32, a block of 8 k in four steps, half-wave
//            q = l/32 taking k = 4q + e at step e; accumulator v of lane l is
//            column l%32, row 8(v/4) + 4q + v%4;
//   f32, 16: v_mfma_f32_16x16x4f32, a block of 16 k in four steps, quarter
//            q = l/16 taking k = 4q + e; accumulator v: column l%16, row 4q + v;
//   bf16, 32: v_mfma_f32_32x32x16_bf16, one step per block of 16 k, half-wave
//            q taking k = 8q .. 8q+7; accumulators as f32, 32.
// At 32 columns a 32 x 32 x 2 step takes 64 cycles for 256 bytes of f32 X,
// about the HBM's share of a SIMD; the 16 x 16 x 4 form moves twice that.
typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef short s8v __attribute__((ext_vector_type(8)));
typedef short s4v __attribute__((ext_vector_type(4)));
typedef __bf16 bf8v __attribute__((ext_vector_type(8)));

template <typename T, int MR>
struct SkMfma;
// LINES: 128-byte lines of each row per staged group (XS), measured per form
template <>
struct SkMfma<float, 32> {
    static constexpr int KBLK = 8, ACC = 16, LINES = 2;
    typedef f4v frag;
    typedef f16v acc_t;
    __device__ static int kofs(int lane) { return 4 * (lane >> 5); }
    __device__ static int row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }
    __device__ static void mma(const frag& a, const frag& b, acc_t& c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], b[e], c, 0, 0, 0);
    }
};
template <>
struct SkMfma<float, 16> {
    static constexpr int KBLK = 16, ACC = 4, LINES = 1;
    typedef f4v frag;
    typedef f4v acc_t;
    __device__ static int kofs(int lane) { return 4 * (lane >> 4); }
    __device__ static int row(int v, int lane) { return 4 * (lane >> 4) + v; }
    __device__ static void mma(const frag& a, const frag& b, acc_t& c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], c, 0, 0, 0);
    }
};
template <>
struct SkMfma<uint16_t, 32> {
    static constexpr int KBLK = 16, ACC = 16, LINES = 2;
    typedef s8v frag;
    typedef f16v acc_t;
    __device__ static int kofs(int lane) { return 8 * (lane >> 5); }
    __device__ static int row(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }
    __device__ static void mma(const frag& a, const frag& b, acc_t& c) {
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf8v, a), __builtin_bit_cast(bf8v, b), c, 0, 0,
                                                    0);
    }
};

// E values p[0], p[st], ... as one fragment: a 16-byte load (VEC: st == 1 and p
// 16-byte aligned) or E loads.
template <bool VEC>
__device__ __forceinline__ f4v sk_run(const float* p, int64_t st) {
    if constexpr (VEC) return *reinterpret_cast<const f4v*>(p);
    f4v v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = p[e * st];
    return v;
}
template <bool VEC>
__device__ __forceinline__ s8v sk_run(const uint16_t* p, int64_t st) {
    if constexpr (VEC) return *reinterpret_cast<const s8v*>(p);
    s8v v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (short)p[e * st];
    return v;
}
// The same for the last, partial block: values at k + e >= K are zero.
__device__ __forceinline__ f4v sk_run_tail(const float* p, int64_t st, int64_t k, int K) {
    f4v v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = k + e < K ? p[e * st] : 0.0f;
    return v;
}
__device__ __forceinline__ s8v sk_run_tail(const uint16_t* p, int64_t st, int64_t k, int K) {
    s8v v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = k + e < K ? (short)p[e * st] : (short)0;
    return v;
}

constexpr int kSkMfmaUnroll = 4;  // blocks of k whose loads are issued together (unstaged X)

// X staged through the wave's own 4 KiB (or 8) of LDS, so that every load
// instruction reads whole 16-byte pieces of few lines:
//   XM 1, X k-contiguous with 16-byte aligned rows: F::LINES x 128 bytes of
//     each of the wave's 32 rows at a time, 8 rows of 8 lanes per instruction.
//     Read straight into the MFMA layout, an instruction took 16-32 rows at
//     32-64 bytes each and the kernel ran at 0.40-0.54 of HBM.  Row r's
//     16-byte chunk c sits in slot c ^ ((r >> 1) & 7): sixteen lanes reading
//     one chunk of 16 consecutive rows, or writing two rows, then cover all
//     64 banks once.
//   XM 2, X r-contiguous with 16-byte aligned k-rows: the wave's 32 values of
//     32 (f32) or 64 (bf16) k-rows at a time, 8 (16) k-rows per instruction.
//     Read as single values, bf16 X took eight 2-byte loads per lane and k
//     block and ran at 0.45-0.49 of HBM.  f32: k-row kr sits at row
//     kr ^ ((kr >> 2) & 1), its chunk c in slot c ^ 4*((kr >> 3) & 1), so the
//     quarter- or half-waves reading k-rows 4 apart use different banks; the
//     fragments are four ds_read_b32.  bf16: [k-row][32 values], read with
//     ds_read_b64_tr_b16 (in a 16-lane group, source lane 4j + q points at
//     k-row kb + j, values c0 + 4q .. c0 + 4q + 3, and result lane i receives
//     value c0 + i of k-rows kb .. kb + 3), two per fragment.
// X is read once (each wave owns its rows over every column): NT (X larger
// than the MALL, stream_nt) gives its loads the non-temporal hint wherever a
// wave reads whole 128-byte lines.  A template flag, since the compiler
// merges a run-time choice between the two loads into one plain load.
// Only the wave touches its region, and a wave's LDS instructions execute in
// order, so no barrier is needed; the asm statements keep the compiler from
// moving the reads above the writes (or the next writes above the reads).
template <typename T, int MR, int RB, int XM, bool VV, bool NT>
__global__ __launch_bounds__(kThreads) void skinny_mfma_kernel(
    const T* __restrict__ X, const T* __restrict__ V, float* __restrict__ y, float* __restrict__ part, int64_t R,
    int S, int K, int64_t xs_r, int64_t xs_k, int64_t vs_s, int64_t vs_k, int64_t ys_i, int64_t ys_s,
    int64_t x_batch, int64_t v_batch, int64_t y_batch, int64_t nrb, int groups, int bpg) {
    using F = SkMfma<T, MR>;
    using frag = typename F::frag;
    static_assert(MR * RB == 32, "a wave owns 32 rows");
    constexpr int U = kSkMfmaUnroll;
    constexpr bool XS = XM == 1;
    constexpr int STAGE = XM == 1 ? 256 * F::LINES : XM == 2 ? 256 : 1;  // 16-byte slots per wave
    __shared__ f4v stage[XM ? kThreads / 64 : 1][STAGE];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t task = (int64_t)blockIdx.x * (kThreads / 64) + wave;
    if (task >= nrb * groups) return;  // whole waves, and the kernel has no barrier
    const int64_t rb = task % nrb;
    const int g = (int)(task / nrb);
    const int64_t b = blockIdx.y;
    X += b * x_batch;
    V += b * v_batch;
    const int kq = F::kofs(lane);
    const int64_t row0 = rb * 32;
    const T* xr[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        const int64_t r = row0 + i * MR + (lane % MR);
        xr[i] = X + (r < R ? r : R - 1) * xs_r;
    }
    const int sl = lane % MR;
    const T* vr = V + (int64_t)(sl < S ? sl : S - 1) * vs_s;
    typename F::acc_t acc[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) acc[i] = typename F::acc_t{};

    const int nblk = (K + F::KBLK - 1) / F::KBLK, nfull = K / F::KBLK;
    int blk = g * bpg;
    const int b1 = blk + bpg < nblk ? blk + bpg : nblk;
    const int bf = b1 < nfull ? b1 : nfull;
    if constexpr (XS) {
        constexpr int UBL = 128 / (F::KBLK * (int)sizeof(T));  // blocks per 128 bytes of a row
        constexpr int UB = UBL * F::LINES;                       // blocks per staged group
        constexpr int CPB = F::KBLK * (int)sizeof(T) / 16;      // 16-byte chunks of a row per block
        // copy: instruction (l, j) moves line l of rows 8j + lane/8, chunk lane%8
        const char* src[4];
        int dsl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = 8 * j + (lane >> 3);
            const int64_t rr = row0 + r < R ? row0 + r : R - 1;
            src[j] = reinterpret_cast<const char*>(X + rr * xs_r) + (lane & 7) * 16;
            dsl[j] = r * 8 + ((lane & 7) ^ ((r >> 1) & 7));
        }
        // reads: row block i, lane row i*MR + lane%MR, chunk (u % UBL)*CPB + lane/MR of line u / UBL
        int rdx[RB];
        const int cq = lane / MR;
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const int r = i * MR + (lane % MR);
            rdx[i] = r * 8;
        }
        f4v* st = stage[wave];
        const int ng = (bf - blk) / UB;
        f4v data[F::LINES][4];
        frag vc[UB], vn[UB];
        auto load_x = [&](int b0) {
            const int64_t kb = (int64_t)b0 * F::KBLK * (int64_t)sizeof(T);
#pragma unroll
            for (int l = 0; l < F::LINES; ++l)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f4v* q = reinterpret_cast<const f4v*>(src[j] + kb + 128 * l);
                    if constexpr (NT) data[l][j] = __builtin_nontemporal_load(q);
                    else data[l][j] = *q;
                }
        };
        auto load_v = [&](int b0, frag(&vv)[UB]) {
#pragma unroll
            for (int u = 0; u < UB; ++u) {
                const int64_t k = (int64_t)(b0 + u) * F::KBLK + kq;
                vv[u] = sk_run<VV>(vr + k * vs_k, vs_k);
            }
        };
        if (ng > 0) {
            load_x(blk);
            load_v(blk, vc);
        }
        for (int gi = 0; gi < ng; ++gi, blk += UB) {
#pragma unroll
            for (int l = 0; l < F::LINES; ++l)
#pragma unroll
                for (int j = 0; j < 4; ++j) st[l * 256 + dsl[j]] = data[l][j];
            asm volatile("" ::: "memory");
            if (gi + 1 < ng) {  // the next group's X and V, in flight during this group's math
                load_x(blk + UB);
                load_v(blk + UB, vn);
            }
#pragma unroll
            for (int u = 0; u < UB; ++u)
#pragma unroll
                for (int i = 0; i < RB; ++i) {
                    const int r = i * MR + (lane % MR);
                    const int c = (u % UBL) * CPB + cq;
                    const f4v t = st[(u / UBL) * 256 + rdx[i] + (c ^ ((r >> 1) & 7))];
                    F::mma(__builtin_bit_cast(frag, t), vc[u], acc[i]);
                }
            asm volatile("" ::: "memory");
#pragma unroll
            for (int u = 0; u < UB; ++u) vc[u] = vn[u];
        }
    } else if constexpr (XM == 2) {
        constexpr int ESZ = (int)sizeof(T), EPC = 16 / ESZ;  // values per 16-byte chunk
        constexpr int LPK = 32 / EPC;                         // lanes (chunks) per k-row of the wave's 32 values
        constexpr int KPI = 64 / LPK;                         // k-rows per load instruction
        constexpr int GK = 4 * KPI;                           // k-rows per staged group (4 loads per lane)
        constexpr int UB = GK / F::KBLK;                      // blocks per staged group
        // copy: instruction j moves k-rows KPI*j + lane/LPK, chunk lane%LPK of
        // the wave's values (a chunk past R reads the last one, never stored)
        const int cl = lane % LPK;
        const int64_t cstart = row0 + (int64_t)cl * EPC <= R - EPC ? row0 + (int64_t)cl * EPC : R - EPC;
        const T* src0 = X + cstart;
        int krj[4], dsl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int kr = KPI * j + lane / LPK;
            krj[j] = kr;
            if constexpr (ESZ == 4) dsl[j] = (kr ^ ((kr >> 2) & 1)) * 8 + (cl ^ (((kr >> 3) & 1) << 2));
            else dsl[j] = kr * 4 + cl;
        }
        f4v* st = stage[wave];
        const int ng = (bf - blk) / UB;
        f4v data[4];
        frag vc[UB], vn[UB];
        auto load_x = [&](int b0) {
            const int64_t k0 = (int64_t)b0 * F::KBLK;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f4v* q = reinterpret_cast<const f4v*>(src0 + (k0 + krj[j]) * xs_k);
                // f32: the wave's 32 values are a whole 128-byte line, read once; bf16:
                // half a line, whose other half the next wave reads (a cached load)
                if constexpr (NT && ESZ == 4) data[j] = __builtin_nontemporal_load(q);
                else data[j] = *q;
            }
        };
        auto load_v = [&](int b0, frag(&vv)[UB]) {
#pragma unroll
            for (int u = 0; u < UB; ++u) {
                const int64_t k = (int64_t)(b0 + u) * F::KBLK + kq;
                vv[u] = sk_run<VV>(vr + k * vs_k, vs_k);
            }
        };
        if (ng > 0) {
            load_x(blk);
            load_v(blk, vc);
        }
        for (int gi = 0; gi < ng; ++gi, blk += UB) {
#pragma unroll
            for (int j = 0; j < 4; ++j) st[dsl[j]] = data[j];
            asm volatile("" ::: "memory");
            if (gi + 1 < ng) {  // the next group's X and V, in flight during this group's math
                load_x(blk + UB);
                load_v(blk + UB, vn);
            }
#pragma unroll
            for (int u = 0; u < UB; ++u)
#pragma unroll
                for (int i = 0; i < RB; ++i) {
                    frag a;
                    if constexpr (ESZ == 4) {
                        // value r of k-rows u*KBLK + kq + e
                        const float* sf = reinterpret_cast<const float*>(st);
                        const int r = i * MR + (lane % MR);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int kr = u * F::KBLK + kq + e;
                            const int c = (r >> 2) ^ (((kr >> 3) & 1) << 2);
                            a[e] = sf[((kr ^ ((kr >> 2) & 1)) * 8 + c) * 4 + (r & 3)];
                        }
                    } else {
                        // 16-lane group g: values c0 = 16 (g & 1) .., k-rows
                        // u*16 + 8 (g >> 1) .. + 7 (two reads of four)
                        const int gq = lane >> 4, li = lane & 15;
                        const int kr = u * 16 + 8 * (gq >> 1) + (li >> 2);
                        const int c0 = 16 * (gq & 1) + 4 * (li & 3);
                        typedef __attribute__((address_space(3))) s4v lds_s4v;
                        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)st;
                        const uint32_t ad = base + (uint32_t)(kr * 64 + c0 * 2);
                        const s4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v*)(uintptr_t)ad);
                        const s4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4v*)(uintptr_t)(ad + 4 * 64));
                        a = __builtin_bit_cast(frag, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                    }
                    F::mma(a, vc[u], acc[i]);
                }
            asm volatile("" ::: "memory");
#pragma unroll
            for (int u = 0; u < UB; ++u) vc[u] = vn[u];
        }
    } else {
        for (; blk + U <= bf; blk += U) {
            frag a[U][RB], v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t k = (int64_t)(blk + u) * F::KBLK + kq;
#pragma unroll
                for (int i = 0; i < RB; ++i) a[u][i] = sk_run<false>(xr[i] + k * xs_k, xs_k);
                v[u] = sk_run<VV>(vr + k * vs_k, vs_k);
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int i = 0; i < RB; ++i) F::mma(a[u][i], v[u], acc[i]);
        }
    }
    for (; blk < bf; ++blk) {
        const int64_t k = (int64_t)blk * F::KBLK + kq;
        frag a[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) a[i] = sk_run<XS>(xr[i] + k * xs_k, xs_k);
        const frag v = sk_run<VV>(vr + k * vs_k, vs_k);
#pragma unroll
        for (int i = 0; i < RB; ++i) F::mma(a[i], v, acc[i]);
    }
    if (blk < b1) {  // the partial last block
        const int64_t k = (int64_t)blk * F::KBLK + kq;
        frag a[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) a[i] = sk_run_tail(xr[i] + k * xs_k, xs_k, k, K);
        const frag v = sk_run_tail(vr + k * vs_k, vs_k, k, K);
#pragma unroll
        for (int i = 0; i < RB; ++i) F::mma(a[i], v, acc[i]);
    }

    if (groups == 1) {
        y += b * y_batch;
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int v = 0; v < F::ACC; ++v) {
                const int64_t r = row0 + i * MR + F::row(v, lane);
                if (r < R && sl < S) y[r * ys_i + sl * ys_s] = acc[i][v];
            }
    } else {
        float* p = part + ((b * groups + g) * nrb + rb) * (RB * F::ACC * 64) + lane;
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int v = 0; v < F::ACC; ++v) p[(i * F::ACC + v) * 64] = acc[i][v];
    }
}

// Y from the groups' partial blocks, added in ascending group order (eight
// loads in flight); one thread per accumulator element of a batch entry.
template <typename T, int MR, int RB>
__global__ __launch_bounds__(kThreads) void skinny_mfma_fold(const float* __restrict__ part, float* __restrict__ y,
                                                             int64_t R, int S, int64_t ys_i, int64_t ys_s,
                                                             int64_t y_batch, int64_t nrb, int groups) {
    using F = SkMfma<T, MR>;
    constexpr int PER_RB = RB * F::ACC * 64;
    const int64_t per = nrb * PER_RB;  // floats per batch entry and group
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (t >= per) return;
    const int64_t b = blockIdx.y;
    const float* p = part + b * groups * per + t;
    float acc = p[0];
    int g = 1;
    for (; g + 8 <= groups; g += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[(int64_t)(g + u) * per];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = acc + v[u];
    }
    for (; g < groups; ++g) acc = acc + p[(int64_t)g * per];
    const int64_t rb = t / PER_RB;
    const int rem = (int)(t - rb * PER_RB);
    const int i = rem / (F::ACC * 64), v = (rem / 64) % F::ACC, lane = rem % 64;
    const int64_t r = (rb * RB + i) * MR + F::row(v, lane);
    const int s = lane % MR;
    if (r < R && s < S) y[b * y_batch + r * ys_i + s * ys_s] = acc;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

unsigned capped_grid(int64_t blocks) {
    const int64_t cap = (int64_t)(ch::num_cus() > 0 ? ch::num_cus() : 1) * 64;
    if (blocks > cap) blocks = cap;
    return (unsigned)(blocks < 1 ? 1 : blocks);
}

template <typename T>
int32_t row_dots(const T* X, const T* v, float* y, int64_t rows, int K, int64_t rows_per_vec) {
    // vector loads when every row and vector start is 16-byte aligned
    const bool vec = (int64_t)K * (int64_t)sizeof(T) % 16 == 0 && aligned16(X) && aligned16(v);
    const bool nt = stream_nt(rows * (int64_t)K * (int64_t)sizeof(T));
    const int E = vec ? Vec16<T>::N : 1;
    const int chunks = K / E;
    int lpr = 1;
    while (lpr < 64 && lpr < chunks) lpr <<= 1;
    const int64_t blocks = (rows + kThreads / lpr - 1) / (kThreads / lpr);
    const int cus = ch::num_cus() > 0 ? ch::num_cus() : 1;
    // Fewer workgroups than CUs: cut the rows' k ranges into slices of at
    // least 4 loads per thread, up to about four workgroups per CU.
    const int64_t min_slice = (int64_t)kThreads * E * 4;
    int64_t slices = std::min<int64_t>(((int64_t)4 * cus + rows - 1) / rows, K / min_slice);
    if (blocks < cus && slices > 1 && rows <= 65535) {
        int64_t slice = (K + slices - 1) / slices;
        slice = (slice + E - 1) / E * E;  // slices start on a load boundary
        slices = (K + slice - 1) / slice;
        float* part = (float*)ch::scratch(8, sizeof(float) * (size_t)(rows * slices));
        if (!part) return CLEAVE_HIP_ERR_OOM;
        const dim3 g((unsigned)slices, (unsigned)rows);
        if (vec && nt)
            row_dots_split_kernel<T, true, true><<<g, kThreads, 0, ch::stream()>>>(X, v, part, K, rows_per_vec,
                                                                               (int)slices, slice);
        else if (vec)
            row_dots_split_kernel<T, true, false><<<g, kThreads, 0, ch::stream()>>>(X, v, part, K, rows_per_vec,
                                                                                (int)slices, slice);
        else
            row_dots_split_kernel<T, false, false><<<g, kThreads, 0, ch::stream()>>>(X, v, part, K, rows_per_vec,
                                                                                 (int)slices, slice);
        int32_t st = ch::check_hip(hipGetLastError(), "row_dots_split_kernel");
        if (st != CLEAVE_HIP_OK) return st;
        row_dots_fold<<<(unsigned)((rows + kThreads - 1) / kThreads), kThreads, 0, ch::stream()>>>(part, y, rows,
                                                                                                   (int)slices);
        return ch::check_hip(hipGetLastError(), "row_dots_fold");
    }
    if (vec && nt)
        row_dots_kernel<T, true, true><<<capped_grid(blocks), kThreads, 0, ch::stream()>>>(X, v, y, rows, K,
                                                                                        rows_per_vec, lpr);
    else if (vec)
        row_dots_kernel<T, true, false><<<capped_grid(blocks), kThreads, 0, ch::stream()>>>(X, v, y, rows, K,
                                                                                         rows_per_vec, lpr);
    else
        row_dots_kernel<T, false, false><<<capped_grid(blocks), kThreads, 0, ch::stream()>>>(X, v, y, rows, K,
                                                                                          rows_per_vec, lpr);
    return ch::check_hip(hipGetLastError(), "row_dots_kernel");
}

template <typename T>
int32_t weighted_sums(const T* X, const T* v, float* y, int K, int64_t cols, int batch) {
    const bool vec = cols * (int64_t)sizeof(T) % 16 == 0 && aligned16(X);
    const int E = vec ? Vec16<T>::N : 1;
    const int64_t nseg = ((cols + E - 1) / E + kThreads - 1) / kThreads;
    // about four blocks per CU over the whole batch, as the column sums
    int64_t groups = 4LL * ch::num_cus() / (nseg * batch);
    if (groups < 1) groups = 1;
    if (groups > K) groups = K;
    const int64_t rpg = (K + groups - 1) / groups;
    groups = (K + rpg - 1) / rpg;
    float* part = (float*)ch::scratch(8, sizeof(float) * (size_t)(batch * groups * cols));
    if (!part) return CLEAVE_HIP_ERR_OOM;
    const dim3 g1((unsigned)(nseg * groups), (unsigned)batch);
    if (vec && stream_nt((int64_t)batch * K * cols * (int64_t)sizeof(T)))
        wsum_stage1<T, true, true><<<g1, kThreads, 0, ch::stream()>>>(X, v, part, K, cols, nseg, groups, rpg);
    else if (vec)
        wsum_stage1<T, true, false><<<g1, kThreads, 0, ch::stream()>>>(X, v, part, K, cols, nseg, groups, rpg);
    else
        wsum_stage1<T, false, false><<<g1, kThreads, 0, ch::stream()>>>(X, v, part, K, cols, nseg, groups, rpg);
    int32_t st = ch::check_hip(hipGetLastError(), "wsum_stage1");
    if (st != CLEAVE_HIP_OK) return st;
    const dim3 g2((unsigned)((cols + kWsumCols - 1) / kWsumCols), (unsigned)batch);
    wsum_stage2<<<g2, kThreads, 0, ch::stream()>>>(part, y, cols, groups);
    return ch::check_hip(hipGetLastError(), "wsum_stage2");
}

template <typename T>
int32_t outer(const T* a, const T* b, float* c, int M, int N, int batch) {
    const int64_t rows = (int64_t)batch * M;
    // whole 16-byte C chunks, and b chunks aligned to their load
    const bool vec = N % 4 == 0 && aligned16(c) && ((uintptr_t)b % (4 * sizeof(T))) == 0;
    outer_kernel<T><<<capped_grid(rows), kThreads, 0, ch::stream()>>>(a, b, c, M, N, rows, vec);
    return ch::check_hip(hipGetLastError(), "outer_kernel");
}

template <typename T, int MR, int RB, int XM, bool VV>
int32_t skinny_mfma_launch(const T* X, const T* V, float* y, float* part, int64_t R, int S, int K, int64_t xs_r,
                           int64_t xs_k, int64_t vs_s, int64_t vs_k, int64_t ys_i, int64_t ys_s, int64_t x_batch,
                           int64_t v_batch, int64_t y_batch, int batch, int64_t nrb, int groups, int bpg) {
    const int64_t waves = nrb * groups;
    const dim3 g((unsigned)((waves + kThreads / 64 - 1) / (kThreads / 64)), (unsigned)batch);
    // the unstaged form (XM 0) and bf16 with r contiguous never take the hint
    constexpr bool kMayNt = XM == 1 || (XM == 2 && sizeof(T) == 4);
    if (kMayNt && stream_nt((int64_t)batch * R * K * (int64_t)sizeof(T)))
        skinny_mfma_kernel<T, MR, RB, XM, VV, kMayNt><<<g, kThreads, 0, ch::stream()>>>(
            X, V, y, part, R, S, K, xs_r, xs_k, vs_s, vs_k, ys_i, ys_s, x_batch, v_batch, y_batch, nrb, groups, bpg);
    else
        skinny_mfma_kernel<T, MR, RB, XM, VV, false><<<g, kThreads, 0, ch::stream()>>>(
            X, V, y, part, R, S, K, xs_r, xs_k, vs_s, vs_k, ys_i, ys_s, x_batch, v_batch, y_batch, nrb, groups, bpg);
    int32_t st = ch::check_hip(hipGetLastError(), "skinny_mfma_kernel");
    if (st != CLEAVE_HIP_OK || groups == 1) return st;
    const int64_t per = nrb * RB * SkMfma<T, MR>::ACC * 64;
    const dim3 g2((unsigned)((per + kThreads - 1) / kThreads), (unsigned)batch);
    skinny_mfma_fold<T, MR, RB><<<g2, kThreads, 0, ch::stream()>>>(part, y, R, S, ys_i, ys_s, y_batch, nrb, groups);
    return ch::check_hip(hipGetLastError(), "skinny_mfma_fold");
}

// Y (R x S, element (r, s) at r*ys_i + s*ys_s) = X V^T on the matrix cores, S <= 32.
template <typename T, int MR, int RB>
int32_t skinny_mfma_mr(const T* X, const T* V, float* y, int64_t R, int S, int K, int64_t xs_r, int64_t xs_k,
                       int64_t vs_s, int64_t vs_k, int64_t ys_i, int64_t ys_s, int64_t x_batch, int64_t v_batch,
                       int64_t y_batch, int batch) {
    using F = SkMfma<T, MR>;
    constexpr int64_t esz = sizeof(T);
    // X staged through LDS with 16-byte loads (XM 1 along k, 2 along r):
    // unit stride along one, and every row (k-row) and batch entry aligned.
    // With r contiguous the k-row pitch is R, so no 16-byte piece straddles R.
    const bool xv = xs_k == 1 && aligned16(X) && (xs_r * esz) % 16 == 0 && (x_batch * esz) % 16 == 0;
    const bool xt = !xv && xs_r == 1 && xs_k == R && aligned16(X) && (xs_k * esz) % 16 == 0 &&
                    (x_batch * esz) % 16 == 0;
    const bool vv = vs_k == 1 && aligned16(V) && (vs_s * esz) % 16 == 0 && (v_batch * esz) % 16 == 0;
    const int64_t nrb = (R + MR * RB - 1) / (MR * RB);
    const int nblk = (K + F::KBLK - 1) / F::KBLK;
    // Groups of k: enough waves for 8 per CU over the batch (16 with X
    // unstaged), each group at least 8 blocks deep, and the partial blocks at
    // most an eighth of X's bytes.
    const int cus = ch::num_cus() > 0 ? ch::num_cus() : 1;
    const int64_t want = (xv || xt ? 8LL : 16LL) * cus;
    int64_t groups = (want + nrb * batch - 1) / (nrb * batch);
    groups = std::min<int64_t>(groups, std::max(1, nblk / 8));
    const int64_t part_per_group = nrb * (int64_t)(MR * RB * MR) * 4;  // bytes per batch entry
    groups = std::min<int64_t>(groups, std::max<int64_t>(1, R * K * esz / 8 / part_per_group));
    if (groups < 1) groups = 1;
    int bpg = (int)((nblk + groups - 1) / groups);
    if (xv || xt) {  // whole staged groups: 128 bytes of the rows, or 32 (f32) / 64 (bf16) k-rows
        const int ub = xv ? 128 * F::LINES / (F::KBLK * (int)sizeof(T)) : (int)(128 / esz) / F::KBLK;
        bpg = (bpg + ub - 1) / ub * ub;
    }
    groups = (nblk + bpg - 1) / bpg;
    float* part = nullptr;
    if (groups > 1) {
        part = (float*)ch::scratch(8, (size_t)(batch * groups * part_per_group));
        if (!part) return CLEAVE_HIP_ERR_OOM;
    }
#define CH_SK_ARGS X, V, y, part, R, S, K, xs_r, xs_k, vs_s, vs_k, ys_i, ys_s, x_batch, v_batch, y_batch, batch, nrb, \
                   (int)groups, bpg
    if (xv) return vv ? skinny_mfma_launch<T, MR, RB, 1, true>(CH_SK_ARGS)
                      : skinny_mfma_launch<T, MR, RB, 1, false>(CH_SK_ARGS);
    if (xt) return vv ? skinny_mfma_launch<T, MR, RB, 2, true>(CH_SK_ARGS)
                      : skinny_mfma_launch<T, MR, RB, 2, false>(CH_SK_ARGS);
    return vv ? skinny_mfma_launch<T, MR, RB, 0, true>(CH_SK_ARGS) : skinny_mfma_launch<T, MR, RB, 0, false>(CH_SK_ARGS);
#undef CH_SK_ARGS
}

int32_t skinny_mfma(const float* X, const float* V, float* y, int64_t R, int S, int K, int64_t xs_r, int64_t xs_k,
                    int64_t vs_s, int64_t vs_k, int64_t ys_i, int64_t ys_s, int64_t x_batch, int64_t v_batch,
                    int64_t y_batch, int batch) {
    if (S <= 16)
        return skinny_mfma_mr<float, 16, 2>(X, V, y, R, S, K, xs_r, xs_k, vs_s, vs_k, ys_i, ys_s, x_batch, v_batch,
                                            y_batch, batch);
    return skinny_mfma_mr<float, 32, 1>(X, V, y, R, S, K, xs_r, xs_k, vs_s, vs_k, ys_i, ys_s, x_batch, v_batch,
                                        y_batch, batch);
}
int32_t skinny_mfma(const uint16_t* X, const uint16_t* V, float* y, int64_t R, int S, int K, int64_t xs_r,
                    int64_t xs_k, int64_t vs_s, int64_t vs_k, int64_t ys_i, int64_t ys_s, int64_t x_batch,
                    int64_t v_batch, int64_t y_batch, int batch) {
    return skinny_mfma_mr<uint16_t, 32, 1>(X, V, y, R, S, K, xs_r, xs_k, vs_s, vs_k, ys_i, ys_s, x_batch, v_batch,
                                           y_batch, batch);
}

// C (batch x M x N) = op(A) op(B) with min(M, N) <= 32 on the matrix cores:
// X is the operand along the long output dimension, V the other.  A, B, C
// packed back to back per product.
template <typename T>
int32_t skinny_product(const T* a, const T* b, float* c, int M, int N, int K, int batch, int ta, int tb) {
    const int64_t sa = (int64_t)M * K, sb = (int64_t)K * N, sc = (int64_t)M * N;
    if (N <= M)  // X(m, k) = op(A)[m][k], V(n, k) = op(B)[k][n]
        return skinny_mfma(a, b, c, M, N, K, ta ? 1 : K, ta ? M : 1, tb ? K : 1, tb ? 1 : N, (int64_t)N, 1, sa, sb,
                           sc, batch);
    // X(n, k) = op(B)[k][n], V(m, k) = op(A)[m][k]
    return skinny_mfma(b, a, c, N, M, K, tb ? K : 1, tb ? 1 : N, ta ? 1 : K, ta ? M : 1, 1, (int64_t)N, sb, sa, sc,
                       batch);
}

// C (batch x M x N) = op(A) op(B) with M, N or K equal to 1; A, B, C packed
// back to back per product.
template <typename T>
int32_t vector_product(const T* a, const T* b, float* c, int M, int N, int K, int batch, int ta, int tb) {
    if (K == 1) return outer(a, b, c, M, N, batch);  // a: M values, b: N values per product
    if (N == 1) {
        // c[i] = sum_k op(A)[i][k] b[k]
        if (!ta) return row_dots(a, b, c, (int64_t)batch * M, K, M);  // A is M x K
        return weighted_sums(a, b, c, K, M, batch);                     // A is stored K x M
    }
    // M == 1: c[j] = sum_k a[k] op(B)[k][j]
    if (tb) return row_dots(b, a, c, (int64_t)batch * N, K, N);  // B is stored N x K
    return weighted_sums(b, a, c, K, N, batch);                   // B is K x N
}

}  // namespace

namespace ch {
int32_t matmul_vector_f32(const float* a, const float* b, float* c, int M, int N, int K, int batch, int ta, int tb) {
    return vector_product(a, b, c, M, N, K, batch, ta, tb);
}
int32_t matmul_skinny_f32(const float* a, const float* b, float* c, int M, int N, int K, int batch, int ta, int tb) {
    return skinny_product(a, b, c, M, N, K, batch, ta, tb);
}
int32_t matmul_skinny_bf16(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch, int ta,
                           int tb) {
    return skinny_product(a, b, c, M, N, K, batch, ta, tb);
}
int32_t matmul_vector_bf16(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch, int ta,
                           int tb) {
    return vector_product(a, b, c, M, N, K, batch, ta, tb);
}
}  // namespace ch
