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

// 16 bytes of T as floats.
template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
    static constexpr int N = 4;
    typedef float raw __attribute__((ext_vector_type(4)));
    __device__ static void load(const float* p, float (&o)[4]) {
        const raw r = *reinterpret_cast<const raw*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = r[i];
    }
};
template <>
struct Vec16<uint16_t> {
    static constexpr int N = 8;
    typedef uint32_t raw __attribute__((ext_vector_type(4)));
    __device__ static void load(const uint16_t* p, float (&o)[8]) {
        const raw r = *reinterpret_cast<const raw*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[2 * i] = __uint_as_float(r[i] << 16);
            o[2 * i + 1] = __uint_as_float(r[i] & 0xFFFF0000u);
        }
    }
};

// ---- row dots ---------------------------------------------------------------------
//
// y[r] = sum_k X[r][k] v[(r / rows_per_vec) * K + k] for r < rows.  A row is
// owned by `lpr` lanes (a power of two up to 64, sized to K), so a short row
// does not leave most of a wave idle; lane l of a row takes the 16-byte
// chunks l, l + lpr, ... (VEC) or the elements l, l + lpr, ... (scalar), four
// chunks in flight, and the row's lanes are then added by a shuffle tree.
template <typename T, bool VEC>
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
                        Vec16<T>::load(x + k + u * step, a[u]);
                        Vec16<T>::load(w + k + u * step, b[u]);
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u)
#pragma unroll
                        for (int e = 0; e < E; ++e) acc = acc + a[u][e] * b[u][e];
                }
                for (; k < K; k += step) {
                    float a[E], b[E];
                    Vec16<T>::load(x + k, a);
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
template <typename T, bool VEC>
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
                Vec16<T>::load(x + k + u * step, a[u]);
                Vec16<T>::load(w + k + u * step, b[u]);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int e = 0; e < E; ++e) acc = acc + a[u][e] * b[u][e];
        }
        for (; k < k1; k += step) {
            float a[E], b[E];
            Vec16<T>::load(x + k, a);
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
template <typename T, bool VEC>
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
                    Vec16<T>::load(X + (r + u) * cols + c, a[u]);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[e] = acc[e] + w[u] * a[u][e];
            }
            for (; r < r1; ++r) {
                float a[E];
                const float w = to_f32(v[r]);
                Vec16<T>::load(X + r * cols + c, a);
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

__global__ __launch_bounds__(kThreads) void wsum_stage2(const float* __restrict__ part, float* __restrict__ y,
                                                        int64_t cols, int64_t groups) {
    const int64_t b = blockIdx.y;
    const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (j >= cols) return;
    const float* p = part + b * groups * cols + j;
    float acc = p[0];
    int64_t g = 1;
    for (; g + 8 <= groups; g += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = p[(g + u) * cols];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = acc + t[u];
    }
    for (; g < groups; ++g) acc = acc + p[g * cols];
    y[b * cols + j] = acc;
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
// Y[i][s] = sum_k X[i][k] V(s, k) for i < R, s < S <= SB, with X k-contiguous
// (pitch K) and V(s, k) = V[s*vs_s + k*vs_k].  A workgroup owns 32 rows of X,
// eight lanes per row; it walks K in chunks of 256, staging V's chunk in LDS
// as [SB][k] (zeros past S and K), and lane l of a row takes the 16-byte
// pieces l, l + 8, ... of the chunk, so eight lanes read one 128-byte line.
// Staged as [k][SB], the lanes' reads of four k apart fell on the same banks:
// 65536 x N x 4096 took 0.93 ms at N = 10 and 1.86 ms at N = 32.
// Each value of X meets SB values of V (fma); the row's eight lanes are then
// added by a shuffle tree.  Batch entries along blockIdx.y.
constexpr int kSkinnyKC = 256, kSkinnyRows = kThreads / 8;

template <typename T, int SB, bool VEC>
__global__ __launch_bounds__(kThreads) void skinny_dots_kernel(
    const T* __restrict__ X, const T* __restrict__ V, float* __restrict__ y, int64_t R, int S, int K,
    int64_t vs_s, int64_t vs_k, int64_t ys_i, int64_t ys_s, int64_t x_batch, int64_t v_batch, int64_t y_batch) {
    // rows padded by 4 floats: the staging writes of consecutive s then spread over the banks
    __shared__ __attribute__((aligned(16))) float vs[SB][kSkinnyKC + 4];
    const int64_t b = blockIdx.y;
    X += b * x_batch;
    V += b * v_batch;
    y += b * y_batch;
    const int l8 = threadIdx.x & 7;
    const int64_t row = (int64_t)blockIdx.x * kSkinnyRows + (threadIdx.x >> 3);
    const T* x = X + (row < R ? row : 0) * (int64_t)K;
    float acc[SB];
#pragma unroll
    for (int s = 0; s < SB; ++s) acc[s] = 0.0f;
    for (int kc0 = 0; kc0 < K; kc0 += kSkinnyKC) {
        __syncthreads();  // the previous chunk's readers are done
        // consecutive threads read consecutive elements of V: along k when V's
        // rows are k-contiguous, along s when V is stored k-major
        if (vs_k == 1) {
            for (int i = threadIdx.x; i < kSkinnyKC * SB; i += kThreads) {
                const int s = i / kSkinnyKC, k = i % kSkinnyKC;
                vs[s][k] = (s < S && kc0 + k < K) ? to_f32(V[s * vs_s + (int64_t)(kc0 + k)]) : 0.0f;
            }
        } else {
            for (int i = threadIdx.x; i < kSkinnyKC * SB; i += kThreads) {
                const int k = i / SB, s = i % SB;
                vs[s][k] = (s < S && kc0 + k < K) ? to_f32(V[s * vs_s + (int64_t)(kc0 + k) * vs_k]) : 0.0f;
            }
        }
        __syncthreads();
        if (row < R) {
#pragma unroll 2
            for (int j = 0; j < kSkinnyKC / 32; ++j) {
                const int kl = 32 * j + 4 * l8;  // this lane's 4 k of the chunk
                float xv[4];
                if constexpr (VEC) {
                    if (kc0 + kl >= K) continue;  // K % 4 == 0: whole pieces only
                    load4(x + kc0 + kl, xv);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) xv[e] = kc0 + kl + e < K ? to_f32(x[kc0 + kl + e]) : 0.0f;
                }
                // vs[s][kl .. kl+3]: the row's eight lanes read one 128-byte
                // stretch of a row of vs, so the reads do not conflict
#pragma unroll
                for (int s = 0; s < SB; ++s) {
                    typedef float f4 __attribute__((ext_vector_type(4)));
                    const f4 v4 = *reinterpret_cast<const f4*>(&vs[s][kl]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[s] = __builtin_fmaf(xv[e], v4[e], acc[s]);
                }
            }
        }
    }
#pragma unroll
    for (int s = 0; s < SB; ++s)
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) acc[s] = acc[s] + __shfl_xor(acc[s], o);
    if (row < R && l8 == 0) {
#pragma unroll
        for (int s = 0; s < SB; ++s)
            if (s < S) y[row * ys_i + s * ys_s] = acc[s];
    }
}

// Y[j][s] = sum_k X[k][j] W(k, s) for j < J, s < S <= SB, with X j-contiguous
// (pitch J) and W(k, s) = W[k*ws_k + s*ws_s].  Stage 1: a thread owns four
// columns (VEC) or one and walks a group of rows in ascending order, W's rows
// of the group staged in LDS 64 at a time, into part[b][group][s][j]; stage 2
// adds the groups in ascending order.
constexpr int kSkinnyWK = 64;

template <typename T, int SB, bool VEC>
__global__ __launch_bounds__(kThreads) void skinny_sums_stage1(
    const T* __restrict__ X, const T* __restrict__ W, float* __restrict__ part, int K, int64_t J, int S,
    int64_t ws_k, int64_t ws_s, int64_t nseg, int64_t groups, int64_t rpg, int64_t x_batch, int64_t w_batch) {
    constexpr int E = VEC ? 4 : 1;
    __shared__ float ws[kSkinnyWK][SB];
    const int64_t b = blockIdx.y;
    X += b * x_batch;
    W += b * w_batch;
    const int64_t seg = blockIdx.x % nseg, group = blockIdx.x / nseg;
    const int64_t c = (seg * kThreads + threadIdx.x) * E;
    const int64_t r0 = group * rpg;
    const int64_t r1 = r0 + rpg < K ? r0 + rpg : K;
    float acc[SB][E];
#pragma unroll
    for (int s = 0; s < SB; ++s)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[s][e] = 0.0f;
    for (int64_t k0 = r0; k0 < r1; k0 += kSkinnyWK) {
        __syncthreads();
        for (int i = threadIdx.x; i < kSkinnyWK * SB; i += kThreads) {
            const int k = i / SB, s = i % SB;
            ws[k][s] = (s < S && k0 + k < r1) ? to_f32(W[(k0 + k) * ws_k + s * ws_s]) : 0.0f;
        }
        __syncthreads();
        if (c < J) {
            const int64_t kn = r1 - k0 < kSkinnyWK ? r1 - k0 : kSkinnyWK;
            for (int k = 0; k < kn; ++k) {
                float xv[E];
                const T* xr = X + (k0 + k) * J + c;
                if constexpr (VEC) {
                    load4(xr, xv);
                } else {
                    xv[0] = to_f32(xr[0]);
                }
#pragma unroll
                for (int s = 0; s < SB; ++s)
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[s][e] = __builtin_fmaf(xv[e], ws[k][s], acc[s][e]);
            }
        }
    }
    if (c >= J) return;
    float* p = part + (b * groups + group) * (int64_t)S * J + c;
#pragma unroll
    for (int s = 0; s < SB; ++s)
        if (s < S) {
#pragma unroll
            for (int e = 0; e < E; ++e) p[s * J + e] = acc[s][e];
        }
}

__global__ __launch_bounds__(kThreads) void skinny_sums_stage2(const float* __restrict__ part, float* __restrict__ y,
                                                               int64_t J, int S, int64_t groups, int64_t ys_j,
                                                               int64_t ys_s, int64_t y_batch) {
    const int64_t b = blockIdx.y;
    const int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x;  // s * J + j
    if (t >= (int64_t)S * J) return;
    const int64_t s = t / J, j = t - s * J;
    const int64_t gs = (int64_t)S * J;
    const float* p = part + b * groups * gs + t;
    float acc = p[0];
    int64_t g = 1;
    for (; g + 8 <= groups; g += 8) {  // eight loads in flight, added in order
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[(g + u) * gs];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = acc + v[u];
    }
    for (; g < groups; ++g) acc = acc + p[g * gs];
    y[b * y_batch + j * ys_j + s * ys_s] = acc;
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
        if (vec)
            row_dots_split_kernel<T, true><<<g, kThreads, 0, ch::stream()>>>(X, v, part, K, rows_per_vec, (int)slices, slice);
        else
            row_dots_split_kernel<T, false><<<g, kThreads, 0, ch::stream()>>>(X, v, part, K, rows_per_vec, (int)slices, slice);
        int32_t st = ch::check_hip(hipGetLastError(), "row_dots_split_kernel");
        if (st != CLEAVE_HIP_OK) return st;
        row_dots_fold<<<(unsigned)((rows + kThreads - 1) / kThreads), kThreads, 0, ch::stream()>>>(part, y, rows,
                                                                                                   (int)slices);
        return ch::check_hip(hipGetLastError(), "row_dots_fold");
    }
    if (vec)
        row_dots_kernel<T, true><<<capped_grid(blocks), kThreads, 0, ch::stream()>>>(X, v, y, rows, K, rows_per_vec, lpr);
    else
        row_dots_kernel<T, false><<<capped_grid(blocks), kThreads, 0, ch::stream()>>>(X, v, y, rows, K, rows_per_vec, lpr);
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
    if (vec)
        wsum_stage1<T, true><<<g1, kThreads, 0, ch::stream()>>>(X, v, part, K, cols, nseg, groups, rpg);
    else
        wsum_stage1<T, false><<<g1, kThreads, 0, ch::stream()>>>(X, v, part, K, cols, nseg, groups, rpg);
    int32_t st = ch::check_hip(hipGetLastError(), "wsum_stage1");
    if (st != CLEAVE_HIP_OK) return st;
    const dim3 g2((unsigned)((cols + kThreads - 1) / kThreads), (unsigned)batch);
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

template <typename T, int SB>
int32_t skinny_dots_sb(const T* X, const T* V, float* y, int64_t R, int S, int K, int64_t vs_s, int64_t vs_k,
                       int64_t ys_i, int64_t ys_s, int64_t x_batch, int64_t v_batch, int64_t y_batch, int batch) {
    const bool vec = K % 4 == 0 && ((uintptr_t)X % (4 * sizeof(T))) == 0;
    const dim3 g((unsigned)((R + kSkinnyRows - 1) / kSkinnyRows), (unsigned)batch);
    if (vec)
        skinny_dots_kernel<T, SB, true><<<g, kThreads, 0, ch::stream()>>>(X, V, y, R, S, K, vs_s, vs_k, ys_i, ys_s,
                                                                         x_batch, v_batch, y_batch);
    else
        skinny_dots_kernel<T, SB, false><<<g, kThreads, 0, ch::stream()>>>(X, V, y, R, S, K, vs_s, vs_k, ys_i, ys_s,
                                                                          x_batch, v_batch, y_batch);
    return ch::check_hip(hipGetLastError(), "skinny_dots_kernel");
}

template <typename T, int SB>
int32_t skinny_sums_sb(const T* X, const T* W, float* y, int K, int64_t J, int S, int64_t ws_k, int64_t ws_s,
                       int64_t ys_j, int64_t ys_s, int64_t x_batch, int64_t w_batch, int64_t y_batch, int batch) {
    const bool vec = J % 4 == 0 && ((uintptr_t)X % (4 * sizeof(T))) == 0;
    const int E = vec ? 4 : 1;
    const int64_t nseg = ((J + E - 1) / E + kThreads - 1) / kThreads;
    // about four blocks per CU over the batch, and partials (S values per
    // column per group) at most a quarter of the bytes of X
    int64_t groups = 4LL * ch::num_cus() / (nseg * batch);
    const int64_t by_bytes = (int64_t)K * (int64_t)sizeof(T) / (16LL * S);
    if (groups > by_bytes) groups = by_bytes;
    if (groups < 1) groups = 1;
    if (groups > K) groups = K;
    const int64_t rpg = (K + groups - 1) / groups;
    groups = (K + rpg - 1) / rpg;
    float* part = (float*)ch::scratch(8, sizeof(float) * (size_t)(batch * groups * S * J));
    if (!part) return CLEAVE_HIP_ERR_OOM;
    const dim3 g1((unsigned)(nseg * groups), (unsigned)batch);
    if (vec)
        skinny_sums_stage1<T, SB, true><<<g1, kThreads, 0, ch::stream()>>>(X, W, part, K, J, S, ws_k, ws_s, nseg,
                                                                           groups, rpg, x_batch, w_batch);
    else
        skinny_sums_stage1<T, SB, false><<<g1, kThreads, 0, ch::stream()>>>(X, W, part, K, J, S, ws_k, ws_s, nseg,
                                                                            groups, rpg, x_batch, w_batch);
    int32_t st = ch::check_hip(hipGetLastError(), "skinny_sums_stage1");
    if (st != CLEAVE_HIP_OK) return st;
    const dim3 g2((unsigned)(((int64_t)S * J + kThreads - 1) / kThreads), (unsigned)batch);
    skinny_sums_stage2<<<g2, kThreads, 0, ch::stream()>>>(part, y, J, S, groups, ys_j, ys_s, y_batch);
    return ch::check_hip(hipGetLastError(), "skinny_sums_stage2");
}

template <typename T>
int32_t skinny_dots(const T* X, const T* V, float* y, int64_t R, int S, int K, int64_t vs_s, int64_t vs_k,
                    int64_t ys_i, int64_t ys_s, int64_t x_batch, int64_t v_batch, int64_t y_batch, int batch) {
    if (S <= 4) return skinny_dots_sb<T, 4>(X, V, y, R, S, K, vs_s, vs_k, ys_i, ys_s, x_batch, v_batch, y_batch, batch);
    if (S <= 8) return skinny_dots_sb<T, 8>(X, V, y, R, S, K, vs_s, vs_k, ys_i, ys_s, x_batch, v_batch, y_batch, batch);
    if (S <= 16)
        return skinny_dots_sb<T, 16>(X, V, y, R, S, K, vs_s, vs_k, ys_i, ys_s, x_batch, v_batch, y_batch, batch);
    return skinny_dots_sb<T, 32>(X, V, y, R, S, K, vs_s, vs_k, ys_i, ys_s, x_batch, v_batch, y_batch, batch);
}

template <typename T>
int32_t skinny_sums(const T* X, const T* W, float* y, int K, int64_t J, int S, int64_t ws_k, int64_t ws_s,
                    int64_t ys_j, int64_t ys_s, int64_t x_batch, int64_t w_batch, int64_t y_batch, int batch) {
    if (S <= 4) return skinny_sums_sb<T, 4>(X, W, y, K, J, S, ws_k, ws_s, ys_j, ys_s, x_batch, w_batch, y_batch, batch);
    if (S <= 8) return skinny_sums_sb<T, 8>(X, W, y, K, J, S, ws_k, ws_s, ys_j, ys_s, x_batch, w_batch, y_batch, batch);
    if (S <= 16)
        return skinny_sums_sb<T, 16>(X, W, y, K, J, S, ws_k, ws_s, ys_j, ys_s, x_batch, w_batch, y_batch, batch);
    return skinny_sums_sb<T, 32>(X, W, y, K, J, S, ws_k, ws_s, ys_j, ys_s, x_batch, w_batch, y_batch, batch);
}

// C (batch x M x N) = op(A) op(B) with min(M, N) <= 32: the matrix operand
// whose long side is the output's streams once; the small operand is staged
// in LDS.  A, B, C packed back to back per product.
template <typename T>
int32_t skinny_product(const T* a, const T* b, float* c, int M, int N, int K, int batch, int ta, int tb) {
    const int64_t sa = (int64_t)M * K, sb = (int64_t)K * N, sc = (int64_t)M * N;
    if (N <= M) {
        // S = N: C[m][n] = sum_k op(A)[m][k] op(B)[k][n]; B(n, k) at tb ? n*K + k : k*N + n
        const int64_t vs_s = tb ? K : 1, vs_k = tb ? 1 : N;
        if (!ta)  // A is M x K: rows of A against the N vectors of B
            return skinny_dots(a, b, c, M, N, K, vs_s, vs_k, (int64_t)N, 1, sa, sb, sc, batch);
        // A is stored K x M: C[m][n] = sum_k A[k][m] B(n, k)
        return skinny_sums(a, b, c, K, M, N, vs_k, vs_s, (int64_t)N, 1, sa, sb, sc, batch);
    }
    // S = M: C[m][n] = sum_k A(m, k) op(B)[k][n]; A(m, k) at ta ? k*M + m : m*K + k
    const int64_t vs_s = ta ? 1 : K, vs_k = ta ? M : 1;
    if (tb)  // B is stored N x K: rows of B against the M vectors of A
        return skinny_dots(b, a, c, N, M, K, vs_s, vs_k, 1, (int64_t)N, sb, sa, sc, batch);
    // B is K x N: C[m][n] = sum_k B[k][n] A(m, k)
    return skinny_sums(b, a, c, K, N, M, vs_k, vs_s, 1, (int64_t)N, sb, sa, sc, batch);
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
