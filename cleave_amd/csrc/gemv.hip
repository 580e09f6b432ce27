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
int32_t matmul_vector_bf16(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch, int ta,
                           int tb) {
    return vector_product(a, b, c, M, N, K, batch, ta, tb);
}
}  // namespace ch
