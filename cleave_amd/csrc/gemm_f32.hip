// gemm_f32.hip -- fp32 matmul on CDNA4 matrix cores (v_mfma_f32_32x32x2f32).
//
// Shapes that divide a 256 x 256 x 16 tile, with a tile per CU, run the
// ping-pong kernel of gemm_f32_pingpong.hpp; shapes that divide a
// 128 x 128 x 16 tile run the large-tile kernel of gemm_f32_tiled.hpp (LDS
// filled by global_load_lds, four MFMA k-steps per 16-byte operand read),
// also on 128 x 64 tiles when those balance the CUs better; small products
// run 32 x 32 tiles with K split over a workgroup's waves
// (gemm_f32_small.hpp), or the large-tile kernel with 64 x 64 tiles.  Large
// products of other shapes run those kernels on zero-padded copies
// (gemm_pad.hpp); the rest run the general kernel below.
//
// Replaces linalg.matmul as cleave lowers it (stdlib/linalg/matrix.cleave:27-61,
// region cleave/src/mlir_lower.rs:2089-2120): C = 0; C[i,j] += A[i,k]*B[k,j].
// The A^T B and A B^T forms are the reverse-mode halves of the MatMul product
// rule (stdlib/linalg/matrix.cleave:24).
//
// General kernel (one workgroup = one BM x BN tile of C):
//   * 256 threads = 4 waves in a 2 x 2 grid; each wave owns a (BM/2) x (BN/2)
//     block made of 32 x 32 MFMA tiles, accumulators kept in registers.
//   * K is walked in BK slices.  Both operands are staged in LDS k-major
//     ([k][m] and [k][n]) so every MFMA operand read is 32 consecutive floats
//     per half-wave (conflict-free ds_read_b32).  A slice that is contiguous
//     along m/n in global memory is copied with 16-byte stores; one that is
//     contiguous along k is transposed on the way in.
//   * Two LDS buffers: the next slice's global loads are issued before the
//     current slice's MFMAs, and written to the other buffer afterwards, so a
//     single barrier per slice suffices.
//   * Workgroups are dispatched round-robin over the 8 XCDs; the tile index is
//     remapped so each XCD works on a contiguous, grouped band of tiles and its
//     private L2 sees the A rows / B columns its neighbours also read.
//   * EDGE instantiations guard every global access (any M, N, K); the fast
//     path needs M % BM == N % BN == K % BK == 0.
#include "common.hpp"
#include "gemm_common.hpp"
#include "gemm_f32_pingpong.hpp"
#include "gemm_f32_small.hpp"
#include "gemm_f32_tiled.hpp"
#include "gemm_pad.hpp"

namespace ch {
int32_t matmul_vector_f32(const float* a, const float* b, float* c, int M, int N, int K, int batch, int ta, int tb);
int32_t matmul_skinny_f32(const float* a, const float* b, float* c, int M, int N, int K, int batch, int ta, int tb);
}

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
// Native clang vectors: HIP's float4 struct defeats register promotion of the
// staging arrays (they land in scratch memory).
typedef float f4 __attribute__((ext_vector_type(4)));

template <int BM, int BN, int BK, bool TA, bool TB, bool EDGE>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A,
                                                       const float* __restrict__ B,
                                                       float* __restrict__ C, int M, int N,
                                                       int K, int64_t lda, int64_t ldb,
                                                       int64_t ldc, int64_t strideA,
                                                       int64_t strideB, int64_t strideC,
                                                       int tiles_m, int tiles_n) {
    constexpr int NT = 256;
    constexpr int WTM = BM / 2, WTN = BN / 2;  // wave tile
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int PA = BM + 4, PB = BN + 4;  // LDS row pitch (floats)
    __shared__ float As[2][BK][PA];
    __shared__ float Bs[2][BK][PB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    int tm, tn;
    ch::tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    A += (int64_t)blockIdx.y * strideA;
    B += (int64_t)blockIdx.y * strideB;
    C += (int64_t)blockIdx.y * strideC;

    // ---- global -> register staging -------------------------------------
    constexpr int A_VEC = BM * BK / 4 / NT;  // float4 per thread
    constexpr int B_VEC = BN * BK / 4 / NT;
    static_assert(A_VEC * NT * 4 == BM * BK && B_VEC * NT * 4 == BN * BK, "tile/threads");
    f4 ra[A_VEC], rb[B_VEC];

    auto load_a = [&](int k0) {
#pragma unroll
        for (int q = 0; q < A_VEC; ++q) {
            int idx = tid + NT * q;
            int r, c;  // element (m, k) of the first of 4
            if (!TA) { r = idx / (BK / 4); c = (idx % (BK / 4)) * 4; }  // along k
            else     { c = idx / (BM / 4); r = (idx % (BM / 4)) * 4; }  // along m
            int gm = m0 + r, gk = k0 + c;
            if (!EDGE) {
                const float* p = !TA ? A + (int64_t)gm * lda + gk : A + (int64_t)gk * lda + gm;
                ra[q] = *reinterpret_cast<const f4*>(p);
            } else {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    int mm = !TA ? gm : gm + e, kk = !TA ? gk + e : gk;
                    v[e] = (mm < M && kk < K) ? (!TA ? A[(int64_t)mm * lda + kk] : A[(int64_t)kk * lda + mm]) : 0.0f;
                }
                ra[q] = f4{v[0], v[1], v[2], v[3]};
            }
        }
    };
    auto load_b = [&](int k0) {
#pragma unroll
        for (int q = 0; q < B_VEC; ++q) {
            int idx = tid + NT * q;
            int r, c;  // element (k, n) of the first of 4
            if (!TB) { r = idx / (BN / 4); c = (idx % (BN / 4)) * 4; }  // along n
            else     { c = idx / (BK / 4); r = (idx % (BK / 4)) * 4; }  // along k
            int gk = k0 + r, gn = n0 + c;
            if (!EDGE) {
                const float* p = !TB ? B + (int64_t)gk * ldb + gn : B + (int64_t)gn * ldb + gk;
                rb[q] = *reinterpret_cast<const f4*>(p);
            } else {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    int kk = !TB ? gk : gk + e, nn = !TB ? gn + e : gn;
                    v[e] = (kk < K && nn < N) ? (!TB ? B[(int64_t)kk * ldb + nn] : B[(int64_t)nn * ldb + kk]) : 0.0f;
                }
                rb[q] = f4{v[0], v[1], v[2], v[3]};
            }
        }
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int q = 0; q < A_VEC; ++q) {
            int idx = tid + NT * q;
            if (!TA) {
                int m = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
                As[buf][k + 0][m] = ra[q].x;
                As[buf][k + 1][m] = ra[q].y;
                As[buf][k + 2][m] = ra[q].z;
                As[buf][k + 3][m] = ra[q].w;
            } else {
                int k = idx / (BM / 4), m = (idx % (BM / 4)) * 4;
                *reinterpret_cast<f4*>(&As[buf][k][m]) = ra[q];
            }
        }
    };
    auto store_b = [&](int buf) {
#pragma unroll
        for (int q = 0; q < B_VEC; ++q) {
            int idx = tid + NT * q;
            if (!TB) {
                int k = idx / (BN / 4), n = (idx % (BN / 4)) * 4;
                *reinterpret_cast<f4*>(&Bs[buf][k][n]) = rb[q];
            } else {
                int n = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
                Bs[buf][k + 0][n] = rb[q].x;
                Bs[buf][k + 1][n] = rb[q].y;
                Bs[buf][k + 2][n] = rb[q].z;
                Bs[buf][k + 3][n] = rb[q].w;
            }
        }
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16f{};

    const int nk = (K + BK - 1) / BK;
    load_a(0);
    load_b(0);
    store_a(0);
    store_b(0);
    __syncthreads();

    const int half = lane >> 5, col = lane & 31;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = (kt + 1) < nk;
        if (more) {
            load_a((kt + 1) * BK);
            load_b((kt + 1) * BK);
        }
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) a[i] = As[cur][kk + half][wm * WTM + i * 32 + col];
#pragma unroll
            for (int j = 0; j < FN; ++j) b[j] = Bs[cur][kk + half][wn * WTN + j * 32 + col];
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            store_a(cur ^ 1);
            store_b(cur ^ 1);
        }
        __syncthreads();
    }

    // ---- epilogue: 32x32 accumulator layout, lane holds column lane%32 and
    // rows 8*(v/4) + 4*(lane/32) + v%4 for v = 0..15.
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                int r = m0 + wm * WTM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                int c = n0 + wn * WTN + j * 32 + col;
                if (!EDGE || (r < M && c < N)) C[(int64_t)r * ldc + c] = acc[i][j][v];
            }
}

constexpr int BM = 128, BN = 128, BK = 16;

template <bool TA, bool TB>
int32_t launch_general(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda,
               int64_t ldb, int64_t ldc, int batch, int64_t sA, int64_t sB, int64_t sC) {
    // The 16-byte loads of the fast path also need every row start aligned.
    const bool fast = (M % BM == 0) && (N % BN == 0) && (K % BK == 0) && (lda % 4 == 0) &&
                      (ldb % 4 == 0) && (sA % 4 == 0) && (sB % 4 == 0) &&
                      ((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)batch);
    if (fast)
        gemm_f32_kernel<BM, BN, BK, TA, TB, false><<<grid, 256, 0, ch::stream()>>>(
            a, b, c, M, N, K, lda, ldb, ldc, sA, sB, sC, tiles_m, tiles_n);
    else
        gemm_f32_kernel<BM, BN, BK, TA, TB, true><<<grid, 256, 0, ch::stream()>>>(
            a, b, c, M, N, K, lda, ldb, ldc, sA, sB, sC, tiles_m, tiles_n);
    CH_LAUNCHED("gemm_f32_kernel");
    return CLEAVE_HIP_OK;
}

// Large-tile kernel (gemm_f32_tiled.hpp) when the shape divides its tile;
// false when it does not.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, bool TA, bool TB>
bool launch_tiled(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda,
                  int64_t ldb, int batch, int64_t sA, int64_t sB, int64_t sC, int32_t* status) {
    using P = ch::F32Tiled<BM, BN, BK, WM, WN, STAGES, !TA, TB>;
    if (!P::fits(M, N, K, lda, ldb) || ((uintptr_t)a & 15) || ((uintptr_t)b & 15) || (sA % 4) ||
        (sB % 4))
        return false;
    const int tiles_m = M / BM, tiles_n = N / BN;
    if ((int64_t)tiles_m * tiles_n * batch > 0x7FFFFFFF) return false;
    dim3 grid((unsigned)(tiles_m * tiles_n * batch));
    ch::gemm_f32_tiled_kernel<BM, BN, BK, WM, WN, STAGES, !TA, TB><<<grid, P::THREADS, 0, ch::stream()>>>(
        a, b, c, M, N, K, lda, ldb, sA, sB, sC, tiles_m, tiles_n, batch);
    *status = ch::check_hip(hipGetLastError(), "gemm_f32_tiled_kernel");
    return true;
}

// The tiled kernel's EDGE form (gemm_f32_tiled.hpp) on any shape whose
// operands it can mask (fits_edge); false otherwise.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, bool TA, bool TB>
bool launch_tiled_edge(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda,
                       int64_t ldb, int batch, int64_t sA, int64_t sB, int64_t sC, int32_t* status,
                       bool padded = false) {
    using P = ch::F32Tiled<BM, BN, BK, WM, WN, STAGES, !TA, TB>;
    if (!P::fits_edge(M, N, K, lda, ldb, padded) || ((uintptr_t)a & 15) || ((uintptr_t)b & 15) || (sA % 4) || (sB % 4))
        return false;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    if ((int64_t)tiles_m * tiles_n * batch > 0x7FFFFFFF) return false;
    dim3 grid((unsigned)(tiles_m * tiles_n * batch));
    ch::gemm_f32_tiled_kernel<BM, BN, BK, WM, WN, STAGES, !TA, TB, true><<<grid, P::THREADS, 0, ch::stream()>>>(
        a, b, c, M, N, K, lda, ldb, sA, sB, sC, tiles_m, tiles_n, batch);
    *status = ch::check_hip(hipGetLastError(), "gemm_f32_tiled_kernel");
    return true;
}

// Small-product kernel (gemm_f32_small.hpp): 32 x 32 tiles, K split over
// K/64 waves of the workgroup; false when the shape does not fit it.
template <bool TA, bool TB>
bool launch_small(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda,
                  int64_t ldb, int batch, int64_t sA, int64_t sB, int64_t sC, int32_t* status) {
    using P = ch::F32Small;
    if (!P::fits(M, N, K, lda, ldb, !TA, TB)) return false;
    if (!TA && (((uintptr_t)a & 15) || (sA % 4))) return false;  // 16-byte loads along k
    if (TB && (((uintptr_t)b & 15) || (sB % 4))) return false;
    const int tiles_m = M / P::TILE, tiles_n = N / P::TILE;
    if ((int64_t)tiles_m * tiles_n * batch > 0x7FFFFFFF) return false;
    dim3 grid((unsigned)(tiles_m * tiles_n * batch));
    ch::gemm_f32_small_kernel<!TA, TB><<<grid, 64 * (K / P::KW), 0, ch::stream()>>>(
        a, b, c, M, N, K, lda, ldb, sA, sB, sC, tiles_m, tiles_n, batch);
    *status = ch::check_hip(hipGetLastError(), "gemm_f32_small_kernel");
    return true;
}

// Ping-pong kernel (gemm_f32_pingpong.hpp) when the shape divides its
// TILE x TILE x 16 tile; false when it does not.  kslices > 1: the batch is
// that many K slices of each of batch / kslices products (the kernel's
// kslices form).
template <bool TA, bool TB, int TILE = 256>
bool launch_pingpong(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda,
                     int64_t ldb, int batch, int64_t sA, int64_t sB, int64_t sC, int32_t* status,
                     int kslices = 1) {
    using P = ch::F32PingPong<!TA, TB, 0, TILE>;
    if (!P::fits(M, N, K, lda, ldb) || ((uintptr_t)a & 15) || ((uintptr_t)b & 15) || (sA % 4) || (sB % 4))
        return false;
    const int tiles_m = M / P::BM, tiles_n = N / P::BN;
    if ((int64_t)tiles_m * tiles_n * batch > 0x7FFFFFFF) return false;
    dim3 grid((unsigned)(tiles_m * tiles_n * batch));
    ch::gemm_f32_pingpong_kernel<!TA, TB, 0, TILE><<<grid, P::THREADS, 0, ch::stream()>>>(
        a, b, c, M, N, K, lda, ldb, sA, sB, sC, tiles_m, tiles_n, batch, kslices, ch::MlpFuse{});
    *status = ch::check_hip(hipGetLastError(), "gemm_f32_pingpong_kernel");
    return true;
}

// c[i] = part[0][i] + part[1][i] + ... + part[S-1][i], in slice order; n is
// a multiple of 4 and every slice 16-byte aligned.
__global__ __launch_bounds__(256) void sum_slices_kernel(const float* __restrict__ part, float* __restrict__ c,
                                                         int64_t n, int S, int64_t stride) {
    const int64_t n4 = n / 4 * 4;
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < n4; i += (int64_t)gridDim.x * 256 * 4) {
        f4 acc = *reinterpret_cast<const f4*>(part + i);
        int s = 1;
        for (; s + 8 <= S; s += 8) {  // eight loads in flight, added in order
            f4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const f4*>(part + (int64_t)(s + u) * stride + i);
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = acc + v[u];
        }
        for (; s < S; ++s) acc = acc + *reinterpret_cast<const f4*>(part + (int64_t)s * stride + i);
        *reinterpret_cast<f4*>(c + i) = acc;
    }
    // the last n % 4 entries, in the same order
    if (blockIdx.x == 0 && threadIdx.x < n - n4) {
        const int64_t i = n4 + threadIdx.x;
        float acc = part[i];
        for (int s = 1; s < S; ++s) acc = acc + part[(int64_t)s * stride + i];
        c[i] = acc;
    }
}

// K slices for a product with few tiles and a long K.  S (a power of two)
// slices are computed as S products into a scratch buffer and added in order
// (deterministic).  Shapes of 256 x 256 tiles: slices that fill the CUs with
// ping-pong tiles, each at least 2048 deep, so that the partial sums' extra
// traffic (S + 1 passes over C) stays a few percent of the product.
// Otherwise, with fewer 64 x 64 tiles than CUs: up to two workgroups per CU
// on the small-product or 64 x 64 kernels, each slice at least 512 deep.
// 1 = no split.
int split_count(int M, int N, int K) {
    const int cus = ch::num_cus();
    if (M % 256 == 0 && N % 256 == 0) {
        const int64_t tiles = (int64_t)(M / 256) * (N / 256);
        int S = 1;
        while (tiles * S * 2 <= cus && K % (16 * S * 2) == 0 && K / (S * 2) >= 2048) S *= 2;
        // the slices must fill the CUs for the ping-pong kernel to take them
        if (tiles * S >= cus) return S;
    }
    // 128 x 128 tiles that one round of their ping-pong kernel would leave
    // under 77% full: K slices for that kernel (1024^2 x 4096: 66.7 against
    // 77.2 us as 64 x 64 tiles; 1024^2 x 8192 121.9 against 152.6; 512^2 x
    // 16384 66.9 against 72.0 as 8 slices of 64 x 64 tiles)
    if (M % 128 == 0 && N % 128 == 0 && (double)(M / 128) * (N / 128) < 0.77 * cus) {
        const int64_t tiles = (int64_t)(M / 128) * (N / 128);
        // as many slices, at least 512 deep, as fit one round, if that round
        // is at least 77% full (384 x 3072^2: 3 slices, 216 tiles)
        for (int S = (int)(cus / tiles); S >= 2; --S)
            if (K % (16 * S) == 0 && K / S >= 512) {
                if (tiles * S >= 0.77 * cus) return S;
                break;
            }
        // else a power of two that fills at least a round
        int S = 1;
        while (tiles * S < cus && K % (16 * S * 2) == 0 && K / (S * 2) >= 1024) S *= 2;
        if (S > 1 && tiles * S >= cus) return S;
    }
    if (M % 64 || N % 64) return 1;
    const int64_t tiles = (int64_t)(M / 64) * (N / 64);
    if (tiles >= cus) return 1;
    int S = 1;
    while (tiles * S * 2 <= 2 * cus && K % (64 * S * 2) == 0 && K / (S * 2) >= 512) S *= 2;
    return S;
}

int32_t dispatch(const float* a, const float* b, float* c, int M, int N, int K, int batch, int ta, int tb,
                 int splits);

}  // namespace

namespace ch {
// c (n entries) = the S slices of part, `stride` floats apart, added in
// order; stride % 4 == 0, c and part 16-byte aligned.  Also the bf16
// products' K slices (gemm_bf16.hip).
int32_t sum_slices_f32(const float* part, float* c, int64_t n, int S, int64_t stride) {
    const int64_t blocks = (n / 4 + 255) / 256, cap = (int64_t)ch::num_cus() * 8;
    const int64_t grid = blocks < 1 ? 1 : (blocks < cap ? blocks : cap);
    sum_slices_kernel<<<(unsigned)grid, 256, 0, ch::stream()>>>(part, c, n, S, stride);
    return ch::check_hip(hipGetLastError(), "sum_slices_kernel");
}
}  // namespace ch

namespace {

template <bool TA, bool TB>
int32_t launch(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda, int64_t ldb,
               int64_t ldc, int batch, int64_t sA, int64_t sB, int64_t sC);

// launch<TA, TB> for run-time flags.
int32_t launch_layout(int ta, int tb, const float* a, const float* b, float* c, int M, int N, int K, int64_t lda,
                      int64_t ldb, int64_t ldc, int batch, int64_t sA, int64_t sB, int64_t sC) {
    if (!ta && !tb) return launch<false, false>(a, b, c, M, N, K, lda, ldb, ldc, batch, sA, sB, sC);
    if (!ta && tb) return launch<false, true>(a, b, c, M, N, K, lda, ldb, ldc, batch, sA, sB, sC);
    if (ta && !tb) return launch<true, false>(a, b, c, M, N, K, lda, ldb, ldc, batch, sA, sB, sC);
    return launch<true, true>(a, b, c, M, N, K, lda, ldb, ldc, batch, sA, sB, sC);
}

// One product (batch 1, C of pitch N; A and B of pitches lda and ldb, so that
// a band of a larger product's rows keeps its operand pitches) as S > 1 K
// slices (K a multiple of 16 S) computed into the slice buffer and added in
// order, when that buffer can be had: *st is the outcome; false when not
// split.
bool run_k_slices(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda, int64_t ldb, int ta,
                  int tb, int S, int32_t* st) {
    if (((uintptr_t)c & 15) != 0) return false;
    float* part = S > 1 ? (float*)ch::scratch_try(9, sizeof(float) * (size_t)S * M * N) : nullptr;
    if (!part) return false;
    const int kk = K / S;
    const int64_t sA = ta ? (int64_t)kk * lda : kk, sB = tb ? kk : (int64_t)kk * ldb;
    *st = launch_layout(ta, tb, a, b, part, M, N, kk, lda, ldb, N, S, sA, sB, (int64_t)M * N);
    if (*st == CLEAVE_HIP_OK) *st = ch::sum_slices_f32(part, c, (int64_t)M * N, S, (int64_t)M * N);
    return true;
}

// split_count's K slices, when it asks for more than one.
bool try_k_split(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda, int64_t ldb, int ta,
                 int tb, int32_t* st) {
    return run_k_slices(a, b, c, M, N, K, lda, ldb, ta, tb, split_count(M, N, K), st);
}

// Rough time of `batch` aligned products launched together, in us, by the
// kernel the launchers pick: rounds of 256 x 256 tiles (0.96 of peak per
// tile), rounds of 128 x 128 tiles on the ping-pong kernel (0.93) when the
// last is at least 77% full, the tiled kernels (0.78 of that, as measured at
// 2176^3 - 3584^3), or, below a round, small tiles (0.70).
double est_launch_us(int M, int N, int K, int batch) {
    const double cus = ch::num_cus() > 0 ? ch::num_cus() : 1, peak = 157.3e12;
    const int64_t big = (int64_t)(M / 256) * (N / 256) * batch, t128 = (int64_t)(M / 128) * (N / 128) * batch;
    if (M % 256 == 0 && N % 256 == 0 && big >= cus)
        return std::ceil(big / cus) * cus * 2.0 * 256 * 256 * K / (peak * 0.96) * 1e6;
    const double flops = 2.0 * M * N * K * batch;
    if (M % 128 == 0 && N % 128 == 0 && t128 >= 0.77 * cus) {
        const double rounds = std::ceil(t128 / cus);
        if (t128 >= 0.77 * rounds * cus) return rounds * cus * 2.0 * 128 * 128 * K / (peak * 0.93) * 1e6;
        return flops / (peak * 0.93 * 0.78) * 1e6;
    }
    return flops / (peak * 0.70) * 1e6;
}

// The slice sum's S + 1 passes over an M x N C at 6.5 TB/s, plus 4 us of
// launches.
double est_sum_us(int M, int N, int S) { return (S + 1) * 4.0 * M * N / 6.5e12 * 1e6 + 4.0; }

// Rough time of one aligned product as launched: split_count's K slices
// when it asks for them, else one launch.
double est_us(int M, int N, int K) {
    const int S = split_count(M, N, K);
    if (S > 1) return est_launch_us(M, N, K / S, S) + est_sum_us(M, N, S);
    return est_launch_us(M, N, K, 1);
}

int32_t product(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda, int64_t ldb, int ta,
                int tb, int depth);

// A product whose tiles (256 x 256 from a round of them, else 128 x 128 from
// more than a round) end in a ragged round: the first M1 rows of C, the
// whole rounds, run as one product and the remaining rows as another, which
// takes its own kernel (K slices, 128 x 128 tiles, or a split of its own).
// Returns M1 (0: no such split) and, in *us, est_us of the two parts plus
// 4 us for the extra launches.  Measured (128 x 128 tiles; the rest as K
// slices that fill one more round, added in order into their rows): 3072^3
// 409 against 451 us, 3584^3 644 against 826, 2304^3 184 against 207, 2176^3
// 157 against 196, 3072^2 x 1024 151 against 156.
int round_split_rows(int M, int N, int K, double* us) {
    const int cus = ch::num_cus() > 0 ? ch::num_cus() : 1;
    if (K % 16) return 0;
    const int64_t big = (int64_t)(M / 256) * (N / 256), t128 = (int64_t)(M / 128) * (N / 128);
    int tile;
    int64_t T;
    if (M % 256 == 0 && N % 256 == 0 && big >= cus) tile = 256, T = big;
    else if (M % 128 == 0 && N % 128 == 0 && t128 > cus) tile = 128, T = t128;
    else return 0;
    const int tn = N / tile, tm = M / tile;
    const int t1 = (int)(T / cus * cus / tn);  // tile-rows of whole rounds
    if (t1 <= 0 || t1 >= tm) return 0;
    const int M1 = t1 * tile;
    *us = est_us(M1, N, K) + est_us(M - M1, N, K) + 4.0;
    return M1;
}

// K slices of a product of more than a round of 128 x 128 tiles, S of them
// (2-8, each at least 1024 deep, too few 256 x 256 tiles for that kernel to
// take them) so that the slices' tiles fill at least 90% of their last
// round: est_launch_us of the slices (rounds of the 128 x 128 ping-pong
// kernel) plus the slice sum.  Returns the cheapest S (0: none) and its time
// in *us.
int round_slices(int M, int N, int K, double* us) {
    const int cus = ch::num_cus() > 0 ? ch::num_cus() : 1;
    if (M % 128 || N % 128) return 0;
    const int64_t t = (int64_t)(M / 128) * (N / 128);
    const int64_t big = (M % 256 == 0 && N % 256 == 0) ? (int64_t)(M / 256) * (N / 256) : 0;
    if (t <= cus) return 0;
    int best = 0;
    for (int S = 2; S <= 8; ++S) {
        if (K % (16 * S) || K / S < 1024 || big * S >= cus) continue;
        const double rounds = std::ceil((double)(t * S) / cus);
        if ((double)(t * S) < 0.9 * rounds * cus) continue;
        const double u = est_launch_us(M, N, K / S, S) + est_sum_us(M, N, S);
        if (!best || u < *us) best = S, *us = u;
    }
    return best;
}

// One product (batch 1, C of pitch N; A and B of pitches lda and ldb, so that
// a band of a larger product's rows keeps its operand pitches): K slices
// for few tiles; at a ragged round, a band of rows or K slices that fill
// whole rounds, where the estimate is at least 3% under the whole's, and
// the slices only 8% under the band's (the estimate prices the band's tiled
// kernels low where all their tiles are resident at once: 1024 x 5632 x 2048
// ran 185 us as a band, 189 as slices).  Measured: 2048 x
// 3072 x 4032 (384 tiles) as 2 slices in 3 full rounds 352 us against 411 as
// a band of 768 rows; 896 x 5632 x 4096 (308) as 4 slices in 5 rounds 310
// against 330; 1536 x 4096^2 (384) stays a band of 512 rows, 351 against 358
// as slices; else the launchers.  Deterministic: the kernels are chosen by
// the shape alone, and slices are added in order.
int32_t product(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda, int64_t ldb, int ta,
                int tb, int depth) {
    int32_t st = CLEAVE_HIP_OK;
    if (try_k_split(a, b, c, M, N, K, lda, ldb, ta, tb, &st)) return st;
    const bool aligned = ((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0 && ((uintptr_t)c & 15) == 0;
    if (depth < 3 && aligned) {
        const double whole = est_us(M, N, K);
        double us_rows = 0, us_sl = 0;
        const int M1 = round_split_rows(M, N, K, &us_rows);
        const int S = round_slices(M, N, K, &us_sl);
        if (S && us_sl < 0.97 * whole && (!M1 || us_sl < 0.92 * us_rows) &&
            run_k_slices(a, b, c, M, N, K, lda, ldb, ta, tb, S, &st))
            return st;
        if (M1 && us_rows < 0.97 * whole) {
            // A keeps its full pitch (its rows, or with ta its columns, are offset)
            const float* a2 = ta ? a + M1 : a + (int64_t)M1 * lda;
            st = product(a, b, c, M1, N, K, lda, ldb, ta, tb, depth + 1);
            if (st == CLEAVE_HIP_OK) st = product(a2, b, c + (int64_t)M1 * N, M - M1, N, K, lda, ldb, ta, tb, depth + 1);
            return st;
        }
    }
    return launch_layout(ta, tb, a, b, c, M, N, K, lda, ldb, N, 1, (int64_t)M * K, (int64_t)K * N,
                         (int64_t)M * N);
}

// The aligned kernels; false when none takes the shape.
template <bool TA, bool TB>
bool launch_fast(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda,
                 int64_t ldb, int64_t ldc, int batch, int64_t sA, int64_t sB, int64_t sC, int32_t* st) {
    if (ldc == N) {
        // 256 x 256 x 16 tile (ping-pong, 8 waves of 128 x 64) when it still
        // yields a tile per CU; smaller shapes below.
        const int64_t big_tiles = (int64_t)(M / 256) * (N / 256) * batch;
        if (big_tiles >= ch::num_cus() &&
            launch_pingpong<TA, TB>(a, b, c, M, N, K, lda, ldb, batch, sA, sB, sC, st))
            return true;
        // Up to two 32 x 32 tiles per CU with K <= 1024 (config 1's 256^3 is
        // 64 tiles): a tile per workgroup, K split over its waves, 32 MFMAs
        // per wave.  Measured against 64 x 64 tiles: 512^3 6.2 against
        // 11.7 us, 640^3 (400 tiles) 12.7 against 14.5, 512 x 1024 x 512
        // (512 tiles) 10.1 against 12.1; 768^3 (576 tiles) 19.2 against 17.4.
        const int cus = ch::num_cus();
        const int64_t tiles32 = (int64_t)(M / 32) * (N / 32) * batch;
        if (tiles32 <= 2 * cus &&
            launch_small<TA, TB>(a, b, c, M, N, K, lda, ldb, batch, sA, sB, sC, st))
            return true;
        // The ping-pong kernel on 128 x 128 tiles (8 waves of 64 x 32, a
        // 6-deep ring: one workgroup per CU) where its last round of tiles is
        // at least 77% full.  Against the tiled kernels below: 2048^3 117.6
        // against 131.2 us, 2048^2 x 4096 229.6 against 256.8, 3072 x 4096 x
        // 2048 (three rounds) 349.7 against 363.4, 2560^3 (400 tiles, 78%)
        // 285.0 against 304.1; 3072^3 (576, 75%) 510.4 against 453.8 and
        // 2304^3 (324, 63%) 256.7 against 208.2 stay tiled.
        const int64_t tiles128 = (int64_t)(M / 128) * (N / 128) * batch;
        {
            const int64_t rounds = (tiles128 + cus - 1) / cus;
            if (tiles128 > 0 && (double)tiles128 >= 0.77 * (double)(rounds * cus) &&
                launch_pingpong<TA, TB, 128>(a, b, c, M, N, K, lda, ldb, batch, sA, sB, sC, st))
                return true;
        }
        // Fewer 128 x 128 tiles than CUs: 64 x 64 tiles with a 4-deep ring
        // (five workgroups per CU) put the product on 4x the CUs.  1024^3 23.9
        // against 66.7 us on 128 x 128 tiles, 1280^3 49.0 against 84.7,
        // 1536^3 82.9 against 103; a 16-deep ring measured 2-18% slower.
        if (tiles128 < cus &&
            launch_tiled<64, 64, 16, 2, 2, 4, TA, TB>(a, b, c, M, N, K, lda, ldb, batch, sA, sB, sC, st))
            return true;
        // 128 x 128 tiles run four workgroups per CU, 128 x 64 tiles six.
        // Where the last round of 128 x 128 tiles would fill under 70% of
        // the CUs' slots, the twice as many 128 x 64 tiles balance better:
        // 2304^3 (324 tiles) 233 against 282 us, 3072^3 (576) 489 against
        // 551, 4224^3 (1089) 1122 against 1222; at 3072 x 4096 x 2048 (768,
        // 75%) 414 against 397, at 4096^2 x 1024 (1024, full) 289 against 271.
        if (tiles128 > cus) {
            const int64_t slots = 4 * (int64_t)cus, rounds = (tiles128 + slots - 1) / slots;
            if ((double)tiles128 < 0.7 * (double)(rounds * slots) &&
                launch_tiled<128, 64, 16, 2, 2, 2, TA, TB>(a, b, c, M, N, K, lda, ldb, batch, sA, sB, sC, st))
                return true;
        }
        if (launch_tiled<128, 128, 16, 2, 2, 2, TA, TB>(a, b, c, M, N, K, lda, ldb, batch, sA, sB, sC, st))
            return true;
    }
    return false;
}

// Products of at least this many flops (2 M N K per product) that no aligned
// kernel takes run on zero-padded copies (gemm_pad.hpp); smaller ones run
// the general kernel, one launch against the padded route's three (~10 us
// together; measured when it was four).  Measured crossing: ~80^3 (64 x 64 x 63 10.2 us general, 12.4
// padded; 100^3 15.9 against 12.5).
constexpr double kPadMinFlops = 1u << 20;
// Skinny products (gemv.hip) from the same size: 3 x 5 x 7 took 7.2 us there
// (two launches) against 4.7 us on the general kernel.
constexpr double kSkinnyMinFlops = 1u << 20;
// 256 x 256 tiles (4096^3) 0.86 of peak, one workgroup per CU; 128 x 128
// tiles (4224^3) 0.78, four workgroups per CU.  4097^3 measured 1.23 ms
// padded to 4224^3, 1.83 ms padded to 4352^2 x 4160 (289 tiles of 256).
constexpr ch::PadModel kPadModel{0.86, 0.78, false, 1.0};
constexpr int64_t kEdgeTilesPerCu = 4;

// Time of one 64 x 64 guarded-edge tile per k on a CU, in microseconds,
// whatever the number of tiles sharing it (one to five): 2000^3 (four tiles
// a CU) 132 us, 2500 x 640 x 16384 (two on most CUs) 535.
constexpr double kEdgeTileKUs = 0.0163;
// The same for a 128 x 128 tile (3000 x 5000 x 2000, four tiles on most
// CUs, 479 us): 8% less per flop than 64 x 64 when the tiles are many.
constexpr double kEdge128TileKUs = 0.0599;

// One ragged product (an M or N off the 64 grid) with a long K as S K
// slices on the 64 x 64 kernel's guarded-edge form, its batch running over
// the slices, added in order (deterministic); each slice at least 512 deep
// and whole 16-byte chunks (K % 4S == 0).  At most a round of tiles: the
// most slices, up to kEdgeTilesPerCu tiles per CU over all of them (2048 x
// 200 x 2000: 40.2 us in one launch of 128 tiles).  Up to kEdgeTilesPerCu
// tiles per CU and K from 4096: the count (up to 16) that evens out the
// tiles per CU, priced as the busiest CU's tiles times the slice depth
// (kEdgeTileKUs) plus the slices written and read back at 5 TB/s, when that
// saves 5%: 2500 x 640 x 16384 (400 tiles, 2 on most CUs) 8 slices, 535 ->
// 437-446 us; 1500^2 x 16384 A^T.B 4, 792 -> 603; 1200 x 1100 x 12000 A.B^T
// 5, 377 -> 278; 1536 x 1100 x 8192 4, 269 -> 239.  From K = 4096 the
// slices run on 128 x 128 tiles instead (up to 4 per CU) where the same
// pricing (kEdge128TileKUs) puts them 3% under the 64 x 64 choice, at
// least three per CU: 1000^2 x 65536 16 slices, 1082 -> 988 us; 1000^2 x
// 32768 A.B^T 532 -> 503; 1001 x 1003 x 32768 (aligned copies) 586 -> 554;
// 2000^2 x 8192 4 slices (unsplit before) 530 -> 506.  It priced 700 x 900 x 30000
// and 512 x 2000 x 20000 within 3% of their times on 128 x 128 tiles (373
// and 372 us, against 335 and 330 on 64 x 64), which it therefore keeps.
// `padded`: the operands are aligned copies (ch::edge_chunks).  False when
// not split.
template <bool TA, bool TB>
bool try_edge_slices(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda, int64_t ldb,
                     bool padded, int32_t* st) {
    if (((uintptr_t)c & 15) || (M % 64 == 0 && N % 64 == 0)) return false;
    const int64_t cus = ch::num_cus() > 0 ? ch::num_cus() : 1;
    const int64_t tiles = (int64_t)((M + 63) / 64) * ((N + 63) / 64);
    // predicted time: the busiest CU's tiles times the slice depth, plus
    // the slices written and read back at 5 TB/s
    auto cost = [&](int64_t t, double tile_k_us, int s) {
        const double busiest = (double)((t * s + cus - 1) / cus);
        return busiest * ((double)K / s) * tile_k_us + (s > 1 ? 8.0 * s * (double)M * N / 5.0e6 : 0.0);
    };
    int S = 1;
    if (tiles <= cus) {
        S = (int)std::min<int64_t>(kEdgeTilesPerCu * cus / tiles, K / 512);
        while (S >= 2 && K % (4 * S) != 0) --S;
    } else {
        if (tiles > kEdgeTilesPerCu * cus || K < 4096) return false;
        double best = 0.95 * cost(tiles, kEdgeTileKUs, 1);
        for (int s = 2; s <= 16 && K / s >= 512; ++s)
            if (K % (4 * s) == 0 && cost(tiles, kEdgeTileKUs, s) < best) best = cost(tiles, kEdgeTileKUs, s), S = s;
    }
    bool big = false;  // 128 x 128 tiles, at least three per CU (the rate kEdge128TileKUs holds for)
    if (K >= 4096) {
        const int64_t t128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
        double best = 0.97 * cost(tiles, kEdgeTileKUs, S);
        for (int s = 2; s <= 64 && K / s >= 512 && t128 * s <= kEdgeTilesPerCu * cus; ++s)
            if (K % (4 * s) == 0 && t128 * s >= 3 * cus && cost(t128, kEdge128TileKUs, s) < best)
                best = cost(t128, kEdge128TileKUs, s), S = s, big = true;
    }
    if (S < 2) return false;
    const int kk = K / S;
    const int64_t sA = TA ? (int64_t)kk * lda : kk, sB = TB ? kk : (int64_t)kk * ldb;
    using P = ch::F32Tiled<64, 64, 16, 2, 2, 4, !TA, TB>;
    if (!P::fits_edge(M, N, kk, lda, ldb, padded) || ((uintptr_t)a & 15) || ((uintptr_t)b & 15) || sA % 4 ||
        sB % 4)
        return false;
    const int64_t n = (int64_t)M * N, n4 = (n + 3) / 4 * 4;
    float* part = (float*)ch::scratch_try(9, sizeof(float) * (size_t)S * n4);
    if (!part) return false;
    bool launched;
    if (big)
        launched =
            launch_tiled_edge<128, 128, 16, 2, 2, 2, TA, TB>(a, b, part, M, N, kk, lda, ldb, S, sA, sB, n4, st, padded);
    else
        launched =
            (tiles * S <= 2 * cus &&
             launch_tiled_edge<64, 64, 32, 2, 2, 4, TA, TB>(a, b, part, M, N, kk, lda, ldb, S, sA, sB, n4, st, padded)) ||
            launch_tiled_edge<64, 64, 16, 2, 2, 4, TA, TB>(a, b, part, M, N, kk, lda, ldb, S, sA, sB, n4, st, padded);
    if (!launched) *st = launch_general<TA, TB>(a, b, part, M, N, kk, lda, ldb, N, S, sA, sB, n4);
    if (*st == CLEAVE_HIP_OK) *st = ch::sum_slices_f32(part, c, n, S, n4);
    return true;
}

template <bool TA, bool TB>
int32_t launch(const float* a, const float* b, float* c, int M, int N, int K, int64_t lda,
               int64_t ldb, int64_t ldc, int batch, int64_t sA, int64_t sB, int64_t sC) {
    int32_t st = CLEAVE_HIP_OK;
    if (launch_fast<TA, TB>(a, b, c, M, N, K, lda, ldb, ldc, batch, sA, sB, sC, &st)) return st;
    // whole packed products only (not the K-slices of a split product)
    const bool packed = lda == (TA ? M : K) && ldb == (TB ? K : N) && ldc == N && sA == (int64_t)M * K &&
                        sB == (int64_t)K * N && sC == (int64_t)M * N;
    // one output dimension of at most 32: stream the long operand (gemv.hip);
    // tiny products stay on the general kernel (one launch)
    if (packed && (M <= 32 || N <= 32) && 2.0 * M * N * K * batch >= kSkinnyMinFlops)
        return ch::matmul_skinny_f32(a, b, c, M, N, K, batch, TA, TB);
    if (packed && 2.0 * M * N * K * batch >= kPadMinFlops) {
        // Up to kEdgeTilesPerCu tiles of 64 x 64 per CU: the 64 x 64 kernel
        // with guarded edges on the operands in place, one launch.  Up to two
        // tiles per CU its k-tiles are 32 deep (64 KiB of LDS, two workgroups
        // per CU), beyond that 16 (five): f32 1000^3 22.4 against 23.8 us,
        // 1000 x 2000 x 1000 37.7 against 38.3, 500^3 12.1 against 13.0;
        // 1500^3 80.1 against 77.1, 2000^3 136.9 against 132.2.  With K up to
        // 512 also beyond that: padding such a product's C and cropping it
        // moved more than the math took (10000^2 x 256 604 against 470 us on
        // padded copies, 3000^2 x 500 103 against 82, 5000 x 8000 x 300 A.B^T
        // 269 against 229; 16000^2 x 128 A^T.B level).
        const int64_t tiles64 = (int64_t)((M + 63) / 64) * ((N + 63) / 64) * batch;
        const int64_t cus = ch::num_cus();
        const bool edge16 = tiles64 <= kEdgeTilesPerCu * cus || K <= 512;
        // The same kernels on aligned copies (ch::run_aligned): K slices for
        // one product with a long K over few or unevenly spread tiles
        // (try_edge_slices), else one launch.
        auto edge = [&](const float* pa, const float* pb, int64_t plda, int64_t pldb, int64_t psA, int64_t psB,
                        int Kq, int32_t* s) {
            if (batch == 1 && try_edge_slices<TA, TB>(pa, pb, c, M, N, Kq, plda, pldb, true, s)) return true;
            if (tiles64 <= 2 * cus && launch_tiled_edge<64, 64, 32, 2, 2, 4, TA, TB>(
                                          pa, pb, c, M, N, Kq, plda, pldb, batch, psA, psB, sC, s, true))
                return true;
            return launch_tiled_edge<64, 64, 16, 2, 2, 4, TA, TB>(pa, pb, c, M, N, Kq, plda, pldb, batch, psA, psB,
                                                                  sC, s, true);
        };
        if (batch == 1 && try_edge_slices<TA, TB>(a, b, c, M, N, K, lda, ldb, false, &st)) return st;
        // Few tiles and a long K that the slices do not divide: K rounded up
        // to a multiple of 2048 in aligned copies of both operands, then the
        // slices.
        if (batch == 1 && K >= 16384 && K % 2048 != 0 && (M % 64 || N % 64) && tiles64 <= cus) {
            const ch::AlignPlan kp = ch::align_plan(M, N, K, batch, TA, TB, a, b, 4, 2048);
            if (ch::run_aligned(kp, a, b, M, N, K, batch, TA, TB, edge, &st)) return st;
        }
        if (tiles64 <= 2 * cus &&
            launch_tiled_edge<64, 64, 32, 2, 2, 4, TA, TB>(a, b, c, M, N, K, lda, ldb, batch, sA, sB, sC, &st))
            return st;
        if (edge16 &&
            launch_tiled_edge<64, 64, 16, 2, 2, 4, TA, TB>(a, b, c, M, N, K, lda, ldb, batch, sA, sB, sC, &st))
            return st;
        // Rows that are not whole 16-byte chunks (an extent that is not a
        // multiple of 4, a misaligned view): the same kernels on aligned
        // copies of those operands, C in place.  Against the padded route
        // below (same box, two runs): 1001^3 30.5 against 33.8 us, 3000 x
        // 3001 x 501 89 against 105.
        if (edge16) {
            const ch::AlignPlan ap = ch::align_plan(M, N, K, batch, TA, TB, a, b, 4);
            if (ch::run_aligned(ap, a, b, M, N, K, batch, TA, TB, edge, &st)) return st;
        }
        // Past four 64 x 64 tiles per CU with K over 512, at least three
        // 128 x 128 tiles per CU: that kernel with guarded edges, in place,
        // instead of padded copies and a crop (same box, two runs: 3000 x
        // 5000 x 2000 506 -> 479 us, 4000^2 x 1000 A^T.B^T 268 -> 250, 4000 x
        // 3000 x 3000 A^T.B 553 -> 543, 6000^3 level).  With fewer tiles it
        // ran slower than the routes above: 1500^3 101 against 78 us (144
        // tiles), 3000 x 1000 x 6000 A.B^T 384 against 295 (192), 2500^2 x
        // 4096 497 against 457 on the padded route (400).
        const int64_t tiles128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128) * batch;
        if (!edge16 && tiles128 >= 3 * cus &&
            launch_tiled_edge<128, 128, 16, 2, 2, 2, TA, TB>(a, b, c, M, N, K, lda, ldb, batch, sA, sB, sC, &st))
            return st;
        const ch::PadPlan p = ch::pad_plan(M, N, K, batch, TA, TB, a, b, 4, ch::num_cus(), kPadModel);
        auto gemm = [batch](const float* pa, const float* pb, float* pc, int Mp, int Np, int Kp) {
            const int64_t plda = TA ? Mp : Kp, pldb = TB ? Kp : Np;
            const int64_t psA = (int64_t)Mp * Kp, psB = (int64_t)Kp * Np, psC = (int64_t)Mp * Np;
            int32_t s = CLEAVE_HIP_OK;
            if (batch == 1) return product(pa, pb, pc, Mp, Np, Kp, plda, pldb, TA, TB, 0);
            if (launch_fast<TA, TB>(pa, pb, pc, Mp, Np, Kp, plda, pldb, Np, batch, psA, psB, psC, &s)) return s;
            return launch_general<TA, TB>(pa, pb, pc, Mp, Np, Kp, plda, pldb, Np, batch, psA, psB, psC);
        };
        if (ch::run_padded(p, a, b, c, batch, TA, TB, gemm, &st)) return st;
    }
    return launch_general<TA, TB>(a, b, c, M, N, K, lda, ldb, ldc, batch, sA, sB, sC);
}

// A batch of packed products with fewer 128 x 128 tiles than 77% of a round
// and a long K: S K slices of each product, at least 512 deep, whose tiles
// fill one round at least 77%, in one launch of the 128 x 128 ping-pong
// kernel, then added in order (deterministic).  *st is the outcome; false
// when not split.
template <bool TA, bool TB>
bool try_batched_k_slices(const float* a, const float* b, float* c, int M, int N, int K, int batch, int32_t* st) {
    const int cus = ch::num_cus() > 0 ? ch::num_cus() : 1;
    if (M % 128 || N % 128 || ((uintptr_t)c & 15)) return false;
    const int64_t t = (int64_t)(M / 128) * (N / 128) * batch;
    if (t >= 0.77 * cus) return false;
    int S = 0;
    for (int s = (int)(cus / t); s >= 2; --s)
        if (K % (16 * s) == 0 && K / s >= 512) {
            if (t * s >= 0.77 * cus) S = s;
            break;
        }
    if (S == 0 || (int64_t)batch * S > 0x7FFFFFFF) return false;
    const int64_t n = (int64_t)batch * M * N;
    float* part = (float*)ch::scratch_try(9, sizeof(float) * (size_t)S * n);
    if (!part) return false;
    const int64_t lda = TA ? M : K, ldb = TB ? K : N;
    if (!launch_pingpong<TA, TB, 128>(a, b, part, M, N, K / S, lda, ldb, batch * S, (int64_t)M * K,
                                      (int64_t)K * N, (int64_t)M * N, st, S))
        return false;
    if (*st == CLEAVE_HIP_OK) *st = ch::sum_slices_f32(part, c, n, S, n);
    return true;
}

// batch >= 1 independent products packed back to back, or (splits > 1, batch
// must be 1) one product whose K range is cut into `splits` equal slices,
// slice s writing its partial sum to c + s*M*N.
int32_t dispatch(const float* a, const float* b, float* c, int M, int N, int K, int batch,
                 int ta, int tb, int splits) {
    // a dimension of 1: matrix-vector or outer products (gemv.hip)
    if (splits <= 1 && (M == 1 || N == 1 || K == 1)) return ch::matmul_vector_f32(a, b, c, M, N, K, batch, ta, tb);
    const int64_t lda = ta ? M : K, ldb = tb ? K : N, ldc = N;
    if (splits <= 1 && batch == 1) return product(a, b, c, M, N, K, lda, ldb, ta, tb, 0);
    if (splits <= 1) {
        int32_t st = CLEAVE_HIP_OK;
        bool done;
        if (!ta && !tb) done = try_batched_k_slices<false, false>(a, b, c, M, N, K, batch, &st);
        else if (!ta && tb) done = try_batched_k_slices<false, true>(a, b, c, M, N, K, batch, &st);
        else if (ta && !tb) done = try_batched_k_slices<true, false>(a, b, c, M, N, K, batch, &st);
        else done = try_batched_k_slices<true, true>(a, b, c, M, N, K, batch, &st);
        if (done) return st;
    }
    int64_t sA = (int64_t)M * K, sB = (int64_t)K * N, sC = (int64_t)M * N;
    int kk = K;
    if (splits > 1) {
        kk = K / splits;
        sA = ta ? (int64_t)kk * lda : kk;
        sB = tb ? kk : (int64_t)kk * ldb;
        batch = splits;
    }
    if (!ta && !tb) return launch<false, false>(a, b, c, M, N, kk, lda, ldb, ldc, batch, sA, sB, sC);
    if (!ta && tb) return launch<false, true>(a, b, c, M, N, kk, lda, ldb, ldc, batch, sA, sB, sC);
    if (ta && !tb) return launch<true, false>(a, b, c, M, N, kk, lda, ldb, ldc, batch, sA, sB, sC);
    return launch<true, true>(a, b, c, M, N, kk, lda, ldb, ldc, batch, sA, sB, sC);
}

}  // namespace

namespace ch {
// Internal entry used by the MLP step (same kernels, no argument checks).
// splits > 1 requires K % splits == 0 and c sized splits*M*N.
int32_t gemm_f32_device(const float* a, const float* b, float* c, int M, int N, int K, int ta,
                        int tb, int splits) {
    return dispatch(a, b, c, M, N, K, 1, ta, tb, splits);
}
}  // namespace ch

extern "C" {

int32_t cleave_hip_matmul_f32(const float* a, int64_t alen, const float* b, int64_t blen,
                              float* c, int64_t clen, int32_t M, int32_t N, int32_t K,
                              int32_t trans_a, int32_t trans_b) {
    CH_REQUIRE(M > 0 && N > 0 && K > 0, "cleave_hip_matmul_f32: dims must be positive (M=%d N=%d K=%d)", M, N, K);
    CH_REQUIRE((trans_a == 0 || trans_a == 1) && (trans_b == 0 || trans_b == 1),
               "cleave_hip_matmul_f32: trans flags must be 0 or 1");
    CH_REQUIRE(alen == (int64_t)M * K, "cleave_hip_matmul_f32: alen %lld != M*K %lld", (long long)alen, (long long)M * K);
    CH_REQUIRE(blen == (int64_t)K * N, "cleave_hip_matmul_f32: blen %lld != K*N %lld", (long long)blen, (long long)K * N);
    CH_REQUIRE(clen == (int64_t)M * N, "cleave_hip_matmul_f32: clen %lld != M*N %lld", (long long)clen, (long long)M * N);
    CH_REQUIRE(a && b && c, "cleave_hip_matmul_f32: null buffer");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_matmul_f32", a, alen * 4);
    CH_DEVICE("cleave_hip_matmul_f32", b, blen * 4);
    CH_DEVICE("cleave_hip_matmul_f32", c, clen * 4);
    return dispatch(a, b, c, M, N, K, 1, trans_a, trans_b, 1);
}

int32_t cleave_hip_matmul_batched_f32(const float* a, int64_t alen, const float* b,
                                      int64_t blen, float* c, int64_t clen, int32_t batch,
                                      int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                      int32_t trans_b) {
    CH_REQUIRE(batch > 0 && batch <= 65535 && M > 0 && N > 0 && K > 0,
               "cleave_hip_matmul_batched_f32: bad dims (batch=%d M=%d N=%d K=%d)", batch, M, N, K);
    CH_REQUIRE((trans_a == 0 || trans_a == 1) && (trans_b == 0 || trans_b == 1),
               "cleave_hip_matmul_batched_f32: trans flags must be 0 or 1");
    const int64_t na = ch::count3(batch, M, K), nb = ch::count3(batch, K, N), nc = ch::count3(batch, M, N);
    CH_REQUIRE(na >= 0 && nb >= 0 && nc >= 0 && alen == na && blen == nb && clen == nc,
               "cleave_hip_matmul_batched_f32: lengths do not match batch*M*K, batch*K*N, batch*M*N");
    CH_REQUIRE(a && b && c, "cleave_hip_matmul_batched_f32: null buffer");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_matmul_batched_f32", a, alen * 4);
    CH_DEVICE("cleave_hip_matmul_batched_f32", b, blen * 4);
    CH_DEVICE("cleave_hip_matmul_batched_f32", c, clen * 4);
    return dispatch(a, b, c, M, N, K, batch, trans_a, trans_b, 1);
}

}  // extern "C"
