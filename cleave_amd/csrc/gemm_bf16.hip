// gemm_bf16.hip -- bf16-input / fp32-accumulate matmul on CDNA4 matrix cores
// (v_mfma_f32_32x32x16_bf16), plus its batched form.
//
// Shapes that divide a 256 x 256 x 32 tile run the ping-pong kernel of
// gemm_bf16_pingpong.hpp; 128 x 128 x 64 tiles run the large-tile kernel of
// gemm_bf16_tiled.hpp (LDS filled by global_load_lds,
// transposing LDS reads for m/n-contiguous operands).  Large products of
// other shapes run those kernels' guarded-edge forms on the operands in
// place, or on aligned copies of operands whose rows are not whole 16-byte
// chunks (gemm_pad.hpp); zero-padded copies of the whole product remain for
// operands past the edge forms' 2 GiB; the rest run the general kernel
// below, which guards every access.
//
// Same operator as gemm_f32.hip (linalg.matmul of stdlib/linalg/matrix.cleave:
// 27-61) with bf16 operands; the reference is f32/f64 only, so this is an
// extension checked against the f32 loop run on the upcast values.
//
// General kernel.  LDS layout: both operands are staged [row][k] with k contiguous and a row
// pitch of BK+8 elements (80 bytes), so the 16-byte MFMA operand reads of 16
// consecutive lanes land in 16 distinct bank quads.  An operand that is
// k-contiguous in global memory is copied in 16-byte chunks; one that is
// contiguous along m/n is read as 8(k) x 2(m/n) blocks of 4-byte words and
// transposed in registers before a pair of 16-byte LDS stores.
#include <type_traits>

#include "common.hpp"
#include "gemm_bf16_pingpong.hpp"
#include "gemm_bf16_tiled.hpp"
#include "gemm_common.hpp"
#include "gemm_pad.hpp"

namespace ch {
int32_t matmul_vector_bf16(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch, int ta,
                           int tb);
int32_t matmul_skinny_bf16(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch, int ta,
                           int tb);
int32_t sum_slices_f32(const float* part, float* c, int64_t n, int S, int64_t stride);
}

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
// Native clang vector (HIP's uint4 struct defeats register promotion).
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 32, NT = 256;
constexpr int PITCH = BK + 8;  // elements

// Registers holding one thread's share of a 128 x BK operand tile.
template <bool KCONTIG>
struct Stage;
template <>
struct Stage<true> {  // 128 rows x 32 k = 512 chunks of 8 -> 2 per thread
    u4 v[2];
};
template <>
struct Stage<false> {  // 64 row-pairs x 4 k-groups of 8 -> 1 block per thread
    uint32_t w[8];
};

// X is the operand, `ld` its leading dimension.  KCONTIG: element (r, k) at
// X[r*ld + k]; otherwise at X[k*ld + r].  rows/ks bound the valid region
// (EDGE only).
template <bool KCONTIG, bool EDGE>
__device__ __forceinline__ void load_tile(Stage<KCONTIG>& s, const uint16_t* __restrict__ X,
                                          int64_t ld, int r0, int k0, int rows, int ks, int tid) {
    if constexpr (KCONTIG) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            int idx = tid + NT * q;
            int r = idx >> 2, kc = (idx & 3) * 8;
            int gr = r0 + r, gk = k0 + kc;
            if (!EDGE) {
                s.v[q] = *reinterpret_cast<const u4*>(X + (int64_t)gr * ld + gk);
            } else {
                uint16_t e[8];
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    e[t] = (gr < rows && gk + t < ks) ? X[(int64_t)gr * ld + gk + t] : (uint16_t)0;
                s.v[q] = u4{e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16),
                           e[4] | ((uint32_t)e[5] << 16), e[6] | ((uint32_t)e[7] << 16)};
            }
        }
    } else {
        int rp = (tid & 63) * 2, kg = (tid >> 6) * 8;
        int gr = r0 + rp;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            int gk = k0 + kg + t;
            if (!EDGE) {
                s.w[t] = *reinterpret_cast<const uint32_t*>(X + (int64_t)gk * ld + gr);
            } else {
                uint32_t lo = (gk < ks && gr < rows) ? X[(int64_t)gk * ld + gr] : 0u;
                uint32_t hi = (gk < ks && gr + 1 < rows) ? X[(int64_t)gk * ld + gr + 1] : 0u;
                s.w[t] = lo | (hi << 16);
            }
        }
    }
}

template <bool KCONTIG>
__device__ __forceinline__ void store_tile(const Stage<KCONTIG>& s, uint16_t (*L)[PITCH], int tid) {
    if constexpr (KCONTIG) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            int idx = tid + NT * q;
            int r = idx >> 2, kc = (idx & 3) * 8;
            *reinterpret_cast<u4*>(&L[r][kc]) = s.v[q];
        }
    } else {
        int rp = (tid & 63) * 2, kg = (tid >> 6) * 8;
        u4 lo, hi;  // rows rp and rp+1, k = kg..kg+7
        lo.x = (s.w[0] & 0xFFFFu) | (s.w[1] << 16);
        lo.y = (s.w[2] & 0xFFFFu) | (s.w[3] << 16);
        lo.z = (s.w[4] & 0xFFFFu) | (s.w[5] << 16);
        lo.w = (s.w[6] & 0xFFFFu) | (s.w[7] << 16);
        hi.x = (s.w[0] >> 16) | (s.w[1] & 0xFFFF0000u);
        hi.y = (s.w[2] >> 16) | (s.w[3] & 0xFFFF0000u);
        hi.z = (s.w[4] >> 16) | (s.w[5] & 0xFFFF0000u);
        hi.w = (s.w[6] >> 16) | (s.w[7] & 0xFFFF0000u);
        *reinterpret_cast<u4*>(&L[rp][kg]) = lo;
        *reinterpret_cast<u4*>(&L[rp + 1][kg]) = hi;
    }
}

template <bool TA, bool TB, bool EDGE>
__global__ __launch_bounds__(NT) void gemm_bf16_kernel(const uint16_t* __restrict__ A,
                                                       const uint16_t* __restrict__ B,
                                                       float* __restrict__ C, int M, int N, int K,
                                                       int64_t lda, int64_t ldb, int64_t strideA,
                                                       int64_t strideB, int64_t strideC, int tiles_m,
                                                       int tiles_n) {
    constexpr bool AK = !TA;  // A k-contiguous when stored M x K
    constexpr bool BKC = TB;  // B k-contiguous when stored N x K
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][PITCH];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN][PITCH];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    ch::tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    A += (int64_t)blockIdx.y * strideA;
    B += (int64_t)blockIdx.y * strideB;
    C += (int64_t)blockIdx.y * strideC;

    Stage<AK> sa;
    Stage<BKC> sb;
    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v16f{};

    const int nk = (K + BK - 1) / BK;
    load_tile<AK, EDGE>(sa, A, lda, m0, 0, M, K, tid);
    load_tile<BKC, EDGE>(sb, B, ldb, n0, 0, N, K, tid);
    store_tile<AK>(sa, As[0], tid);
    store_tile<BKC>(sb, Bs[0], tid);
    __syncthreads();

    const int half = lane >> 5, r32 = lane & 31;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            load_tile<AK, EDGE>(sa, A, lda, m0, (kt + 1) * BK, M, K, tid);
            load_tile<BKC, EDGE>(sb, B, ldb, n0, (kt + 1) * BK, N, K, tid);
        }
#pragma unroll
        for (int ks = 0; ks < BK; ks += 16) {
            v8bf a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const v8bf*>(&As[cur][wm * 64 + i * 32 + r32][ks + 8 * half]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const v8bf*>(&Bs[cur][wn * 64 + j * 32 + r32][ks + 8 * half]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            store_tile<AK>(sa, As[cur ^ 1], tid);
            store_tile<BKC>(sb, Bs[cur ^ 1], tid);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                int r = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                int c = n0 + wn * 64 + j * 32 + r32;
                if (!EDGE || (r < M && c < N)) C[(int64_t)r * N + c] = acc[i][j][v];
            }
}

// Operand pitches and per-product strides, in elements: packed products, or
// the K slices of one product (gemm_bf16's split below).
struct Strides {
    int64_t lda, ldb, sA, sB, sC;
    bool padded = false;  // aligned copies: every row holds its last chunk whole (ch::edge_chunks)
};
template <bool TA, bool TB>
Strides packed(int M, int N, int K) {
    return {TA ? M : K, TB ? K : N, (int64_t)M * K, (int64_t)K * N, (int64_t)M * N};
}
// Every product's operand base 16-byte aligned.
bool bases_aligned(const uint16_t* a, const uint16_t* b, const Strides& s) {
    return ((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0 && s.sA % 8 == 0 && s.sB % 8 == 0;
}

template <bool TA, bool TB>
int32_t launch(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch, const Strides& s) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)batch);
    // 4-byte (transposed) or 16-byte (k-contiguous) global reads need the
    // matching alignment of every row start.
    const bool fast = (M % BM == 0) && (N % BN == 0) && (K % BK == 0) && s.lda % 8 == 0 && s.ldb % 8 == 0 &&
                      bases_aligned(a, b, s);
    if (fast)
        gemm_bf16_kernel<TA, TB, false><<<grid, NT, 0, ch::stream()>>>(a, b, c, M, N, K, s.lda, s.ldb, s.sA, s.sB,
                                                                       s.sC, tiles_m, tiles_n);
    else
        gemm_bf16_kernel<TA, TB, true><<<grid, NT, 0, ch::stream()>>>(a, b, c, M, N, K, s.lda, s.ldb, s.sA, s.sB,
                                                                      s.sC, tiles_m, tiles_n);
    CH_LAUNCHED("gemm_bf16_kernel");
    return CLEAVE_HIP_OK;
}

// Whether the 32 x 32 store loop of the tiled kernel writes C non-temporally
// (its NTC form): C rows of whole 128-byte lines, every product's C 128-byte
// aligned.
bool nt_c(const float* c, int N, const Strides& s) {
    return N % 32 == 0 && ((uintptr_t)c & 127) == 0 && s.sC % 32 == 0;
}
// The 16 x 16 accumulator store paths (ping-pong, paired-copy and 256 x 256
// tiled kernels, tiles::store_acc16_lines) store C non-temporally when one
// launch writes at least this many bytes of it, in whole 128-byte lines.
// Same box, two runs: a C of 256 MiB or more gains (8192^3 A.B 712-718 ->
// 699-706 us, A.B^T 742 -> 714-723, 65536 x 1024 x 1024 149 -> 122, 16384^2
// x 512 437 -> 296, 16384^2 x 1024 A^T.B 622 -> 500, 32768 x 8192 x 1024 568
// -> 473); one that the 256 MiB MALL holds loses (4096^3, 64 MiB, 95.5 ->
// 98.5; batched 64 x 512^3 24.2 -> 25.1; 4096 x 8192 x 2048, 128 MiB, 106
// -> 111) or is level (6144^2 x 4096, 144 MiB, 239 -> 237).
constexpr int64_t kNtStoreBytes = 192ll << 20;
bool nt_c16(const float* c, int M, int N, int batch, const Strides& s) {
    return nt_c(c, N, s) && (int64_t)batch * M * N * 4 >= kNtStoreBytes;
}

// Large-tile kernel (gemm_bf16_tiled.hpp) for shapes that divide its tile.
// Returns false when the shape or alignment does not fit.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int MI, bool TA, bool TB>
bool launch_tiled(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch, const Strides& s,
                  int32_t* status, int kslices = 1) {
    using P = ch::Bf16Tiled<BM, BN, BK, WM, WN, STAGES, !TA, TB, MI>;
    const int64_t lda = s.lda, ldb = s.ldb;
    if (!P::fits(M, N, K, lda, ldb) || !bases_aligned(a, b, s)) return false;
    const int tiles_m = M / BM, tiles_n = N / BN;
    if ((int64_t)tiles_m * tiles_n * batch > 0x7FFFFFFF) return false;
    dim3 grid((unsigned)(tiles_m * tiles_n * batch));
    // 32 x 32 stores: non-temporal in whole lines at any size; 16 x 16: past kNtStoreBytes
    if (MI == 32 ? nt_c(c, N, s) : nt_c16(c, M, N, batch, s))
        ch::gemm_bf16_tiled_kernel<BM, BN, BK, WM, WN, STAGES, !TA, TB, MI, false, true>
            <<<grid, P::THREADS, 0, ch::stream()>>>(a, b, c, M, N, K, lda, ldb, s.sA, s.sB, s.sC, tiles_m, tiles_n,
                                                    batch, kslices);
    else
        ch::gemm_bf16_tiled_kernel<BM, BN, BK, WM, WN, STAGES, !TA, TB, MI><<<grid, P::THREADS, 0, ch::stream()>>>(
            a, b, c, M, N, K, lda, ldb, s.sA, s.sB, s.sC, tiles_m, tiles_n, batch, kslices);
    *status = ch::check_hip(hipGetLastError(), "gemm_bf16_tiled_kernel");
    return true;
}

// The tiled kernel's EDGE form (gemm_bf16_tiled.hpp) on any shape whose
// operands it can mask (fits_edge); false otherwise.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, int MI, bool TA, bool TB>
bool launch_tiled_edge(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch,
                       const Strides& s, int32_t* status) {
    using P = ch::Bf16Tiled<BM, BN, BK, WM, WN, STAGES, !TA, TB, MI>;
    if (!P::fits_edge(M, N, K, s.lda, s.ldb, s.padded) || !bases_aligned(a, b, s)) return false;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    if ((int64_t)tiles_m * tiles_n * batch > 0x7FFFFFFF) return false;
    dim3 grid((unsigned)(tiles_m * tiles_n * batch));
    if (nt_c(c, N, s))
        ch::gemm_bf16_tiled_kernel<BM, BN, BK, WM, WN, STAGES, !TA, TB, MI, true, true>
            <<<grid, P::THREADS, 0, ch::stream()>>>(a, b, c, M, N, K, s.lda, s.ldb, s.sA, s.sB, s.sC, tiles_m, tiles_n,
                                                    batch, 1);
    else
        ch::gemm_bf16_tiled_kernel<BM, BN, BK, WM, WN, STAGES, !TA, TB, MI, true>
            <<<grid, P::THREADS, 0, ch::stream()>>>(a, b, c, M, N, K, s.lda, s.ldb, s.sA, s.sB, s.sC, tiles_m, tiles_n,
                                                    batch, 1);
    *status = ch::check_hip(hipGetLastError(), "gemm_bf16_tiled_kernel");
    return true;
}

// Ragged products that the padded route would run on 128 x 128 tiles (fewer
// 256 x 256 tiles than half a round): the same tiles with guarded edges on
// the operands in place (three stages up to a round of tiles, as
// launch_fast, else two), or, for a round at most with a k-contiguous A,
// 64 x 128 tiles; false when the shape does not fit them.
template <bool TA, bool TB>
bool launch_edge(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch,
                 const Strides& s, int32_t* st) {
    const int64_t cus = ch::num_cus();
    const int64_t big = (int64_t)((M + 255) / 256) * ((N + 255) / 256) * batch;
    if (big * 2 >= cus) {
        // At least half a round of 256 x 256 tiles.  A short K runs on 128 x
        // 128 tiles, two workgroups per CU, as the aligned short-K products;
        // padding such a product's C and cropping it doubled its C traffic
        // (10000^2 x 256: 283 against 139 us, 16000^2 x 248: 760 against 330).
        // A longer K: the paired-copy kernel's EDGE form (launch_pairs_edge),
        // or for A^T.B the padded copies (on these tiles 8000^3 A^T.B took
        // 1190 against 883 us).
        const bool short_k = K <= 256 || (big <= cus && K <= 512);
        if (!short_k) return false;
        return launch_tiled_edge<128, 128, 64, 2, 2, 2, 32, TA, TB>(a, b, c, M, N, K, batch, s, st);
    }
    const int64_t tiles128 = (int64_t)((M + 127) / 128) * ((N + 127) / 128) * batch;
    if (tiles128 <= cus) {
        if constexpr (!TA) {
            if (launch_tiled_edge<64, 128, 64, 2, 2, 3, 32, TA, TB>(a, b, c, M, N, K, batch, s, st)) return true;
        }
        return launch_tiled_edge<128, 128, 64, 2, 2, 3, 32, TA, TB>(a, b, c, M, N, K, batch, s, st);
    }
    return launch_tiled_edge<128, 128, 64, 2, 2, 2, 32, TA, TB>(a, b, c, M, N, K, batch, s, st);
}

// The paired-copy kernel's EDGE form (gemm_bf16_pingpong.hpp) for ragged
// shapes in the range where their zero-padded copies would run the
// paired-copy kernel (launch_fast): at least half a round of 256 x 256
// tiles, a k-contiguous operand, and K past the short-K kernels' range (over
// 256, and over 512 for a single round); A^T.B, which has no k-contiguous
// operand, runs the single-ring ping-pong kernel's EDGE form there.  The
// copies and the crop move the operands and C once more; here they are read
// in place.  False otherwise.
template <bool TA, bool TB>
bool launch_pairs_edge(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch,
                       const Strides& s, int32_t* status) {
    if constexpr (TA && !TB) {  // A^T B: no k-contiguous operand to pair; the single-ring kernel
        using P = ch::Bf16PingPong<false, false>;
        const int64_t cus = ch::num_cus();
        const int tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
        const int64_t big = (int64_t)tiles_m * tiles_n * batch;
        if (big * 2 < cus || K <= 256 || (big <= cus && K <= 512)) return false;
        if (!P::fits_edge(M, N, K, s.lda, s.ldb, s.padded) || !bases_aligned(a, b, s)) return false;
        if (big > 0x7FFFFFFF) return false;
        if (nt_c16(c, M, N, batch, s))
            ch::gemm_bf16_pingpong_kernel<false, false, false, 5, true, true>
                <<<dim3((unsigned)big), P::THREADS, 0, ch::stream()>>>(a, b, c, M, N, K, s.lda, s.ldb, s.sA, s.sB,
                                                                       s.sC, tiles_m, tiles_n, batch);
        else
            ch::gemm_bf16_pingpong_kernel<false, false, false, 5, true>
                <<<dim3((unsigned)big), P::THREADS, 0, ch::stream()>>>(a, b, c, M, N, K, s.lda, s.ldb, s.sA, s.sB,
                                                                       s.sC, tiles_m, tiles_n, batch);
        *status = ch::check_hip(hipGetLastError(), "gemm_bf16_pingpong_kernel");
        return true;
    } else {
        using P = ch::Bf16PingPongPairs<!TA, TB, true>;
        const int64_t cus = ch::num_cus();
        const int tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
        const int64_t big = (int64_t)tiles_m * tiles_n * batch;
        if (big * 2 < cus || K <= 256 || (big <= cus && K <= 512)) return false;
        if (!P::fits_edge(M, N, K, s.lda, s.ldb, s.padded) || !bases_aligned(a, b, s)) return false;
        if (big > 0x7FFFFFFF) return false;
        const int total = (int)big;
        const int resident = cus >= 8 ? (int)(cus / 8 * 8) : (cus > 0 ? (int)cus : 1);
        dim3 grid((unsigned)(total < resident ? total : resident));
        if (nt_c16(c, M, N, batch, s))
            ch::gemm_bf16_pingpong_pairs_kernel<!TA, TB, true, true><<<grid, P::THREADS, 0, ch::stream()>>>(
                a, b, c, M, N, K, s.lda, s.ldb, s.sA, s.sB, s.sC, tiles_m, tiles_n, batch);
        else
            ch::gemm_bf16_pingpong_pairs_kernel<!TA, TB, true><<<grid, P::THREADS, 0, ch::stream()>>>(
                a, b, c, M, N, K, s.lda, s.ldb, s.sA, s.sB, s.sC, tiles_m, tiles_n, batch);
        *status = ch::check_hip(hipGetLastError(), "gemm_bf16_pingpong_pairs_kernel");
        return true;
    }
}

// Ping-pong kernel (gemm_bf16_pingpong.hpp): 256 x 256 x 32 tiles in a ring
// of five k-tiles (all 160 KiB of LDS).
template <bool TA, bool TB>
bool launch_pingpong(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch,
                     const Strides& s, int32_t* status) {
    using P = ch::Bf16PingPong<!TA, TB>;
    const int64_t lda = s.lda, ldb = s.ldb;
    if (!P::fits(M, N, K, lda, ldb) || !bases_aligned(a, b, s)) return false;
    const int tiles_m = M / P::BM, tiles_n = N / P::BN;
    if ((int64_t)tiles_m * tiles_n * batch > 0x7FFFFFFF) return false;
    dim3 grid((unsigned)(tiles_m * tiles_n * batch));
    // byte offset of the last k-tile from an operand's base: k-contiguous
    // operands step 64 bytes per k-tile, m/n-contiguous ones 32 rows
    const uint64_t last_a = (uint64_t)K * (TA ? (uint64_t)lda * 2 : 2);
    const uint64_t last_b = (uint64_t)K * (TB ? 2 : (uint64_t)ldb * 2);
    const int64_t sa = s.sA, sb = s.sB, sc = s.sC;
    const bool off32 = last_a < (1ull << 32) && last_b < (1ull << 32), nt = nt_c16(c, M, N, batch, s);
    auto go = [&](auto off32_t, auto nt_t) {
        ch::gemm_bf16_pingpong_kernel<!TA, TB, decltype(off32_t)::value, 5, false, decltype(nt_t)::value>
            <<<grid, P::THREADS, 0, ch::stream()>>>(a, b, c, M, N, K, lda, ldb, sa, sb, sc, tiles_m, tiles_n, batch);
    };
    using T = std::true_type;
    using F = std::false_type;
    if (off32) nt ? go(T{}, T{}) : go(T{}, F{});
    else nt ? go(F{}, T{}) : go(F{}, F{});
    *status = ch::check_hip(hipGetLastError(), "gemm_bf16_pingpong_kernel");
    return true;
}

// Layouts with a k-contiguous operand (A·B, Aᵀ·Bᵀ, A·Bᵀ): the ping-pong
// kernel that copies such an operand two k-tiles at a time, as whole 128-byte
// rows (gemm_bf16_pingpong.hpp; for A·Bᵀ, A is the paired one).
template <bool TA, bool TB>
bool launch_pairs(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch, const Strides& s,
                  int32_t* status) {
    if constexpr (TA && !TB) {  // Aᵀ·B: no k-contiguous operand to pair
        return false;
    } else {
        using P = ch::Bf16PingPongPairs<!TA, TB>;
        const int64_t lda = s.lda, ldb = s.ldb;
        if (!P::fits(M, N, K, lda, ldb) || !bases_aligned(a, b, s)) return false;
        const int tiles_m = M / P::BM, tiles_n = N / P::BN;
        if ((int64_t)tiles_m * tiles_n * batch > 0x7FFFFFFF) return false;
        // one workgroup per CU (all of the LDS), each looping over its tiles;
        // a multiple of 8 keeps every tile of a workgroup on one XCD
        const int total = tiles_m * tiles_n * batch;
        const int cus = ch::num_cus();
        const int resident = cus >= 8 ? cus / 8 * 8 : (cus > 0 ? cus : 1);
        dim3 grid((unsigned)(total < resident ? total : resident));
        if (nt_c16(c, M, N, batch, s))
            ch::gemm_bf16_pingpong_pairs_kernel<!TA, TB, false, true><<<grid, P::THREADS, 0, ch::stream()>>>(
                a, b, c, M, N, K, lda, ldb, s.sA, s.sB, s.sC, tiles_m, tiles_n, batch);
        else
            ch::gemm_bf16_pingpong_pairs_kernel<!TA, TB><<<grid, P::THREADS, 0, ch::stream()>>>(
                a, b, c, M, N, K, lda, ldb, s.sA, s.sB, s.sC, tiles_m, tiles_n, batch);
        *status = ch::check_hip(hipGetLastError(), "gemm_bf16_pingpong_pairs_kernel");
        return true;
    }
}

// The aligned kernels; false when none takes the shape.
template <bool TA, bool TB>
bool launch_fast(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch, const Strides& s,
                 int32_t* st) {
    // 256 x 256 tiles, when there are enough of them (below): the ping-pong
    // kernel (k-tiles of 32), or the tiled kernel (k-tiles of 64).  With one
    // round of tiles and K up to 512 the two measured equal (64 x 512^3:
    // 25.0-29.3 against 25.5-26.9 us over two runs; 4096^2 x 512: 26.1-26.7
    // against 26.3 us) and the tiled kernel is kept; from K = 1024 the
    // ping-pong kernel is 2-5% faster (4096^2 x 2048: 58.7 against 60.5-61.7
    // us), and with several rounds more so.  With whole-line C stores in all
    // three, 64 x 512^3 measured 24.3-24.5 us tiled, 24.8-24.9 paired-copy
    // ping-pong, 25.0-25.7 single-stage ping-pong (same box).
    //
    // Enough means at least half as many tiles as CUs: one partial round of
    // them beat the 128 x 128 tiles' two or three rounds (3072^3, 144
    // tiles: 65.7 against 85.3 us; 3072 x 4096 x 2048, 192 tiles: 52.9
    // against 69.2 us), and lost below (2560^3, 100 tiles: 52.9 against
    // 45.9 us; 2048^3, 64 tiles: 39.6 against 26.1 us).
    const int cus = ch::num_cus();
    const int64_t big_tiles = (int64_t)(M / 256) * (N / 256) * batch;
    // A short K over more than a round of tiles: the products are bound by
    // their f32 C stores, which two workgroups per CU on 128 x 128 tiles
    // overlap with each other's loads and math.  Against the 256 x 256
    // kernels, one box, same run: 16384^2 x 256 314 against 355 us (A·Bᵀ 315
    // against 398), 10240^2 x 256 103 against 129, 6144^2 x 256 38 against 47,
    // 65536 x 1024 x 256 78 against 85, 8192^2 x 128 Aᵀ·B 51 against 60; but
    // 8192^2 x 256 71-77 against 69-72 (four rounds exactly).
    if (K <= 256 && K % 64 == 0 && big_tiles > cus &&
        launch_tiled<128, 128, 64, 2, 2, 2, 32, TA, TB>(a, b, c, M, N, K, batch, s, st))
        return true;
    if (big_tiles * 2 >= cus) {
        const bool short_single_round = big_tiles <= cus && K <= 512;
        if (!short_single_round && launch_pairs<TA, TB>(a, b, c, M, N, K, batch, s, st)) return true;
        if (!short_single_round && launch_pingpong<TA, TB>(a, b, c, M, N, K, batch, s, st)) return true;
        if (launch_tiled<256, 256, 64, 2, 4, 2, 16, TA, TB>(a, b, c, M, N, K, batch, s, st)) return true;
        if (launch_pingpong<TA, TB>(a, b, c, M, N, K, batch, s, st)) return true;
    }
    // 128 x 128 x 64 tiles, 4 waves of 64 x 64 in 32 x 32 x 16 MFMAs.  Up to
    // one round of them: three LDS stages (96 KiB, one workgroup per CU), or,
    // with a k-contiguous A, 64 x 128 tiles (two workgroups per CU) -- 1024^3
    // 9.7 against 12.8 us, 512^3 6.0 against 7.9, 2048^3 26.1 against 27.3.
    // Several rounds: two stages (64 KiB), two workgroups per CU -- 4224^3
    // 214 against 225 us, 2304^3 37.1 against 47.3, 3072 x 4096 x 2048 69.2
    // against 85.9.
    const int64_t tiles128 = (int64_t)(M / 128) * (N / 128) * batch;
    if (tiles128 <= cus) {
        if constexpr (!TA) {
            if (launch_tiled<64, 128, 64, 2, 2, 3, 32, TA, TB>(a, b, c, M, N, K, batch, s, st)) return true;
        }
        return launch_tiled<128, 128, 64, 2, 2, 3, 32, TA, TB>(a, b, c, M, N, K, batch, s, st);
    }
    return launch_tiled<128, 128, 64, 2, 2, 2, 32, TA, TB>(a, b, c, M, N, K, batch, s, st);
}

// K slices of one product with few 128 x 128 tiles and a long K: up to one
// workgroup per CU, each slice at least 1024 deep (the slices' partial sums
// are then small next to the product); or, where more, a count past one
// round chosen as edge_split_count chooses it (up to 4 tiles per CU, slices
// at least 2000 deep and whole 64-deep k-tiles).  Same box, two runs, against
// one round at most: 1024^2 x 65536 192 -> 116-124 us, A^T.B 173 -> 117-124;
// 1152^2 x 16384 94 -> 62; 1280^2 x 32768 A^T.B^T 150 -> 90; 1024 x 2048 x
// 16384 A.B^T 82 -> 68; 512 x 1024 x 16384 and 2048^2 x 8192 level.  1 = no
// split.
int split_count(int M, int N, int K) {
    const int cus = ch::num_cus();
    const int64_t tiles = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
    if (tiles * 2 > cus) {
        // Fewer 256 x 256 tiles than half a round (the band left by a split at
        // a ragged round, 256 x 9216^2): as many slices, at least 1024 deep,
        // as fit a round, if they make half a round, for those kernels.
        const int64_t big = (M % 256 == 0 && N % 256 == 0) ? (int64_t)(M / 256) * (N / 256) : 0;
        if (big > 0 && big * 2 < cus)
            for (int S = (int)(cus / big); S >= 2; --S)
                if (K % (64 * S) == 0 && K / S >= 1024) return big * S * 2 >= cus ? S : 1;
        return 1;
    }
    int S = 1;
    while (tiles * S * 2 <= cus && K % (64 * S * 2) == 0 && K / (S * 2) >= 1024) S *= 2;
    // past one round: the busiest CU's tiles times the slice depth
    auto work = [&](int s) { return (double)((tiles * s + cus - 1) / cus) * ((double)K / s); };
    double least = 0;
    for (int s = 2; s <= K / 2000 && tiles * s <= 4 * cus; ++s)
        if (tiles * s > cus && K % (64 * s) == 0 && (least == 0 || work(s) < least)) least = work(s);
    int past = 1;
    for (int s = 2; s <= K / 2000 && tiles * s <= 4 * cus; ++s)
        if (tiles * s > cus && K % (64 * s) == 0 && work(s) <= 1.1 * least) past = s;
    return std::max(S, past);
}

// Slices for a product the guarded-edge kernels take (M or N off the
// 128 x 128 tile, or K off the 64-deep k-tile; split_count's rules are for
// the aligned kernels), with at most a round of 128 x 128 tiles; each
// slice's depth whole 16-byte chunks (K % 8S == 0).  The more of: the most
// slices, at least 512 deep, that one round of tiles holds (128 x 300 x 5000
// A^T.B^T, three tiles, 47.7 -> 15.9 us; 300^2 x 3000 31 -> 17); and a
// count past one round, up to 4 tiles per CU over all slices, each slice at
// least 2000 deep: of those, the largest whose busiest CU's tiles times the
// slice depth is within 10% of the least.  A tile alone on a CU runs at
// about a third of the CU's bf16 rate, so more tiles per CU pay for the
// slices' partial sums, but not a third tile on some CUs where two would
// do: 1200 x 1100 x 12000 A.B^T 53 us in 5 slices (2 tiles on the busiest
// CUs), 68 in 6 (3).  Same box, two runs, against one round at most (and no
// split past half a round): 1500^2 x 16384 165 -> 102 us, 1000^2 x 65536
// 212 -> 121, 704 x 896 x 30000 92 -> 64, 5000 x 512 x 8192 A.B^T 62 -> 50,
// 3000 x 700 x 8192 87 -> 61, 2500 x 640 x 16384 A^T.B^T 107 -> 86, 1100 x
// 1000 x 10000 A^T.B^T 64 -> 50, 1001^2 x 32768 117 -> 97; one loss, 2000 x
// 1000 x 8000 A^T.B 49 -> 52 (4 slices against 2).  1 = no split.
int edge_split_count(int M, int N, int K) {
    if (M % 128 == 0 && N % 128 == 0 && K % 64 == 0) return 1;
    const int64_t cus = ch::num_cus() > 0 ? ch::num_cus() : 1;
    const int64_t tiles = (int64_t)((M + 127) / 128) * ((N + 127) / 128);
    if (tiles > cus) return 1;
    int one = 1;  // within one round
    for (int S = (int)std::min<int64_t>(cus / tiles, K / 512); S >= 2; --S)
        if (K % (8 * S) == 0) {
            one = S;
            break;
        }
    // past one round: the busiest CU's tiles times the slice depth
    auto work = [&](int S) { return (double)((tiles * S + cus - 1) / cus) * ((double)K / S); };
    double least = 0;
    for (int S = 2; S <= K / 2000 && tiles * S <= 4 * cus; ++S)
        if (tiles * S > cus && K % (8 * S) == 0 && (least == 0 || work(S) < least)) least = work(S);
    int past = 1;
    for (int S = 2; S <= K / 2000 && tiles * S <= 4 * cus; ++S)
        if (tiles * S > cus && K % (8 * S) == 0 && work(S) <= 1.1 * least) past = S;
    return std::max(one, past);
}

// Whether K slices of depth kk with these strides go to an aligned kernel
// (128 x 128 tiles and whole k-tiles) or a guarded-edge one, not to the
// general kernel: on that kernel 1000^2 x 65536 ran as two slices in
// 2.36 ms, against 0.20 ms for 1024^2 x 65536 on the tiled kernel.
template <bool TA, bool TB>
bool slices_fit(const uint16_t* a, const uint16_t* b, int M, int N, int kk, const Strides& s) {
    if (!bases_aligned(a, b, s)) return false;
    if (M % 128 == 0 && N % 128 == 0 && kk % 64 == 0 && s.lda % 8 == 0 && s.ldb % 8 == 0) return true;
    return ch::edge_chunks<8>(!TA, M, kk, s.lda, s.padded) && ch::edge_chunks<8>(TB, N, kk, s.ldb, s.padded) &&
           ch::edge_bytes<8, 2>(!TA, M, kk, s.lda) < (1ll << 31) &&
           ch::edge_bytes<8, 2>(TB, N, kk, s.ldb) < (1ll << 31);
}

// One product (C of pitch N; A and B of pitches lda and ldb, so that a band
// of a larger product's rows keeps its operand pitches) as split_count's K
// slices into a scratch buffer, added in order (ch::sum_slices_f32,
// deterministic): the aligned kernels, or on a ragged M, N or K the
// guarded-edge ones (`padded`: the operands are aligned copies,
// ch::edge_chunks).  Each slice's C starts on a 16-byte boundary of the
// buffer.  False when not split.
template <bool TA, bool TB>
bool try_k_split(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int64_t lda, int64_t ldb,
                 bool padded, int32_t* st) {
    if (((uintptr_t)c & 15) != 0) return false;
    int S = edge_split_count(M, N, K);
    if (S <= 1) S = split_count(M, N, K);
    if (S <= 1) return false;
    const int kk = K / S;
    const int64_t n = (int64_t)M * N, n4 = (n + 3) / 4 * 4;
    const Strides sl{lda, ldb, TA ? (int64_t)kk * lda : kk, TB ? kk : (int64_t)kk * ldb, n4, padded};
    if (!slices_fit<TA, TB>(a, b, M, N, kk, sl)) return false;
    float* part = (float*)ch::scratch_try(10, sizeof(float) * (size_t)(S * n4));
    if (!part) return false;
    if (!launch_fast<TA, TB>(a, b, part, M, N, kk, S, sl, st) &&
        !launch_edge<TA, TB>(a, b, part, M, N, kk, S, sl, st) &&
        !launch_pairs_edge<TA, TB>(a, b, part, M, N, kk, S, sl, st))
        *st = launch<TA, TB>(a, b, part, M, N, kk, S, sl);
    if (*st == CLEAVE_HIP_OK) *st = ch::sum_slices_f32(part, c, n, S, n4);
    return true;
}

// Products of at least this many flops (2 M N K per product) that no aligned
// kernel takes run on zero-padded copies (gemm_pad.hpp); smaller ones run
// the general kernel, one launch against the padded route's three (~10 us
// together; measured when it was four).  Measured crossing: ~115^3 (100^3 11.1 us general, 12.1 padded;
// 127 x 129 x 131 14.1 against 12.0).
constexpr double kPadMinFlops = 1u << 22;
// 256 x 256 tiles (8192^3) 0.55 of peak, also from half a round of them;
// 128 x 128 tiles (8320^3) 0.31.
constexpr ch::PadModel kPadModel{0.55, 0.31, true, 0.5};

template <bool TA, bool TB>
int32_t launch_any(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch) {
    int32_t st = CLEAVE_HIP_OK;
    if (launch_fast<TA, TB>(a, b, c, M, N, K, batch, packed<TA, TB>(M, N, K), &st)) return st;
    // one output dimension of at most 32: stream the long operand (gemv.hip);
    // tiny products (under 2^20 flops) stay on the general kernel (one launch)
    if ((M <= 32 || N <= 32) && 2.0 * M * N * K * batch >= (1u << 20))
        return ch::matmul_skinny_bf16(a, b, c, M, N, K, batch, TA, TB);
    if (2.0 * M * N * K * batch >= kPadMinFlops) {
        // The guarded-edge kernels on aligned copies (ch::run_aligned): K
        // slices for one product with few tiles and a long K, else one launch.
        auto edge = [&](const uint16_t* pa, const uint16_t* pb, int64_t lda, int64_t ldb, int64_t sA, int64_t sB,
                        int Kq, int32_t* s) {
            if (batch == 1 && M > 32 && N > 32 && try_k_split<TA, TB>(pa, pb, c, M, N, Kq, lda, ldb, true, s))
                return true;
            const Strides str{lda, ldb, sA, sB, (int64_t)M * N, true};
            return launch_edge<TA, TB>(pa, pb, c, M, N, Kq, batch, str, s) ||
                   launch_pairs_edge<TA, TB>(pa, pb, c, M, N, Kq, batch, str, s);
        };
        // Few tiles and a long K that no slice count divides in whole
        // chunks: K rounded up to a multiple of 2048 in aligned copies of
        // both operands, then the slices.
        if (batch == 1 && M > 32 && N > 32 && K >= 16384 && K % 2048 != 0 && edge_split_count(M, N, K) <= 1 &&
            edge_split_count(M, N, (int)ch::pad_up(K, 2048)) > 1) {
            const ch::AlignPlan kp = ch::align_plan(M, N, K, batch, TA, TB, a, b, 2, 2048);
            if (ch::run_aligned(kp, a, b, M, N, K, batch, TA, TB, edge, &st)) return st;
        }
        if (launch_edge<TA, TB>(a, b, c, M, N, K, batch, packed<TA, TB>(M, N, K), &st)) return st;
        if (launch_pairs_edge<TA, TB>(a, b, c, M, N, K, batch, packed<TA, TB>(M, N, K), &st)) return st;
        // Rows that are not whole 16-byte chunks (an extent that is not a
        // multiple of 8, a misaligned view): the same guarded-edge kernels on
        // aligned copies of those operands, C in place (ch::run_aligned).
        // Against the padded route below, which also pads C and crops it
        // (same box, two runs): 12300^2 x 200 239 against 472 us, 5000 x
        // 5004 x 200 37 against 64, 64 x 700 x 900 x 300 94 against 161,
        // 2048 x 1100 x 256 10.2 against 16.4, 3001 x 3000 x 1000 A^T.B 37
        // against 42; 1500^3 level (28.5 against 28.9).
        const ch::AlignPlan ap = ch::align_plan(M, N, K, batch, TA, TB, a, b, 2);
        if (ch::run_aligned(ap, a, b, M, N, K, batch, TA, TB, edge, &st)) return st;
        const ch::PadPlan p = ch::pad_plan(M, N, K, batch, TA, TB, a, b, 2, ch::num_cus(), kPadModel);
        auto gemm = [batch](const uint16_t* pa, const uint16_t* pb, float* pc, int Mp, int Np, int Kp) {
            int32_t s = CLEAVE_HIP_OK;
            if (batch == 1 && try_k_split<TA, TB>(pa, pb, pc, Mp, Np, Kp, TA ? Mp : Kp, TB ? Kp : Np, false, &s))
                return s;
            if (launch_fast<TA, TB>(pa, pb, pc, Mp, Np, Kp, batch, packed<TA, TB>(Mp, Np, Kp), &s)) return s;
            return launch<TA, TB>(pa, pb, pc, Mp, Np, Kp, batch, packed<TA, TB>(Mp, Np, Kp));
        };
        if (ch::run_padded(p, a, b, c, batch, TA, TB, gemm, &st)) return st;
    }
    return launch<TA, TB>(a, b, c, M, N, K, batch, packed<TA, TB>(M, N, K));
}

// Rough time of an aligned product, in us: rounds of 256 x 256 tiles (0.58
// of the dense peak per tile, as 8192^3 runs) from half a round of them, else
// 0.26 (1024^3 - 2048^3 on 128 x 128 or 64 x 128 tiles, and K slices).
double est_us(int M, int N, int K) {
    const double cus = ch::num_cus() > 0 ? ch::num_cus() : 1, peak = 2516e12;
    const int64_t big = (M % 256 == 0 && N % 256 == 0) ? (int64_t)(M / 256) * (N / 256) : 0;
    if (big * 2 >= cus) return std::ceil(big / cus) * cus * 2.0 * 256 * 256 * K / (peak * 0.58) * 1e6;
    return 2.0 * M * N * K / (peak * 0.26) * 1e6;
}

template <bool TA, bool TB>
int32_t product(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int64_t lda, int64_t ldb,
                int depth);

// More than a round of 256 x 256 tiles ending in a ragged round: the first M1
// rows of C, the whole rounds, run as one product and the remaining rows as
// another, which takes its own kernel (K slices, smaller tiles, or a split of
// its own), when est_us gives the two, plus 4 us for the extra launches, at
// least 3% under the whole.  Deterministic: each part's kernels are chosen by
// its shape alone.  *st is the outcome; false when not split.
template <bool TA, bool TB>
bool try_round_split(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int64_t lda, int64_t ldb,
                     int depth, int32_t* st) {
    const int cus = ch::num_cus() > 0 ? ch::num_cus() : 1;
    if (depth >= 3 || M % 256 || N % 256 || K % 64 || ((uintptr_t)a & 15) || ((uintptr_t)b & 15) ||
        ((uintptr_t)c & 15))
        return false;
    const int64_t T = (int64_t)(M / 256) * (N / 256);
    if (T <= cus) return false;
    const int tn = N / 256, tm = M / 256;
    const int t1 = (int)(T / cus * cus / tn);  // tile-rows of whole rounds
    if (t1 <= 0 || t1 >= tm) return false;
    const int M1 = t1 * 256, M2 = M - M1;
    if (est_us(M1, N, K) + est_us(M2, N, K) + 4.0 >= 0.97 * est_us(M, N, K)) return false;
    // A keeps its full pitch (its rows, or with TA its columns, are offset)
    const uint16_t* a2 = TA ? a + M1 : a + (int64_t)M1 * lda;
    *st = product<TA, TB>(a, b, c, M1, N, K, lda, ldb, depth + 1);
    if (*st == CLEAVE_HIP_OK) *st = product<TA, TB>(a2, b, c + (int64_t)M1 * N, M2, N, K, lda, ldb, depth + 1);
    return true;
}

// One product (C of pitch N): K slices for few tiles and a long K (an output
// dimension of at most 32 streams its long operand instead, in launch_any), a
// split at a ragged round, or the launchers.
template <bool TA, bool TB>
int32_t product(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int64_t lda, int64_t ldb,
                int depth) {
    int32_t st = CLEAVE_HIP_OK;
    if (M > 32 && N > 32 && try_k_split<TA, TB>(a, b, c, M, N, K, lda, ldb, false, &st)) return st;
    if (try_round_split<TA, TB>(a, b, c, M, N, K, lda, ldb, depth, &st)) return st;
    if (lda == (TA ? M : K) && ldb == (TB ? K : N)) return launch_any<TA, TB>(a, b, c, M, N, K, 1);
    // a band of rows of a larger product (aligned: 256-row bands)
    const Strides s{lda, ldb, (int64_t)M * K, (int64_t)K * N, (int64_t)M * N};
    if (launch_fast<TA, TB>(a, b, c, M, N, K, 1, s, &st)) return st;
    return launch<TA, TB>(a, b, c, M, N, K, 1, s);
}

// A batch of packed products with at most half a round of 128 x 128 tiles,
// over all its products, and a long K: S K slices of each product, at least
// 1024 deep, whose tiles fill at least half a round, in one launch of the
// 128 x 128 tiled kernel (its kslices form), then added in order
// (deterministic).  *st is the outcome; false when not split.
template <bool TA, bool TB>
bool try_batched_k_slices(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch,
                          int32_t* st) {
    const int cus = ch::num_cus() > 0 ? ch::num_cus() : 1;
    if (M % 128 || N % 128 || ((uintptr_t)c & 15)) return false;
    const int64_t t = (int64_t)(M / 128) * (N / 128) * batch;
    if (t * 2 > cus) return false;
    int S = 0;
    for (int s = (int)(cus / t); s >= 2; --s)
        if (K % (64 * s) == 0 && K / s >= 1024) {
            if (t * s * 2 >= cus) S = s;
            break;
        }
    if (S == 0) return false;
    const int64_t n = (int64_t)batch * M * N;
    float* part = (float*)ch::scratch_try(10, sizeof(float) * (size_t)S * n);
    if (!part) return false;
    if (!launch_tiled<128, 128, 64, 2, 2, 3, 32, TA, TB>(a, b, part, M, N, K / S, batch * S, packed<TA, TB>(M, N, K),
                                                         st, S))
        return false;
    if (*st == CLEAVE_HIP_OK) *st = ch::sum_slices_f32(part, c, n, S, n);
    return true;
}

int32_t dispatch(const uint16_t* a, const uint16_t* b, float* c, int M, int N, int K, int batch,
                 int ta, int tb) {
    // a dimension of 1: matrix-vector or outer products (gemv.hip)
    if (M == 1 || N == 1 || K == 1) return ch::matmul_vector_bf16(a, b, c, M, N, K, batch, ta, tb);
    if (batch == 1) {
        if (!ta && !tb) return product<false, false>(a, b, c, M, N, K, K, N, 0);
        if (!ta && tb) return product<false, true>(a, b, c, M, N, K, K, K, 0);
        if (ta && !tb) return product<true, false>(a, b, c, M, N, K, M, N, 0);
        return product<true, true>(a, b, c, M, N, K, M, K, 0);
    }
    int32_t st = CLEAVE_HIP_OK;
    bool done;
    if (!ta && !tb) done = try_batched_k_slices<false, false>(a, b, c, M, N, K, batch, &st);
    else if (!ta && tb) done = try_batched_k_slices<false, true>(a, b, c, M, N, K, batch, &st);
    else if (ta && !tb) done = try_batched_k_slices<true, false>(a, b, c, M, N, K, batch, &st);
    else done = try_batched_k_slices<true, true>(a, b, c, M, N, K, batch, &st);
    if (done) return st;
    if (!ta && !tb) return launch_any<false, false>(a, b, c, M, N, K, batch);
    if (!ta && tb) return launch_any<false, true>(a, b, c, M, N, K, batch);
    if (ta && !tb) return launch_any<true, false>(a, b, c, M, N, K, batch);
    return launch_any<true, true>(a, b, c, M, N, K, batch);
}

}  // namespace

extern "C" {

int32_t cleave_hip_matmul_bf16(const uint16_t* a, int64_t alen, const uint16_t* b, int64_t blen,
                               float* c, int64_t clen, int32_t M, int32_t N, int32_t K,
                               int32_t trans_a, int32_t trans_b) {
    CH_REQUIRE(M > 0 && N > 0 && K > 0, "cleave_hip_matmul_bf16: dims must be positive (M=%d N=%d K=%d)", M, N, K);
    CH_REQUIRE((trans_a == 0 || trans_a == 1) && (trans_b == 0 || trans_b == 1),
               "cleave_hip_matmul_bf16: trans flags must be 0 or 1");
    CH_REQUIRE(alen == (int64_t)M * K, "cleave_hip_matmul_bf16: alen %lld != M*K %lld", (long long)alen, (long long)M * K);
    CH_REQUIRE(blen == (int64_t)K * N, "cleave_hip_matmul_bf16: blen %lld != K*N %lld", (long long)blen, (long long)K * N);
    CH_REQUIRE(clen == (int64_t)M * N, "cleave_hip_matmul_bf16: clen %lld != M*N %lld", (long long)clen, (long long)M * N);
    CH_REQUIRE(a && b && c, "cleave_hip_matmul_bf16: null buffer");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_matmul_bf16", a, alen * 2);
    CH_DEVICE("cleave_hip_matmul_bf16", b, blen * 2);
    CH_DEVICE("cleave_hip_matmul_bf16", c, clen * 4);
    return dispatch(a, b, c, M, N, K, 1, trans_a, trans_b);
}

int32_t cleave_hip_matmul_batched_bf16(const uint16_t* a, int64_t alen, const uint16_t* b,
                                       int64_t blen, float* c, int64_t clen, int32_t batch,
                                       int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                       int32_t trans_b) {
    CH_REQUIRE(batch > 0 && batch <= 65535 && M > 0 && N > 0 && K > 0,
               "cleave_hip_matmul_batched_bf16: bad dims (batch=%d M=%d N=%d K=%d)", batch, M, N, K);
    CH_REQUIRE((trans_a == 0 || trans_a == 1) && (trans_b == 0 || trans_b == 1),
               "cleave_hip_matmul_batched_bf16: trans flags must be 0 or 1");
    const int64_t na = ch::count3(batch, M, K), nb = ch::count3(batch, K, N), nc = ch::count3(batch, M, N);
    CH_REQUIRE(na >= 0 && nb >= 0 && nc >= 0 && alen == na && blen == nb && clen == nc,
               "cleave_hip_matmul_batched_bf16: lengths do not match batch*M*K, batch*K*N, batch*M*N");
    CH_REQUIRE(a && b && c, "cleave_hip_matmul_batched_bf16: null buffer");
    CH_INIT_OR_RETURN();
    CH_DEVICE("cleave_hip_matmul_batched_bf16", a, alen * 2);
    CH_DEVICE("cleave_hip_matmul_batched_bf16", b, blen * 2);
    CH_DEVICE("cleave_hip_matmul_batched_bf16", c, clen * 4);
    return dispatch(a, b, c, M, N, K, batch, trans_a, trans_b);
}

}  // extern "C"
