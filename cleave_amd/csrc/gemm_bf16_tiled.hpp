// gemm_bf16_tiled.hpp -- the large-tile bf16-in / f32-accumulate GEMM kernel
// for gfx950 (shapes that divide the block tile).
//
// One workgroup computes a BM x BN block of C with WM x WN waves; each wave
// owns a (BM/WM) x (BN/WN) block of 32 x 32 accumulators (v16f per MFMA tile).
// K is walked in BK-deep tiles through a STAGES-deep ring of LDS buffers that
// are filled by global_load_lds (see gemm_tiles.hpp for the layouts):
//
//   prologue: issue tiles 0 .. STAGES-2, wait for tile 0, s_barrier,
//             issue tile STAGES-1, read the fragments of k-step 0
//   for kt, for each of the BK/16 k-steps:
//             read the next k-step's fragments (double-buffered registers)
//             FM x FN MFMAs on this k-step's fragments
//   where the last k-step of tile kt first waits for tile kt+1's copies and
//   for its own LDS reads, passes an s_barrier, issues tile kt+STAGES into
//   tile kt's buffer and reads tile kt+1's first fragments -- so the
//   fragment pipeline never drains at a tile boundary.
//
// The waits are s_waitcnt vmcnt(copies issued after the awaited tile) and the
// barrier is a bare s_barrier, so copies of later tiles stay in flight across
// it.  Both are inline asm with a memory clobber, which keeps the compiler
// from moving LDS reads across them.
//
// EDGE = true (32 x 32 MFMAs) takes any M, N and K >= 1 (tiles_m, tiles_n
// rounded up): the copies become buffer loads that zero-fill what lies
// outside the operand (EdgeCopy, gemm_tiles.hpp) and the stores are masked,
// so a ragged product needs no padded copies and no crop.
#pragma once

#include "gemm_common.hpp"
#include "gemm_tiles.hpp"

namespace ch {

// MI selects the matrix instruction: 32 -> v_mfma_f32_32x32x16_bf16 (32 x 32
// accumulator tiles, 16-deep k-steps), 16 -> v_mfma_f32_16x16x32_bf16 (16 x 16
// tiles, 32-deep k-steps).  On N(0, 0.02^2) data the 16 x 16 form sustains
// ~12% more throughput: the chip is power-limited there, not issue-limited.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, bool AKC, bool BKC, int MI = 32>
struct Bf16Tiled {
    static_assert(MI == 32 || MI == 16, "MFMA shape");
    static constexpr int NW = WM * WN, THREADS = 64 * NW;
    static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / MI, FN = TN / MI;
    static constexpr int KSTEP = MI == 32 ? 16 : 32;  // k per MFMA
    static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES, LDS_BYTES = STAGES * STAGE_BYTES;
    // global_load_lds instructions per wave per k-tile
    static constexpr int LPW = STAGE_BYTES / 1024 / NW;
    static_assert(TM % MI == 0 && TN % MI == 0 && BK % (2 * KSTEP) == 0, "tile shape");
    static_assert(STAGES >= 2 && LPW * (STAGES - 2) < 64, "pipeline depth");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS per workgroup");

    // Shapes this kernel takes without bounds checks.  The copies address an
    // operand with 32-bit byte offsets from a per-tile, per-k-tile scalar
    // base, so the span those offsets reach must stay under 4 GiB.
    static bool fits(int M, int N, int K, int64_t lda, int64_t ldb) {
        const bool dims = M % BM == 0 && N % BN == 0 && K % BK == 0 && lda % 8 == 0 && ldb % 8 == 0;
        // that span: BM (BN) rows of a k-contiguous operand, BK k-rows of an
        // m/n-contiguous one
        const uint64_t a_span = (AKC ? (uint64_t)BM : (uint64_t)BK + 1) * (uint64_t)lda * 2;
        const uint64_t b_span = (BKC ? (uint64_t)BN : (uint64_t)BK + 1) * (uint64_t)ldb * 2;
        return dims && a_span < (1ull << 32) && b_span < (1ull << 32);
    }
    // Bytes from an operand's base to the end of its last chunk (ch::edge_bytes).
    static __host__ __device__ int64_t a_bytes(int M, int K, int64_t lda) {
        return edge_bytes<8, 2>(AKC, M, K, lda);
    }
    static __host__ __device__ int64_t b_bytes(int N, int K, int64_t ldb) {
        return edge_bytes<8, 2>(BKC, N, K, ldb);
    }
    // Shapes the EDGE form takes: whole 16-byte chunks (8 elements) along
    // each operand's pitch and along K, an m/n extent in whole chunks unless
    // `padded` (ch::edge_chunks), and operands under 2 GiB.
    static bool fits_edge(int M, int N, int K, int64_t lda, int64_t ldb, bool padded = false) {
        const bool chunks = edge_chunks<8>(AKC, M, K, lda, padded) && edge_chunks<8>(BKC, N, K, ldb, padded);
        return MI == 32 && M >= 1 && N >= 1 && K >= 1 && chunks && a_bytes(M, K, lda) < (1ll << 31) &&
               b_bytes(N, K, ldb) < (1ll << 31);
    }
};

// `batch` products of M x N x K, product z at A + z strideA, B + z strideB,
// C + z strideC.  With kslices > 1 (batch a multiple of it) the products are
// the K slices of batch / kslices products of depth K * kslices: z = s nb + b
// (nb = batch / kslices) is slice s of product b, at A + b strideA plus s K
// columns (k-contiguous A) or s K rows of A (likewise B), and C + z strideC.
// NTC: C stored non-temporally, for C rows of whole 128-byte lines (the
// launchers' nt_c).
template <int BM, int BN, int BK, int WM, int WN, int STAGES, bool AKC, bool BKC, int MI = 32, bool EDGE = false,
          bool NTC = false>
__global__ __launch_bounds__(64 * WM * WN) void gemm_bf16_tiled_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, float* __restrict__ C, int M,
    int N, int K, int64_t lda, int64_t ldb, int64_t strideA, int64_t strideB, int64_t strideC,
    int tiles_m, int tiles_n, int batch, int kslices) {
    using namespace ch::tiles;
    using P = Bf16Tiled<BM, BN, BK, WM, WN, STAGES, AKC, BKC, MI>;
    typedef float vacc __attribute__((ext_vector_type(MI == 32 ? 16 : 4)));
    constexpr int FM = P::FM, FN = P::FN, NW = P::NW;
    __shared__ __attribute__((aligned(1024))) char smem[P::LDS_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: keeps LDS/DMA bases scalar
    const int wm = wave / WN, wn = wave % WN;
    int bt, tm, tn;  // product (batch entry or K-slice) and tile of this workgroup
    ch::block_coords(blockIdx.x, tiles_m, tiles_n, batch, bt, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    if (kslices > 1) {
        const int nb = batch / kslices, sl = bt / nb, pb = bt - sl * nb;
        A += (int64_t)pb * strideA + (AKC ? (int64_t)sl * K : (int64_t)sl * K * lda);
        B += (int64_t)pb * strideB + (BKC ? (int64_t)sl * K : (int64_t)sl * K * ldb);
    } else {
        A += (int64_t)bt * strideA;
        B += (int64_t)bt * strideB;
    }
    C += (int64_t)bt * strideC;

    static_assert(!EDGE || (MI == 32), "the EDGE form stores 32 x 32 accumulators");
    const uint32_t lds0 = lds_addr(smem);
    // aligned shapes: scalar tile bases and 32-bit lane offsets
    TileCopy<AKC, BM, BK, NW> copy_a;
    TileCopy<BKC, BN, BK, NW> copy_b;
    const char* a_src = nullptr;
    const char* b_src = nullptr;
    int64_t step_a = 0, step_b = 0;
    // EDGE: buffer resources over the operands, masked lane offsets
    EdgeCopy<AKC, BM, BK, NW> edge_a;
    EdgeCopy<BKC, BN, BK, NW> edge_b;
    v4i rsrc_a{}, rsrc_b{};
    if constexpr (EDGE) {
        edge_a.init(lda, m0, M, wave, lane);
        edge_b.init(ldb, n0, N, wave, lane);
        rsrc_a = buffer_rsrc(A, (uint32_t)P::a_bytes(M, K, lda));
        rsrc_b = buffer_rsrc(B, (uint32_t)P::b_bytes(N, K, ldb));
    } else {
        copy_a.init(lda, m0, wave, lane);
        copy_b.init(ldb, n0, wave, lane);
        step_a = copy_a.kstep(lda);
        step_b = copy_b.kstep(ldb);
        a_src = reinterpret_cast<const char*>(A) + copy_a.base_offset(lda, m0);
        b_src = reinterpret_cast<const char*>(B) + copy_b.base_offset(ldb, n0);
    }
    auto issue = [&](int kt, int stage) {
        const uint32_t dst = lds0 + (uint32_t)(stage * P::STAGE_BYTES);
        if constexpr (EDGE) {
            edge_a.issue(rsrc_a, kt, K, (uint32_t)kt * edge_a.kstep(lda), dst, wave);
            edge_b.issue(rsrc_b, kt, K, (uint32_t)kt * edge_b.kstep(ldb), dst + P::A_BYTES, wave);
        } else {
            copy_a.issue(a_src + kt * step_a, dst, wave);
            copy_b.issue(b_src + kt * step_b, dst + P::A_BYTES, wave);
        }
    };

    vacc acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = vacc{};

    // Operand fragments of two consecutive k-steps: step s+1 is read while
    // step s's MFMAs run, also across the k-tile boundary.
    v8bf fa[2][FM], fb[2][FN];
    auto read_step = [&](int buf, const char* tile, int kk) {
        const char* ta = tile;
        const char* tb = tile + P::A_BYTES;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            if constexpr (MI == 32) fa[buf][i] = read_frag<AKC, BM, BK>(ta, wm * P::TM + i * 32, kk, lane);
            else fa[buf][i] = read_frag16<AKC, BM, BK>(ta, wm * P::TM + i * 16, kk, lane);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            if constexpr (MI == 32) fb[buf][j] = read_frag<BKC, BN, BK>(tb, wn * P::TN + j * 32, kk, lane);
            else fb[buf][j] = read_frag16<BKC, BN, BK>(tb, wn * P::TN + j * 16, kk, lane);
        }
    };

    constexpr int KS = BK / P::KSTEP;  // k-steps per k-tile
    static_assert(KS % 2 == 0, "fragment double-buffer parity assumes an even k-step count");
    const int nk = EDGE ? (K + BK - 1) / BK : K / BK;
    // Prologue: tiles 0 .. STAGES-2 in flight; wait for tile 0; then tile
    // STAGES-1 goes into the last free buffer.
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nk) issue(s, s);
    if (nk >= STAGES - 1) {
        constexpr int n = P::LPW * (STAGES - 2);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    asm volatile("s_barrier" ::: "memory");
    if (STAGES - 1 < nk) issue(STAGES - 1, STAGES - 1);
    read_step(0, smem, 0);

    // ds_read instructions per k-step (a transposed fragment takes two).
    constexpr int NR = FM * (AKC ? 1 : 2) + FN * (BKC ? 1 : 2);
    auto mfma_step = [&](int cur) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if constexpr (MI == 32)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cur][i], fb[cur][j], acc[i][j], 0, 0, 0);
                else
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[cur][i], fb[cur][j], acc[i][j], 0, 0, 0);
            }
    };

    for (int kt = 0; kt < nk; ++kt) {
        const char* tile = smem + (kt % STAGES) * P::STAGE_BYTES;
        // k-steps 0 .. KS-2: next step's reads spread between this step's MFMAs
#pragma unroll
        for (int kk = 0; kk + 1 < KS; ++kk) {
            read_step((kk & 1) ^ 1, tile, kk + 1);
            mfma_step(kk & 1);
        }
#pragma unroll
        for (int g = 0; g < (KS - 1) * FM * FN; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            if (g % (FM * FN) < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one ds_read
        }
        // Last k-step.  Tile kt+1 must have landed (tiles kt+2 .. kt+STAGES-1
        // may stay in flight) and every wave must be done reading tile kt
        // before its buffer takes tile kt+STAGES.
        if (kt + 1 < nk) {
            if (kt + STAGES - 1 < nk) {
                constexpr int n = P::LPW * (STAGES - 2);
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(n) : "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            }
            asm volatile("s_barrier" ::: "memory");
            read_step(0, smem + ((kt + 1) % STAGES) * P::STAGE_BYTES, 0);
            if (kt + STAGES < nk) issue(kt + STAGES, kt % STAGES);
        }
        mfma_step((KS - 1) & 1);
    }

    // 32 x 32 accumulator layout: lane holds column l%32, rows
    // 8*(v/4) + 4*(l/32) + v%4, so a store already covers whole 128-byte rows.
    if constexpr (MI == 16) {
        store_acc16_lines<FM, FN, NTC>(C, N, m0 + wm * P::TM, n0 + wn * P::TN, acc, lane);
    } else {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = m0 + wm * P::TM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                    const int c = n0 + wn * P::TN + j * 32 + (lane & 31);
                    if (!EDGE || (r < M && c < N)) {
                        if constexpr (NTC) __builtin_nontemporal_store(acc[i][j][v], C + (int64_t)r * N + c);
                        else C[(int64_t)r * N + c] = acc[i][j][v];
                    }
                }
    }
}

}  // namespace ch
