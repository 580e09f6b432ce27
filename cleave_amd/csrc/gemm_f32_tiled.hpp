// gemm_f32_tiled.hpp -- large-tile fp32 GEMM kernel on v_mfma_f32_32x32x2f32
// for gfx950 (shapes that divide the block tile).
//
// Same pipeline as gemm_bf16_tiled.hpp (LDS ring filled by global_load_lds,
// operand fragments double-buffered across the k-tile barrier, MFMA/ds_read
// interleave pinned with sched_group_barrier); see gemm_tiles.hpp for the LDS
// layouts.  The f32 MFMA sums two k values per instruction, one per
// half-wave.  Over an 8-deep k-block, half-wave h takes k = 4h + s at step s
// (A and B agree, so all 8 terms are summed), which lets a k-contiguous
// operand feed four MFMAs from one ds_read_b128; an m/n-contiguous operand is
// read with four conflict-free ds_read_b32.
//
// EDGE = true takes any M, N and K >= 1 (tiles_m, tiles_n rounded up): the
// copies become buffer loads that zero-fill what lies outside the operand
// (EdgeCopy, gemm_tiles.hpp) and the stores are masked, so a ragged product
// needs no padded copies of its operands and no crop of its result.
#pragma once

#include "gemm_common.hpp"
#include "gemm_tiles.hpp"

namespace ch {

template <int BM, int BN, int BK, int WM, int WN, int STAGES, bool AKC, bool BKC>
struct F32Tiled {
    static constexpr int NW = WM * WN, THREADS = 64 * NW;
    static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    static constexpr int A_BYTES = BM * BK * 4, B_BYTES = BN * BK * 4;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES, LDS_BYTES = STAGES * STAGE_BYTES;
    static constexpr int LPW = (A_BYTES + B_BYTES) / 1024 / NW;  // copy instructions per wave per k-tile
    static_assert(TM % 32 == 0 && TN % 32 == 0 && BK % 16 == 0, "tile shape");
    static_assert(STAGES >= 2 && LPW * (STAGES - 2) < 64, "pipeline depth");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS per workgroup");

    // Shapes this kernel takes without bounds checks.  The copies address an
    // operand with 32-bit byte offsets from a per-tile, per-k-tile scalar
    // base, so the span those offsets reach must stay under 4 GiB.
    static bool fits(int M, int N, int K, int64_t lda, int64_t ldb) {
        const bool dims = M % BM == 0 && N % BN == 0 && K % BK == 0 && lda % 8 == 0 && ldb % 8 == 0;
        // that span: BM (BN) rows of a k-contiguous operand, BK k-rows of an
        // m/n-contiguous one
        const uint64_t a_span = (AKC ? (uint64_t)BM : (uint64_t)BK + 1) * (uint64_t)lda * 4;
        const uint64_t b_span = (BKC ? (uint64_t)BN : (uint64_t)BK + 1) * (uint64_t)ldb * 4;
        return dims && a_span < (1ull << 32) && b_span < (1ull << 32);
    }
    // Bytes from an operand's base to the end of its last chunk (ch::edge_bytes).
    static __host__ __device__ int64_t a_bytes(int M, int K, int64_t lda) {
        return edge_bytes<4, 4>(AKC, M, K, lda);
    }
    static __host__ __device__ int64_t b_bytes(int N, int K, int64_t ldb) {
        return edge_bytes<4, 4>(BKC, N, K, ldb);
    }
    // Shapes the EDGE form takes: whole 16-byte chunks (4 elements) along
    // each operand's pitch and along K, an m/n extent in whole chunks unless
    // `padded` (ch::edge_chunks), and operands under 2 GiB.
    static bool fits_edge(int M, int N, int K, int64_t lda, int64_t ldb, bool padded = false) {
        const bool chunks = edge_chunks<4>(AKC, M, K, lda, padded) && edge_chunks<4>(BKC, N, K, ldb, padded);
        return M >= 1 && N >= 1 && K >= 1 && chunks && a_bytes(M, K, lda) < (1ll << 31) &&
               b_bytes(N, K, ldb) < (1ll << 31);
    }
};

template <int BM, int BN, int BK, int WM, int WN, int STAGES, bool AKC, bool BKC, bool EDGE = false>
__global__ __launch_bounds__(64 * WM * WN) void gemm_f32_tiled_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N,
    int K, int64_t lda, int64_t ldb, int64_t strideA, int64_t strideB, int64_t strideC, int tiles_m,
    int tiles_n, int batch) {
    using namespace ch::tiles;
    using P = F32Tiled<BM, BN, BK, WM, WN, STAGES, AKC, BKC>;
    constexpr int FM = P::FM, FN = P::FN, NW = P::NW;
    __shared__ __attribute__((aligned(1024))) char smem[P::LDS_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    int bt, tm, tn;  // product (batch entry or K-slice) and tile of this workgroup
    ch::block_coords(blockIdx.x, tiles_m, tiles_n, batch, bt, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    A += (int64_t)bt * strideA;
    B += (int64_t)bt * strideB;
    C += (int64_t)bt * strideC;

    const uint32_t lds0 = lds_addr(smem);
    // aligned shapes: scalar tile bases and 32-bit lane offsets
    TileCopy<AKC, BM, BK, NW, 4> copy_a;
    TileCopy<BKC, BN, BK, NW, 4> copy_b;
    const char* a_src = nullptr;
    const char* b_src = nullptr;
    int64_t step_a = 0, step_b = 0;
    // EDGE: buffer resources over the operands, masked lane offsets
    EdgeCopy<AKC, BM, BK, NW, 4> edge_a;
    EdgeCopy<BKC, BN, BK, NW, 4> edge_b;
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

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16f{};

    v4f fa[2][FM], fb[2][FN];
    auto read_block = [&](int buf, const char* tile, int kb) {
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[buf][i] = read_frag_f32<AKC, BM, BK>(tile, wm * P::TM + i * 32, kb, lane);
#pragma unroll
        for (int j = 0; j < FN; ++j)
            fb[buf][j] = read_frag_f32<BKC, BN, BK>(tile + P::A_BYTES, wn * P::TN + j * 32, kb, lane);
    };
    auto mfma_block = [&](int cur) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[cur][i][s], fb[cur][j][s], acc[i][j], 0, 0, 0);
    };

    constexpr int KB = BK / 8;  // 8-deep k-blocks per k-tile
    static_assert(KB % 2 == 0, "fragment double-buffer parity assumes an even k-block count");
    constexpr int NR = FM * (AKC ? 1 : 4) + FN * (BKC ? 1 : 4);  // ds_reads per k-block
    constexpr int NM = 4 * FM * FN;                              // MFMAs per k-block
    const int nk = EDGE ? (K + BK - 1) / BK : K / BK;

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
    read_block(0, smem, 0);

    for (int kt = 0; kt < nk; ++kt) {
        const char* tile = smem + (kt % STAGES) * P::STAGE_BYTES;
#pragma unroll
        for (int kb = 0; kb + 1 < KB; ++kb) {
            read_block((kb & 1) ^ 1, tile, kb + 1);
            mfma_block(kb & 1);
        }
#pragma unroll
        for (int g = 0; g < (KB - 1) * NM; ++g) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (g % NM < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if (kt + 1 < nk) {
            if (kt + STAGES - 1 < nk) {
                constexpr int n = P::LPW * (STAGES - 2);
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(n) : "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            }
            asm volatile("s_barrier" ::: "memory");
            read_block(0, smem + ((kt + 1) % STAGES) * P::STAGE_BYTES, 0);
            if (kt + STAGES < nk) issue(kt + STAGES, kt % STAGES);
        }
        mfma_block((KB - 1) & 1);
    }

    const int half = lane >> 5, col = lane & 31;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = m0 + wm * P::TM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                const int c = n0 + wn * P::TN + j * 32 + col;
                if (!EDGE || (r < M && c < N)) C[(int64_t)r * N + c] = acc[i][j][v];
            }
}

}  // namespace ch
