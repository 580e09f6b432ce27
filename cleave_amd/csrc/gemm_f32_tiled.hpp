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
#pragma once

#include "gemm_common.hpp"
#include "gemm_tiles.hpp"

namespace ch {

// Fusions for the two GEMMs of the MLP step (mlp.hip, MlpFuse in
// gemm_common.hpp); plain GEMMs pass {}.
//   MODE 1 (H = sigmoid(X W1)): the epilogue applies the sigmoid before
//     storing and writes zpart[(tn*WN + wn)*M + row] = sum over this wave's
//     columns of H[row][col] * w2[col] (a partial of z2 = H W2).
//   MODE 2 (dW1 = X^T d1, split-K over the batch): B is H, and each operand
//     value h of column n at batch row k becomes d1 = (d2[k] w2[n]) h (1 - h)
//     as the MFMA consumes it.  The same values give dW2[n] = sum_k h d2[k]:
//     each k-block's contribution is taken by exactly one wave -- M-tile tm
//     takes the k-tiles with kt % tiles_m == tm and, within them, row-half wm
//     the k-block kb == wm -- so every workgroup carries an equal share, and
//     each wave writes its partial to
//     dw2part[((split * tiles_m + tm) * WM + wm) * N + n].  d2 reaches LDS
//     with the k-tile.
template <int BM, int BN, int BK, int WM, int WN, int STAGES, bool AKC, bool BKC, int MODE = 0>
struct F32Tiled {
    static constexpr int NW = WM * WN, THREADS = 64 * NW;
    static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    static constexpr int A_BYTES = BM * BK * 4, B_BYTES = BN * BK * 4;
    static constexpr int AUX_BYTES = MODE == 2 ? 1024 : 0;  // d2 slice of the k-tile
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES + AUX_BYTES, LDS_BYTES = STAGES * STAGE_BYTES;
    // copy instructions per wave per k-tile (MODE 2 adds the d2 slice)
    static constexpr int LPW = (A_BYTES + B_BYTES) / 1024 / NW + (MODE == 2 ? 1 : 0);
    static_assert(TM % 32 == 0 && TN % 32 == 0 && BK % 16 == 0, "tile shape");
    static_assert(MODE != 2 || (!BKC && BK <= 64), "MODE 2 transforms an m/n-contiguous B");
    static_assert(STAGES >= 2 && LPW * (STAGES - 2) < 64, "pipeline depth");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS per workgroup");

    // Shapes this kernel takes without bounds checks.  The copies address an
    // operand with 32-bit byte offsets from a per-k-tile scalar base, so the
    // addressed span of each operand must stay under 4 GiB.
    static bool fits(int M, int N, int K, int64_t lda, int64_t ldb) {
        const bool dims = M % BM == 0 && N % BN == 0 && K % BK == 0 && lda % 8 == 0 && ldb % 8 == 0;
        const uint64_t a_span = (AKC ? (uint64_t)M : (uint64_t)BK + 1) * (uint64_t)lda * 4;
        const uint64_t b_span = (BKC ? (uint64_t)N : (uint64_t)BK + 1) * (uint64_t)ldb * 4;
        return dims && a_span < (1ull << 32) && b_span < (1ull << 32);
    }};

template <int BM, int BN, int BK, int WM, int WN, int STAGES, bool AKC, bool BKC, int MODE = 0>
__global__ __launch_bounds__(64 * WM * WN) void gemm_f32_tiled_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N,
    int K, int64_t lda, int64_t ldb, int64_t strideA, int64_t strideB, int64_t strideC, int tiles_m,
    int tiles_n, int batch, MlpFuse fuse) {
    using namespace ch::tiles;
    using P = F32Tiled<BM, BN, BK, WM, WN, STAGES, AKC, BKC, MODE>;
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

    TileCopy<AKC, BM, BK, NW, 4> copy_a;
    TileCopy<BKC, BN, BK, NW, 4> copy_b;
    copy_a.init(lda, m0, wave, lane);
    copy_b.init(ldb, n0, wave, lane);
    const int64_t step_a = copy_a.kstep(lda), step_b = copy_b.kstep(ldb);
    const uint32_t lds0 = lds_addr(smem);
    // MODE 2: this split's d2 slice starts at batch row bt * K.
    const float* d2 = MODE == 2 ? fuse.d2 + (int64_t)bt * K : nullptr;
    auto issue = [&](int kt, int stage) {
        const uint32_t dst = lds0 + (uint32_t)(stage * P::STAGE_BYTES);
        copy_a.issue(reinterpret_cast<const char*>(A) + kt * step_a, dst, wave);
        copy_b.issue(reinterpret_cast<const char*>(B) + kt * step_b, dst + P::A_BYTES, wave);
        if constexpr (MODE == 2) {
            // every wave copies the BK d2 values (BK/4 lanes x 16 bytes), so
            // each wave's vmcnt accounting stays uniform
            if (lane < BK / 4)
                dma16(d2 + (int64_t)kt * BK, (uint32_t)(lane * 16), dst + P::A_BYTES + P::B_BYTES);
        }
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16f{};

    v4f fa[2][FM], fb[2][FN];
    v4f d2v[2];               // MODE 2: d2 at this lane's 4 k of the k-block
    float w2c[FN];            // MODE 2: w2 at this lane's column of fragment j
    v4f dw2acc[FN];           // MODE 2: partial dW2 of that column
    static_assert(MODE != 2 || (BK / 8) % WM == 0, "each row-half wave takes whole k-blocks of a k-tile");
    // MODE 2: does this wave accumulate dW2 for k-block kb of k-tile kt?
    auto dw2_mine = [&](int kt, int kb) { return (kt % tiles_m) == tm && (kb % WM) == wm; };
    if constexpr (MODE == 2) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            w2c[j] = fuse.w2[n0 + wn * P::TN + j * 32 + (lane & 31)];
            dw2acc[j] = v4f{};
        }
    }
    auto read_block = [&](int buf, const char* tile, int kb) {
        if constexpr (MODE == 2)
            d2v[buf] = *reinterpret_cast<const v4f*>(tile + P::A_BYTES + P::B_BYTES + (8 * kb + 4 * (lane >> 5)) * 4);
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[buf][i] = read_frag_f32<AKC, BM, BK>(tile, wm * P::TM + i * 32, kb, lane);
#pragma unroll
        for (int j = 0; j < FN; ++j)
            fb[buf][j] = read_frag_f32<BKC, BN, BK>(tile + P::A_BYTES, wn * P::TN + j * 32, kb, lane);
    };
    // MODE 2: d1 = (d2[k] w2[n]) h (1 - h), the order of the reference step.
    // Applied to a k-block's fragments right after the previous block's MFMAs
    // are issued, so this VALU work overlaps the matrix core.
    auto transform = [&](int buf, bool mine) {
        if constexpr (MODE == 2) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const v4f h = fb[buf][j];
                if (mine) dw2acc[j] += h * d2v[buf];
#pragma unroll
                for (int s = 0; s < 4; ++s) fb[buf][j][s] = (d2v[buf][s] * w2c[j]) * h[s] * (1.0f - h[s]);
            }
        }
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
    const int nk = K / BK;

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
    transform(0, dw2_mine(0, 0));

    for (int kt = 0; kt < nk; ++kt) {
        const char* tile = smem + (kt % STAGES) * P::STAGE_BYTES;
#pragma unroll
        for (int kb = 0; kb + 1 < KB; ++kb) {
            read_block((kb & 1) ^ 1, tile, kb + 1);
            mfma_block(kb & 1);
            transform((kb & 1) ^ 1, dw2_mine(kt, kb + 1));
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
        if (kt + 1 < nk) transform(0, dw2_mine(kt + 1, 0));
    }

    const int half = lane >> 5, col = lane & 31;
    if constexpr (MODE == 1) {
        // H = sigmoid(acc) = 1 / (1 + exp(-acc)) with the hardware exp2 and
        // reciprocal (about 1 ulp each; the IEEE expf + division would cost
        // ~30 VALU ops per element with the matrix core idle), and per row the
        // sum of H * w2 over this wave's columns: lanes of a half-wave hold
        // the 32 columns of the same rows.
        float w2j[FN];
#pragma unroll
        for (int j = 0; j < FN; ++j) w2j[j] = fuse.w2[n0 + wn * P::TN + j * 32 + col];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            float zs[16];
#pragma unroll
            for (int v = 0; v < 16; ++v) zs[v] = 0.0f;
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float e = __builtin_amdgcn_exp2f(-acc[i][j][v] * 1.4426950408889634f);
                    const float h = __builtin_amdgcn_rcpf(1.0f + e);
                    acc[i][j][v] = h;
                    zs[v] += h * w2j[j];
                }
#pragma unroll
            for (int v = 0; v < 16; ++v)
#pragma unroll
                for (int o = 16; o > 0; o >>= 1) zs[v] += __shfl_xor(zs[v], o);
            if (col == 0) {
                float* zp = fuse.zpart + (int64_t)(tn * WN + wn) * M;
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    zp[m0 + wm * P::TM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3)] = zs[v];
            }
        }
    }
    if constexpr (MODE == 2) {
        // every wave writes its partial (zero when it took no k-block)
        float* dst = fuse.dw2part + ((int64_t)(bt * tiles_m + tm) * WM + wm) * N + n0 + wn * P::TN + col;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            float v = (dw2acc[j][0] + dw2acc[j][1]) + (dw2acc[j][2] + dw2acc[j][3]);
            v += __shfl_xor(v, 32);
            if (half == 0) dst[j * 32] = v;
        }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = m0 + wm * P::TM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                const int c = n0 + wn * P::TN + j * 32 + col;
                C[(int64_t)r * N + c] = acc[i][j][v];
            }
}

}  // namespace ch
