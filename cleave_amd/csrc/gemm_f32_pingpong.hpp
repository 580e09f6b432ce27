// gemm_f32_pingpong.hpp -- f32 GEMM on the ping-pong schedule of
// gemm_pingpong.hpp (gfx950, v_mfma_f32_32x32x2f32, 256 x 256 x 16 tiles,
// or 128 x 128 x 16 for products with fewer 256 x 256 tiles than CUs).
//
// Eight waves; each owns a 128 x 64 block of C (4 x 2 tiles of 32 x 32), or
// 64 x 32 on 128 x 128 tiles.  Waves 0-3 (group 0, the upper half of the
// tile's rows) and 4-7 (group 1, the lower half) sit one per SIMD.  A C phase
// is the k-tile's 64 MFMAs (two 8-deep k-blocks of four k=2 steps), 4096
// matrix-core cycles (16 MFMAs on 128 x 128 tiles), so the two barriers per
// k-tile cost little next to it; the single-barrier schedule of
// gemm_f32_tiled.hpp stops both waves of a SIMD at every k-tile (2048^3:
// 131 us there, 118 us here on 128 x 128 tiles).
//
// Both operands sit in LDS k-major, whatever their layout in global memory,
// and every fragment is read with ds_read2st64_b32 (two k-rows, one float
// per lane).  Measured at 4096^3 with the k-contiguous operand kept
// k-contiguous in LDS and read with ds_read_b128, the M phase cost 0.911 of
// peak against 0.962 for the k-major form; LDS writes in the M phase cost
// nothing measurable.  So the operands move in two ways:
//   m/n-contiguous in global memory (A^T stored K x M, B stored K x N):
//     global_load_lds straight into the k-major tile;
//   k-contiguous (A stored M x K, B^T stored N x K): 16 bytes per lane
//     (4 k of one row) into registers one k-tile ahead, then written to the
//     k-major tile with ds_write2st64_b32 ("staged").
// LDS holds each operand as [16 k-rows][4 stages][256 floats] (64 KiB; A at
// 0, B at 64 KiB): one k-row of one stage is the 1 KiB a copy instruction
// writes, and every fragment, k-row and stage of an operand is one
// loop-invariant register plus an immediate offset below 64 KiB.  128 x 128
// tiles keep [6 stages][16 k-rows][128 floats] (48 KiB per operand; a copy
// instruction writes two k-rows; 96 KiB in all, so one workgroup per CU:
// with four stages two shared a CU and three full rounds of tiles ran 417
// against 350 us).  So the M
// phase issues no VALU instruction; the accumulators live in AGPRs.
// Within a 1 KiB row, 16-byte chunk c of k-row kr sits in slot pp_slot(kr, c)
// = c ^ 8*bit2(kr) ^ 4*bit3(kr).  Bit 2 puts the two half-waves of a fragment
// read (k-rows kr and kr + 4, the same 32 columns) in opposite bank halves;
// bit 3 moves the k-rows 4c + s that one staged write covers apart.  With bit
// 2 alone the staged writes took 1.7 (NN) and 3.0 (NT) bank-conflict cycles
// per LDS instruction, with both bits 0.57 and 1.0; the reads have none.
// Writing the values one ds_write_b32 at a time (instead of the pairs of
// ds_write2st64_b32, whose two values always share a bank) moved the same
// conflict cycles to more instructions.  None of it is on the matrix core's
// path: NN, NT and TT run as fast as TN.
//
// MODE carries the fusions of the MLP step (mlp.hip); MlpFuse (gemm_common.hpp)
// holds their operands.  A group is a row half, and there are WN = 4 waves
// along N:
//   MODE 1 (H = sigmoid(X W1), A staged, B copied): sigmoid in the epilogue,
//     and zpart[(tn*4 + wn)*M + row] = sum over the wave's 64 columns of
//     H[row][col] * w2[col];
//   MODE 2 (slice of X^T d1 / w2, both operands copied): B is H; each B
//     value h at batch row k becomes d2[k] h (1 - h) in the C phase before its
//     MFMAs.  d1 = (d2[k] w2[n]) h (1 - h) also has the column factor w2[n],
//     which the caller applies to the summed slices: two VALU instructions per
//     value here instead of four.  The wave owning the k-block (k-tile kt of
//     M-tile kt % tiles_m, k-block kb of group kb % 2) adds h d2[k] to its
//     dW2 partial, written to dw2part[((split*tiles_m + tm)*2 + grp)*N + n].
//     d2 reaches LDS with the k-tile (every wave copies the same 64 bytes, so
//     each wave's count of copies stays uniform).
#pragma once

#include "gemm_common.hpp"
#include "gemm_pingpong.hpp"
#include "gemm_tiles.hpp"

namespace ch {

template <bool AKC, bool BKC, int MODE = 0, int TILE = 256>
struct F32PingPong {
    static constexpr int BM = TILE, BN = TILE, BK = 16, NW = 8, WN = 4, THREADS = 64 * NW;
    static constexpr int TM = TILE / 2, TN = TILE / 4, FM = TM / 32, FN = TN / 32, KB = BK / 8;
    static constexpr int STAGES = TILE == 256 ? kPingPongStages : 6;
    static constexpr int A_BYTES = BM * BK * 4, B_BYTES = BN * BK * 4;  // one stage of one operand
    static constexpr int ROW = BM * 4;                                    // one k-row of one stage
    // Strides of k-row and stage within an operand's region: 256 x 256 tiles
    // [16 k-rows][4 stages][256] (a copy instruction's 1 KiB is one k-row of
    // one stage); 128 x 128 tiles [4 stages][16 k-rows][128] (its 1 KiB is two
    // consecutive k-rows).
    static constexpr int KSTR = TILE == 256 ? STAGES * ROW : ROW;
    static constexpr int SSTR = TILE == 256 ? ROW : BK * ROW;
    static constexpr int OP_BYTES = BK * STAGES * ROW;                   // A at 0, B at OP_BYTES
    static constexpr int D2_BYTES = MODE == 2 ? STAGES * BK * 4 : 0;    // MODE 2: d2 per stage
    static constexpr int LDS_BYTES = 2 * OP_BYTES + D2_BYTES;
    // Per wave and k-tile: global_load_lds instructions of the m/n-contiguous
    // operands (and of d2).
    static constexpr int OP_LOADS = A_BYTES / 1024 / NW;  // per operand
    static constexpr int LDMA = OP_LOADS * ((AKC ? 0 : 1) + (BKC ? 0 : 1)) + (MODE == 2 ? 1 : 0);
    static_assert(TILE == 256 || TILE == 128, "256 x 256 or 128 x 128 tiles");
    static_assert(A_BYTES == B_BYTES && OP_LOADS >= 1 && OP_BYTES <= 65536, "an operand's ring within 64 KiB");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS per workgroup");
    static_assert(MODE == 0 || (MODE == 1 && AKC && !BKC && TILE == 256) || (MODE == 2 && !AKC && !BKC && TILE == 256),
                  "MODE 1 is the NN form, MODE 2 the TN form, both on 256 x 256 tiles");

    static bool fits(int M, int N, int K, int64_t lda, int64_t ldb) {
        const bool dims = M % BM == 0 && N % BN == 0 && K % BK == 0 && lda % 4 == 0 && ldb % 4 == 0;
        // the 32-bit offsets span one tile: BM (BN) rows of a k-contiguous
        // operand (its first row is in the buffer resource's base), BK k-rows
        // of an m/n-contiguous one
        const uint64_t a_span = (AKC ? (uint64_t)BM : (uint64_t)BK + 1) * (uint64_t)lda * 4;
        const uint64_t b_span = (BKC ? (uint64_t)BN : (uint64_t)BK + 1) * (uint64_t)ldb * 4;
        return dims && a_span < (1ull << 32) && b_span < (1ull << 32);
    }
};

namespace f32pp {

// Slot of 16-byte chunk c (of 64) in k-major LDS row kr.
__device__ __forceinline__ int pp_slot(int kr, int c) { return c ^ (((kr >> 2) & 1) << 3) ^ (((kr >> 3) & 1) << 2); }

typedef __attribute__((address_space(3))) float lds_float;
__device__ __forceinline__ const lds_float* lds_ptr(uint32_t a) { return (const lds_float*)(uintptr_t)a; }
__device__ __forceinline__ lds_float* lds_ptr_w(uint32_t a) { return (lds_float*)(uintptr_t)a; }

using tiles::opaque;

// One staged load: 16 bytes per lane at byte offset voff + soff of the
// operand behind rsrc.  A buffer load: the per-lane offset is one VGPR and
// the k-tile's offset one SGPR, so no VALU address arithmetic; and an
// ordinary (not inline-asm) load, so the compiler knows the registers are in
// flight and waits (vmcnt) before their first use -- including any register
// copy it makes.  The compiler does not count the global_load_lds copies
// (inline asm), so its waits can only be longer than needed, never shorter.
__device__ __forceinline__ tiles::v4f load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, soff, 0);
}
// Raw buffer resource over [p, p + 4 GiB): gfx9-family word 3 (32-bit
// untyped elements); offsets past the end would read as zero, not fault.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)0xFFFFFFFF, 0x00020000);
}

// Staged copy of a k-contiguous operand tile [R rows][16 k] into its
// k-major LDS region (k-row stride KSTR, stage stride SSTR).  Load q
// (q = wave + 8 j) covers rows 16q .. 16q+15, lane l taking row 16q + l/4,
// k-chunk l%4 (64 bytes of each row per load); its four floats go to k-rows
// 4*(l%4) + s, column row.  One register set (data) in the loop: the M phase
// writes tile u+1 to LDS before loading tile u+2 into it.
template <int NW, int R, int KSTR, int SSTR>
struct Staged {
    static constexpr int BK = 16, PER_WAVE = R * BK * 4 / 1024 / NW;
    static_assert(PER_WAVE >= 1, "a load per wave");
    uint32_t voff[PER_WAVE];
    uint32_t waddr[PER_WAVE];  // LDS address of (k-row 4*kc, stage 0, column row)
    tiles::v4f data[PER_WAVE];

    __device__ __forceinline__ void init(int64_t ld, int r0, int wave, int lane, uint32_t region) {
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) {
            const int q = wave + NW * j;
            const int row = 16 * q + (lane >> 2), kc = lane & 3;
            voff[j] = (uint32_t)(((int64_t)(r0 + row) * ld + 4 * kc) * 4);
            // pp_slot(4*kc + s, row/4) does not depend on s
            waddr[j] = region + (uint32_t)(4 * kc * KSTR + pp_slot(4 * kc, row >> 2) * 16 + (row & 3) * 4);
            opaque(voff[j]);
            opaque(waddr[j]);
        }
    }
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rsrc, uint32_t kt_off, tiles::v4f (&d)[PER_WAVE]) const {
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) d[j] = load16(rsrc, voff[j], kt_off);
    }
    // Write registers d into LDS stage ST.
    template <int ST>
    __device__ __forceinline__ void store(const tiles::v4f (&d)[PER_WAVE]) const {
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s) lds_ptr_w(waddr[j] + ST * SSTR + s * KSTR)[0] = d[j][s];
    }
};

// global_load_lds copy of an m/n-contiguous operand tile [16 k][R rows]:
// instruction q (q = wave + 8 j) moves k-rows RPI*q .. RPI*q + RPI-1 (one row
// of 256 floats, or two of 128, stored KSTR apart: contiguous when RPI is 2),
// lane l fetching the 16-byte chunk that belongs in slot l % CPR of its row.
template <int NW, int R, int KSTR>
struct Direct {
    static constexpr int BK = 16, CPR = R / 4, RPI = 64 / CPR, PER_WAVE = BK / RPI / NW;
    static_assert(PER_WAVE >= 1 && (RPI == 1 || KSTR == R * 4), "an instruction's k-rows are contiguous");
    uint32_t voff[PER_WAVE];
    uint32_t dst[PER_WAVE];  // LDS address of the instruction's first k-row, stage 0 (SGPR-uniform)

    __device__ __forceinline__ void init(int64_t ld, int r0, int wave, int lane, uint32_t region) {
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) {
            const int q = wave + NW * j;
            const int kr = RPI * q + lane / CPR;
            const int c = pp_slot(kr, lane % CPR);  // slot lane % CPR holds chunk c (the XOR is its own inverse)
            voff[j] = (uint32_t)(((int64_t)kr * ld + r0 + 4 * c) * 4);
            dst[j] = region + (uint32_t)(RPI * q * KSTR);
        }
    }
    __device__ __forceinline__ void issue(const char* sbase_kt, uint32_t stage_off) const {
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) tiles::dma16(sbase_kt, voff[j], dst[j] + stage_off);
    }
};

}  // namespace f32pp

// `batch` products of M x N x K, product z at A + z strideA, B + z strideB,
// C + z strideC.  With kslices > 1 (batch a multiple of it) the products are
// the K slices of batch / kslices products of depth K * kslices: z = s nb + b
// (nb = batch / kslices) is slice s of product b, at A + b strideA plus s K
// columns (k-contiguous A) or s K rows of A (likewise B), and C + z strideC.
template <bool AKC, bool BKC, int MODE = 0, int TILE = 256>
__global__ __launch_bounds__(512) void gemm_f32_pingpong_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    int64_t lda, int64_t ldb, int64_t strideA, int64_t strideB, int64_t strideC, int tiles_m, int tiles_n,
    int batch, int kslices, MlpFuse fuse) {
    using namespace ch::tiles;
    using namespace ch::f32pp;
    using P = F32PingPong<AKC, BKC, MODE, TILE>;
    constexpr int FM = P::FM, FN = P::FN, NW = P::NW, BK = P::BK, KB = P::KB, S = P::STAGES;
    constexpr int KSTR = P::KSTR, SSTR = P::SSTR;
    constexpr bool STAGED = AKC || BKC;
    __shared__ __attribute__((aligned(1024))) char smem[P::LDS_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = wave / P::WN, wn = wave % P::WN;  // grp is also the wave's row block
    int bt, tm, tn;
    ch::block_coords(blockIdx.x, tiles_m, tiles_n, batch, bt, tm, tn);
    const int m0 = tm * P::BM, n0 = tn * P::BN;
    if (kslices > 1) {
        const int nb = batch / kslices, sl = bt / nb, pb = bt - sl * nb;
        A += (int64_t)pb * strideA + (AKC ? (int64_t)sl * K : (int64_t)sl * K * lda);
        B += (int64_t)pb * strideB + (BKC ? (int64_t)sl * K : (int64_t)sl * K * ldb);
    } else {
        A += (int64_t)bt * strideA;
        B += (int64_t)bt * strideB;
    }
    C += (int64_t)bt * strideC;
    const uint32_t lds0 = lds_addr(smem);
    const int nk = K / BK;

    const uint32_t region_a = lds0, region_b = lds0 + P::OP_BYTES;
    // m/n-contiguous operands: global_load_lds into the k-major tile.
    Direct<NW, TILE, KSTR> dma_a, dma_b;
    // k-contiguous operands: staged through registers.
    using StagedT = Staged<NW, TILE, KSTR, SSTR>;
    StagedT st_a, st_b;
    if constexpr (!AKC) dma_a.init(lda, m0, wave, lane, region_a);
    else st_a.init(lda, 0, wave, lane, region_a);
    if constexpr (!BKC) dma_b.init(ldb, n0, wave, lane, region_b);
    else st_b.init(ldb, 0, wave, lane, region_b);
    // byte step of an operand's base per k-tile
    const int64_t step_a = AKC ? (int64_t)BK * 4 : (int64_t)BK * lda * 4;
    const int64_t step_b = BKC ? (int64_t)BK * 4 : (int64_t)BK * ldb * 4;
    const char* a_base = reinterpret_cast<const char*>(A);
    const char* b_base = reinterpret_cast<const char*>(B);

    // Copies of k-tile kt into stage kt % S.  With STAGED the M phase copies
    // unconditionally: past the last k-tile the source is clamped to it (in
    // bounds) and the bytes land in a stage no later M phase reads.
    // MODE 2: this split's d2 slice starts at batch row bt * K.
    const float* d2 = MODE == 2 ? fuse.d2 + (int64_t)bt * K : nullptr;
    const uint32_t region_d2 = lds0 + 2u * P::OP_BYTES;
    auto issue_dma = [&](int kt) {
        const uint32_t stage_off = (uint32_t)((kt % S) * SSTR);
        const int src = min(kt, nk - 1);
        if constexpr (!AKC) dma_a.issue(a_base + src * step_a, stage_off);
        if constexpr (!BKC) dma_b.issue(b_base + src * step_b, stage_off);
        if constexpr (MODE == 2) {
            if (lane < BK / 4)
                dma16(d2 + (int64_t)src * BK, (uint32_t)(lane * 16), region_d2 + (uint32_t)((kt % S) * BK * 4));
        }
    };
    // a k-contiguous operand's resource starts at its tile's first row: the
    // 32-bit offsets then span 256 rows, so an operand of any size is reached
    const __amdgpu_buffer_rsrc_t rsrc_a = raw_rsrc(A + (AKC ? (int64_t)m0 * lda : 0));
    const __amdgpu_buffer_rsrc_t rsrc_b = raw_rsrc(B + (BKC ? (int64_t)n0 * ldb : 0));
    auto load_staged = [&](int kt) {
        const uint32_t src = (uint32_t)min(kt, nk - 1);
        if constexpr (AKC) st_a.load(rsrc_a, src * (uint32_t)step_a, st_a.data);
        if constexpr (BKC) st_b.load(rsrc_b, src * (uint32_t)step_b, st_b.data);
    };
    auto store_staged = [&](auto stage) {
        constexpr int ST = decltype(stage)::value;
        if constexpr (AKC) st_a.template store<ST>(st_a.data);
        if constexpr (BKC) st_b.template store<ST>(st_b.data);
    };

    // Fragment read addresses: fragment f (A: f < FM, B: f >= FM) of k-block
    // kb, step s, stage ST sits at rd[kb][f] + (8kb + s)*KSTR + ST*SSTR.
    // Half-wave h reads k-rows kr = 8kb + 4h + s, whose slot depends on kr
    // through bit 2 (= h) and bit 3 (= kb).
    uint32_t rd[KB][FM + FN];
    {
        const int h = lane >> 5;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int f = 0; f < FM + FN; ++f) {
                const int col =
                    f < FM ? grp * P::TM + f * 32 + (lane & 31) : wn * P::TN + (f - FM) * 32 + (lane & 31);
                const int kr = 8 * kb + 4 * h;
                rd[kb][f] = (f < FM ? region_a : region_b) +
                            (uint32_t)(4 * h * KSTR + pp_slot(kr, col >> 2) * 16 + (col & 3) * 4);
                opaque(rd[kb][f]);
            }
    }

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16f{};
    v4f fa[KB][FM], fb[KB][FN];

    // MODE 2: d2 at this lane's k-rows of each k-block, and the dW2 partial
    // of its columns.
    v4f d2v[KB];
    v4f dw2acc[FN];
    uint32_t rd_d2 = 0;
    if constexpr (MODE == 2) {
#pragma unroll
        for (int j = 0; j < FN; ++j) dw2acc[j] = v4f{};
        rd_d2 = region_d2 + (uint32_t)(16 * (lane >> 5));  // k = 8kb + 4h + s
        opaque(rd_d2);
    }

    // M phase for k-tile u in stage ST: fragments of tile u; then the staged
    // operand of tile u+1 (loaded in the previous M phase; for u = 0 the
    // prologue wrote it) into its stage;
    // then the staged loads of tile u+2 (into the same registers) and the
    // global_load_lds of tile u+3; then wait for the LDS reads and writes.
    // Before the staged store the compiler waits for its loads with vmcnt(0)
    // (it counts no load issued after them), which also covers the copy of
    // tile u+1, issued a phase before them.  The wave issued nothing in the
    // other group's phase, so that wait finds loads a k-tile old.  Stage
    // (u+1)%4 last held tile u-3 and stage (u+3)%4 tile u-1, both read by
    // both groups before this phase.
    auto m_phase = [&](auto stage, int u) {
        constexpr int ST = decltype(stage)::value;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const uint32_t off = (8 * kb + s) * KSTR + ST * SSTR;
#pragma unroll
                for (int i = 0; i < FM; ++i) fa[kb][i][s] = *lds_ptr(rd[kb][i] + off);
#pragma unroll
                for (int j = 0; j < FN; ++j) fb[kb][j][s] = *lds_ptr(rd[kb][FM + j] + off);
            }
        if constexpr (MODE == 2) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
                d2v[kb] = *reinterpret_cast<const __attribute__((address_space(3))) v4f*>(
                    (uintptr_t)(rd_d2 + ST * BK * 4 + kb * 32));
        }
        if constexpr (STAGED) {
            if (u > 0) store_staged(PingPongStage<(ST + 1) % S>{});  // the prologue wrote tile 1
            load_staged(u + 2);
            issue_dma(u + S - 1);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        } else {
            pingpong_copy<P::LDMA, S>(u, issue_dma);
        }
    };
    // Half-wave h holds k = 8*kb + 4*h + s at step s for both operands, so the
    // four steps of a k-block complete its 8-deep k-sum.
    auto c_phase = [&](int u) {
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
            if constexpr (MODE == 2) {
                if ((u % tiles_m) == tm && kb % 2 == grp) {
                    asm volatile("");  // a branch, not a select in every wave
#pragma unroll
                    for (int j = 0; j < FN; ++j) dw2acc[j] += fb[kb][j] * d2v[kb];
                }
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const float h = fb[kb][j][s];
                        fb[kb][j][s] = d2v[kb][s] * __builtin_fmaf(-h, h, h);  // d2[k] h (1 - h)
                    }
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[kb][i][s], fb[kb][j][s], acc[i][j], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) asm volatile("" : "+a"(acc[i][j]));  // accumulators stay in AGPRs
    };

    if constexpr (STAGED) {
        // Prologue: tiles 0 and 1 in stages 0 and 1 (staged parts written),
        // the copied parts of tiles 0 .. S-2 landed.  Tile 1's staged
        // registers are temporaries: no staged register is live when the
        // groups' loops begin.
        {
            v4f t1a[StagedT::PER_WAVE], t1b[StagedT::PER_WAVE];
            load_staged(0);
            if constexpr (AKC) st_a.load(rsrc_a, (uint32_t)min(1, nk - 1) * (uint32_t)step_a, t1a);
            if constexpr (BKC) st_b.load(rsrc_b, (uint32_t)min(1, nk - 1) * (uint32_t)step_b, t1b);
#pragma unroll
            for (int t = 0; t < S - 1; ++t) issue_dma(t);
            store_staged(PingPongStage<0>{});
            if constexpr (AKC) st_a.template store<1>(t1a);
            if constexpr (BKC) st_b.template store<1>(t1b);
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        }
        pingpong_schedule<P::LDMA, S>(nk, grp, [](int) {}, m_phase, c_phase, /*prologue_copies=*/false);
    } else {
        pingpong_schedule<P::LDMA, S>(nk, grp, issue_dma, m_phase, c_phase, /*prologue_copies=*/true);
    }

    // 32 x 32 accumulator layout: lane holds column l%32, rows 8*(v/4) + 4*(l/32) + v%4.
    // One row of tiles at a time out of the AGPRs (the asm keeps the compiler
    // from reading all 128 first, which would need 128 more VGPRs).
    const int half = lane >> 5, col = lane & 31;
    if constexpr (MODE == 2) {
        // every wave writes its partial (zero when it took no k-block)
        float* dst = fuse.dw2part + ((int64_t)(bt * tiles_m + tm) * 2 + grp) * N + n0 + wn * P::TN + col;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            float v = (dw2acc[j][0] + dw2acc[j][1]) + (dw2acc[j][2] + dw2acc[j][3]);
            v += __shfl_xor(v, 32);
            if (half == 0) dst[j * 32] = v;
        }
    }
    float w2j[FN];
    if constexpr (MODE == 1) {
#pragma unroll
        for (int j = 0; j < FN; ++j) w2j[j] = fuse.w2[n0 + wn * P::TN + j * 32 + col];
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        float zs[16];  // MODE 1: per row, the sum of H * w2 over the wave's columns
#pragma unroll
        for (int v = 0; v < 16; ++v) zs[v] = 0.0f;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            v16f t = acc[i][j];
            asm volatile("" : "+v"(t)::"memory");
            if constexpr (MODE == 1) {
                // H = sigmoid(acc) = 1 / (1 + exp(-acc)) with the hardware exp2
                // and reciprocal (about 1 ulp each)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float e = __builtin_amdgcn_exp2f(-t[v] * 1.4426950408889634f);
                    const float h = __builtin_amdgcn_rcpf(1.0f + e);
                    t[v] = h;
                    zs[v] += h * w2j[j];
                }
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = m0 + grp * P::TM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                const int c = n0 + wn * P::TN + j * 32 + col;
                C[(int64_t)r * N + c] = t[v];
            }
        }
        if constexpr (MODE == 1) {
            // lanes of a half-wave hold the 32 columns of the same rows
#pragma unroll
            for (int v = 0; v < 16; ++v)
#pragma unroll
                for (int o = 16; o > 0; o >>= 1) zs[v] += __shfl_xor(zs[v], o);
            if (col == 0) {
                float* zp = fuse.zpart + (int64_t)(tn * P::WN + wn) * M;
#pragma unroll
                for (int v = 0; v < 16; ++v) zp[m0 + grp * P::TM + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3)] = zs[v];
            }
        }
    }
}

}  // namespace ch
