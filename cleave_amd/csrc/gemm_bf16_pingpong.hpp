// gemm_bf16_pingpong.hpp -- bf16 GEMM with a ping-pong schedule of its two
// wave groups (gfx950, v_mfma_f32_16x16x32_bf16, 256 x 256 x 32 tiles).
//
// Eight waves; each owns a 128 x 64 block of C (8 x 4 tiles of 16 x 16).
// Waves 0-3 (group 0, rows 0-127 of the tile) and 4-7 (group 1, rows
// 128-255) sit one per SIMD, and the two groups alternate between
//   C phase: the k-step's 32 MFMAs back to back, operands already in
//            registers, at raised wave priority;
//   M phase: read the next k-step's fragments from LDS, issue this wave's
//            share of the global -> LDS copy S-1 k-tiles ahead, wait for
//            its own copy of the next k-tile and for the fragment reads.
// The schedule is pingpong_schedule (gemm_pingpong.hpp).  k-tiles are 32 deep
// (one MFMA k-step) in a ring of S LDS stages of 32 KiB.  S = 5 fills the
// 160 KiB of LDS and leaves the copies four k-tiles to land; it measured
// 2-3% faster than S = 4 at 8192^3 on random data.
#pragma once

#include "gemm_common.hpp"
#include "gemm_pingpong.hpp"
#include "gemm_tiles.hpp"

namespace ch {

template <bool AKC, bool BKC, int STAGES_ = 5>
struct Bf16PingPong {
    static constexpr int BM = 256, BN = 256, BK = 32, NW = 8, WN = 4, THREADS = 64 * NW;
    static constexpr int TM = 128, TN = 64, FM = TM / 16, FN = TN / 16, STAGES = STAGES_;
    static_assert(STAGES == 4 || STAGES == 5, "ring depth");
    static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2;
    static constexpr int STAGE_BYTES = A_BYTES + B_BYTES, LDS_BYTES = STAGES * STAGE_BYTES;
    static constexpr int LPW = STAGE_BYTES / 1024 / NW;  // copy instructions per wave per k-tile
    static_assert(LDS_BYTES <= 160 * 1024, "LDS per workgroup");

    static bool fits(int M, int N, int K, int64_t lda, int64_t ldb) {
        const bool dims = M % BM == 0 && N % BN == 0 && K % BK == 0 && lda % 8 == 0 && ldb % 8 == 0;
        // the 32-bit lane offsets span one tile: BM (BN) rows of a k-contiguous
        // operand, BK k-rows of an m/n-contiguous one
        const uint64_t a_span = (AKC ? (uint64_t)BM : (uint64_t)BK + 1) * (uint64_t)lda * 2;
        const uint64_t b_span = (BKC ? (uint64_t)BN : (uint64_t)BK + 1) * (uint64_t)ldb * 2;
        return dims && a_span < (1ull << 32) && b_span < (1ull << 32);
    }
    // Bytes from an operand's base to the end of its last chunk
    // (ch::edge_bytes), and the shapes the EDGE form takes (as
    // Bf16PingPongPairs::fits_edge).
    static __host__ __device__ int64_t a_bytes(int M, int K, int64_t lda) {
        return edge_bytes<8, 2>(AKC, M, K, lda);
    }
    static __host__ __device__ int64_t b_bytes(int N, int K, int64_t ldb) {
        return edge_bytes<8, 2>(BKC, N, K, ldb);
    }
    static bool fits_edge(int M, int N, int K, int64_t lda, int64_t ldb, bool padded = false) {
        const bool chunks = edge_chunks<8>(AKC, M, K, lda, padded) && edge_chunks<8>(BKC, N, K, ldb, padded);
        return M >= 1 && N >= 1 && K >= 1 && chunks && a_bytes(M, K, lda) < (1ll << 31) &&
               b_bytes(N, K, ldb) < (1ll << 31);
    }
};

// OFF32: every k-tile's offset from an operand's base fits 32 bits (K times
// the operand's k-step under 4 GiB), so the M phase forms the copy sources
// with one 32-bit scalar multiply instead of a 64-bit one (0.5-1% at 8192^3).
// EDGE (any M, N and K, fits_edge): tiles_m and tiles_n rounded up; both
// copies become EdgeCopy buffer loads that read zeros past the operands' rows
// (columns) and past K, and the stores skip what lies past M or N.
// NTC: C stored non-temporally (tiles::store_acc16_lines).
template <bool AKC, bool BKC, bool OFF32 = false, int STAGES_ = 5, bool EDGE = false, bool NTC = false>
__global__ __launch_bounds__(512) void gemm_bf16_pingpong_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, float* __restrict__ C, int M,
    int N, int K, int64_t lda, int64_t ldb, int64_t strideA, int64_t strideB, int64_t strideC,
    int tiles_m, int tiles_n, int batch) {
    using namespace ch::tiles;
    using P = Bf16PingPong<AKC, BKC, STAGES_>;
    constexpr int FM = P::FM, FN = P::FN, NW = P::NW, BK = P::BK, LPW = P::LPW, S = P::STAGES;
    __shared__ __attribute__((aligned(1024))) char smem[P::LDS_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = wave / P::WN, wn = wave % P::WN;  // grp is also the wave's row block
    int bt, tm, tn;
    ch::block_coords(blockIdx.x, tiles_m, tiles_n, batch, bt, tm, tn);
    const int m0 = tm * P::BM, n0 = tn * P::BN;
    A += (int64_t)bt * strideA;
    B += (int64_t)bt * strideB;
    C += (int64_t)bt * strideC;

    TileCopy<AKC, P::BM, BK, NW> copy_a;
    TileCopy<BKC, P::BN, BK, NW> copy_b;
    copy_a.init(lda, m0, wave, lane);
    copy_b.init(ldb, n0, wave, lane);
    const int64_t step_a = copy_a.kstep(lda), step_b = copy_b.kstep(ldb);
    const uint32_t lds0 = lds_addr(smem);
    const int nk = EDGE ? (K + BK - 1) / BK : K / BK;
    const uint32_t step_a32 = (uint32_t)step_a, step_b32 = (uint32_t)step_b;
    const char* a_src = reinterpret_cast<const char*>(A) + copy_a.base_offset(lda, m0);
    const char* b_src = reinterpret_cast<const char*>(B) + copy_b.base_offset(ldb, n0);
    EdgeCopy<AKC, P::BM, BK, NW> edge_a;
    EdgeCopy<BKC, P::BN, BK, NW> edge_b;
    v4i rsrc_a{}, rsrc_b{};
    if constexpr (EDGE) {
        edge_a.init(lda, m0, M, wave, lane);
        edge_b.init(ldb, n0, N, wave, lane);
        rsrc_a = buffer_rsrc(A, (uint32_t)P::a_bytes(M, K, lda));
        rsrc_b = buffer_rsrc(B, (uint32_t)P::b_bytes(N, K, ldb));
    }
    auto issue = [&](int kt) {  // k-tile min(kt, nk-1) into stage kt % S
        const int src = min(kt, nk - 1);
        const uint32_t dst = lds0 + (uint32_t)((kt % S) * P::STAGE_BYTES);
        if constexpr (EDGE) {
            edge_a.issue(rsrc_a, src, K, (uint32_t)src * edge_a.kstep(lda), dst, wave);
            edge_b.issue(rsrc_b, src, K, (uint32_t)src * edge_b.kstep(ldb), dst + P::A_BYTES, wave);
        } else if constexpr (OFF32) {
            copy_a.issue(a_src + (uint32_t)src * step_a32, dst, wave);
            copy_b.issue(b_src + (uint32_t)src * step_b32, dst + P::A_BYTES, wave);
        } else {
            copy_a.issue(a_src + src * step_a, dst, wave);
            copy_b.issue(b_src + src * step_b, dst + P::A_BYTES, wave);
        }
    };

    v4f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v4f{};
    v8bf fa[FM], fb[FN];

    // Per-lane LDS addresses of this wave's fragment reads, one set per
    // 64 KiB window of the ring (a DS immediate offset reaches 64 KiB), kept
    // opaque so that each stays one register: the M phase then reads every
    // fragment as register + immediate, with no VALU instruction (left to
    // itself the compiler re-added lane offsets to window bases there, which
    // cost 1-3% at 8192^3).  A KC operand's swizzle repeats every 32 rows, so
    // its fragments two apart share a register; an MN operand's swizzle mixes
    // the fragment's column bits, so each MN fragment has its own.
    constexpr int NWIN = (S + 1) / 2;
    constexpr int NA = AKC ? 2 : FM, NB = BKC ? 2 : FN;
    uint32_t ra[NWIN][NA], rb[NWIN][NB];
#pragma unroll
    for (int w = 0; w < NWIN; ++w) {
        const uint32_t win = lds0 + (uint32_t)(2 * w * P::STAGE_BYTES);
#pragma unroll
        for (int x = 0; x < NA; ++x) {
            ra[w][x] = win + frag16_offset<AKC, P::BM, BK>(grp * P::TM + x * 16, lane);
            opaque(ra[w][x]);
        }
#pragma unroll
        for (int x = 0; x < NB; ++x) {
            rb[w][x] = win + (uint32_t)P::A_BYTES + frag16_offset<BKC, P::BN, BK>(wn * P::TN + x * 16, lane);
            opaque(rb[w][x]);
        }
    }

    // M phase for k-step u (stage ST = u % S, at ST * 32 KiB): fragments of
    // tile u; copy of tile u+S-1 into the stage of tile u-1; wait for this
    // wave's copy of tile u+1 and for the reads.
    auto m_phase = [&](auto stage, int u) {
        constexpr int ST = decltype(stage)::value, W = ST / 2;
        constexpr uint32_t SO = (ST % 2) * P::STAGE_BYTES;  // stage offset within window W
        constexpr uint32_t PAIR = 2 * 16 * BK * 2;            // two 16-row KC fragments
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            if constexpr (AKC) fa[i] = read16_kc_at(ra[W][i & 1] + SO + (uint32_t)(i / 2) * PAIR);
            else fa[i] = read16_mn_at<P::BM>(ra[W][i] + SO);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            if constexpr (BKC) fb[j] = read16_kc_at(rb[W][j & 1] + SO + (uint32_t)(j / 2) * PAIR);
            else fb[j] = read16_mn_at<P::BN>(rb[W][j] + SO);
        }
        pingpong_copy<LPW, S>(u, issue);
    };
    auto c_phase = [&](int) {
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_s_setprio(0);
    };
    pingpong_schedule<LPW, S>(nk, grp, issue, m_phase, c_phase);

    const int r0 = m0 + grp * P::TM, c0 = n0 + wn * P::TN;
    if constexpr (EDGE) store_acc16_lines_masked<FM, FN, NTC>(C, N, r0, c0, acc, lane, M, N);
    else store_acc16_lines<FM, FN, NTC>(C, N, r0, c0, acc, lane);
}

}  // namespace ch

namespace ch {

// The same ping-pong for the layouts with exactly one k-contiguous operand
// (A·B: A; Aᵀ·Bᵀ: B).  A k-contiguous k-tile is a 64-byte segment of each
// row, and copying it as such cost 3-5% against the layout with none.  Here
// that operand ("paired") is copied two k-tiles at a time, whole 128-byte
// rows, into a ring of 3 pair-stages (96 KiB); the m/n-contiguous operand
// ("single") keeps a ring of 4 single k-tile stages (64 KiB).  8192^3 A·B:
// 0.736-0.740 ms against 0.777-0.790 for the single-stage kernel, bit-identical.
//
// Pair-stage layout: [256 rows][8 chunks of 16 bytes], chunk c of row r in
// slot c ^ ((r >> 1) & 7).  A fragment read has each 16-lane quarter read one
// chunk of 16 consecutive rows; rows r and r+1 sit 128 bytes apart and the
// XOR spreads the 8 row pairs over the 8 slots, so the quarter covers all
// 256 bytes of the banks once.
//
// Copy schedule, per M phase u: half u % 2 of the pair u/2 + 2 (2
// instructions per wave: even u the first, odd u the second) and then the
// single k-tile u + 3 (2 per wave), both clamped to the last one, so every M
// phase issues the same 4 (issuing a whole pair at even u made the even
// phases' copy bursts 3x the odd ones').  This wave's copies of k-tile u + 1
// were issued at M(u - 2) or earlier, and exactly 8 instructions follow
// them: those of M(u - 1) and M(u).  So every M phase ends in s_waitcnt
// vmcnt(8).  M(0) would need vmcnt(6), so the prologue instead waits until
// k-tiles 0 and 1 have both landed.
// A·Bᵀ, whose operands are both k-contiguous, pairs A and keeps B as the
// single operand, copied as 64-byte row segments into k-contiguous single
// stages: two pair rings would not fit 160 KiB with copies issued far
// enough ahead.
template <bool AKC, bool BKC, bool EDGE = false>
struct Bf16PingPongPairs {
    static_assert(AKC || BKC, "at least one k-contiguous operand");
    static constexpr bool SKC = AKC && BKC;  // the single operand is k-contiguous too
    static constexpr int BM = 256, BN = 256, BK = 32, NW = 8, WN = 4, THREADS = 64 * NW;
    static constexpr int TM = 128, TN = 64, FM = TM / 16, FN = TN / 16;
    static constexpr int PAIR_BYTES = 256 * 2 * BK * 2, SINGLE_BYTES = 256 * BK * 2;
    static constexpr int PAIRS = 3, SINGLES = 4, PERIOD = 12;  // PERIOD = lcm(2 * PAIRS, SINGLES)
    static constexpr int SINGLE_REGION = PAIRS * PAIR_BYTES;
    static constexpr int LDS_BYTES = SINGLE_REGION + SINGLES * SINGLE_BYTES;
    static_assert(LDS_BYTES <= 160 * 1024, "LDS per workgroup");

    // Also requires every 32-bit byte offset a copy forms under 4 GiB: 256
    // rows of a k-contiguous operand (its tile's first row is in the 64-bit
    // base), K rows of an m/n-contiguous one.
    static bool fits(int M, int N, int K, int64_t lda, int64_t ldb) {
        const bool dims = M % BM == 0 && N % BN == 0 && K % (2 * BK) == 0 && lda % 8 == 0 && ldb % 8 == 0;
        const uint64_t a_span = (uint64_t)(AKC ? BM : K + 1) * (uint64_t)lda * 2;
        const uint64_t b_span = (uint64_t)(BKC ? BN : K + 1) * (uint64_t)ldb * 2;
        return dims && a_span < (1ull << 32) && b_span < (1ull << 32);
    }
    // Bytes from an operand's base to the end of its last chunk (ch::edge_bytes).
    static __host__ __device__ int64_t a_bytes(int M, int K, int64_t lda) {
        return edge_bytes<8, 2>(AKC, M, K, lda);
    }
    static __host__ __device__ int64_t b_bytes(int N, int K, int64_t ldb) {
        return edge_bytes<8, 2>(BKC, N, K, ldb);
    }
    // Shapes the EDGE form takes (any M, N, K >= 1): whole 16-byte chunks (8
    // elements) along each operand's pitch and along K, an m/n extent in
    // whole chunks unless `padded` (ch::edge_chunks), and operands under
    // 2 GiB, so that a masked offset stays out of range.
    static bool fits_edge(int M, int N, int K, int64_t lda, int64_t ldb, bool padded = false) {
        const bool chunks = edge_chunks<8>(AKC, M, K, lda, padded) && edge_chunks<8>(BKC, N, K, ldb, padded);
        return M >= 1 && N >= 1 && K >= 1 && chunks && a_bytes(M, K, lda) < (1ll << 31) &&
               b_bytes(N, K, ldb) < (1ll << 31);
    }
};

// EDGE (any M, N and K, fits_edge): tiles_m and tiles_n rounded up; the
// copies become buffer loads into LDS whose lanes past the operand's rows
// (columns) or past K read zeros (a masked offset past the resource's range,
// as EdgeCopy), K is walked in whole pairs of k-tiles, and the stores skip
// what lies past M or N.
// NTC: C stored non-temporally (tiles::store_acc16_lines).
template <bool AKC, bool BKC, bool EDGE = false, bool NTC = false>
__global__ __launch_bounds__(512) void gemm_bf16_pingpong_pairs_kernel(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, float* __restrict__ C, int M,
    int N, int K, int64_t lda, int64_t ldb, int64_t strideA, int64_t strideB, int64_t strideC,
    int tiles_m, int tiles_n, int batch) {
    using namespace ch::tiles;
    using P = Bf16PingPongPairs<AKC, BKC, EDGE>;
    constexpr int FM = P::FM, FN = P::FN, NW = P::NW, BK = P::BK;
    constexpr int PAIRS = P::PAIRS, SINGLES = P::SINGLES;
    __shared__ __attribute__((aligned(1024))) char smem[P::LDS_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = wave / P::WN, wn = wave % P::WN;
    const uint32_t lds0 = lds_addr(smem);
    const int nk = EDGE ? (K + 2 * BK - 1) / (2 * BK) * 2 : K / BK, np = nk / 2;

    // The paired (k-contiguous) operand and the single one.  Each copy's
    // 64-bit scalar base holds the tile's first row (paired operand; single
    // operand when k-contiguous) or first column (single, m/n-contiguous),
    // so the 32-bit lane offsets below are the same for every tile.
    const int64_t pld = AKC ? lda : ldb, sld = AKC ? ldb : lda;
    constexpr bool SKC = P::SKC;
    using SCopy = TileCopy<SKC, 256, BK, NW>;
    const char* pbase;
    const char* sbase;
    float* Ct;
    int m0, n0;
    // EDGE: resources over this product's operands; per-lane pair-copy
    // offsets from the paired operand's base (kOutOfRange past its rows) and
    // the k of each lane's chunk in pair 0; the single operand's EdgeCopy.
    const int pext = AKC ? M : N, sext = AKC ? N : M;  // rows of the paired / single operand
    v4i rsrc_p{}, rsrc_s{};
    uint32_t pvoff_e[4];
    int pk0[4];
    EdgeCopy<SKC, 256, BK, NW> ecopy;
    auto set_tile = [&](int t) {
        int bt, tm, tn;
        ch::block_coords(t, tiles_m, tiles_n, batch, bt, tm, tn);
        m0 = tm * P::BM;
        n0 = tn * P::BN;
        const int pr0 = AKC ? m0 : n0, sr0 = AKC ? n0 : m0;
        const uint16_t* Ab = A + (int64_t)bt * strideA;
        const uint16_t* Bb = B + (int64_t)bt * strideB;
        if constexpr (EDGE) {
            rsrc_p = buffer_rsrc(AKC ? Ab : Bb, (uint32_t)(AKC ? P::a_bytes(M, K, lda) : P::b_bytes(N, K, ldb)));
            rsrc_s = buffer_rsrc(AKC ? Bb : Ab, (uint32_t)(AKC ? P::b_bytes(N, K, ldb) : P::a_bytes(M, K, lda)));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int q = wave + NW * j;
                const int r = 8 * q + (lane >> 3);
                const int c = (lane & 7) ^ ((r >> 1) & 7);
                pvoff_e[j] = pr0 + r < pext ? (uint32_t)(((int64_t)(pr0 + r) * pld + 8 * c) * 2) : kOutOfRange;
                pk0[j] = 8 * c;
            }
            ecopy.init(sld, sr0, sext, wave, lane);
        } else {
            pbase = reinterpret_cast<const char*>(AKC ? Ab : Bb) + (int64_t)pr0 * pld * 2;
            sbase = reinterpret_cast<const char*>(AKC ? Bb : Ab) + (SKC ? (int64_t)sr0 * sld * 2 : (int64_t)sr0 * 2);
        }
        Ct = C + (int64_t)bt * strideC;
    };

    // pair copy: instruction q = wave + 8 j moves rows 8q .. 8q+7; lane l takes
    // row 8q + l/8 and slot l%8, which holds chunk (l%8) ^ ((row >> 1) & 7)
    uint32_t pvoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int q = wave + NW * j;
        const int r = 8 * q + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        pvoff[j] = (uint32_t)(((int64_t)r * pld + 8 * c) * 2);
    }
    SCopy scopy;
    scopy.init(sld, 0, wave, lane);
    const uint32_t sstep = (uint32_t)scopy.kstep(sld);
    // half h of pair p: instructions j = 2h, 2h + 1 (rows 8q .. 8q+7, q = wave + 8j)
    auto issue_pair_half = [&](auto stage, auto half, int p) {
        constexpr int PS = decltype(stage)::value, HF = decltype(half)::value;
        const int pc = min(p, np - 1);
        if constexpr (EDGE) {
            const uint32_t soff = (uint32_t)pc * (uint32_t)(2 * BK * 2);
#pragma unroll
            for (int j = 2 * HF; j < 2 * HF + 2; ++j)
                dma16_buf(rsrc_p, pk0[j] + pc * 2 * BK < K ? pvoff_e[j] : kOutOfRange, soff,
                          lds0 + (uint32_t)(PS * P::PAIR_BYTES + 1024 * (wave + NW * j)));
        } else {
            const char* src = pbase + (uint32_t)pc * (uint32_t)(2 * BK * 2);
#pragma unroll
            for (int j = 2 * HF; j < 2 * HF + 2; ++j)
                dma16(src, pvoff[j], lds0 + (uint32_t)(PS * P::PAIR_BYTES + 1024 * (wave + NW * j)));
        }
    };
    auto issue_pair = [&](auto stage, int p) {
        issue_pair_half(stage, std::integral_constant<int, 0>{}, p);
        issue_pair_half(stage, std::integral_constant<int, 1>{}, p);
    };
    auto issue_single = [&](auto stage, int kt) {
        constexpr int SS = decltype(stage)::value;
        const int kc = min(kt, nk - 1);
        const uint32_t dst = lds0 + (uint32_t)(P::SINGLE_REGION + SS * P::SINGLE_BYTES);
        if constexpr (EDGE) ecopy.issue(rsrc_s, kc, K, (uint32_t)kc * ecopy.kstep(sld), dst, wave);
        else scopy.issue(sbase + (uint32_t)kc * sstep, dst, wave);
    };

    // Fragment addresses.  Paired operand: per 64 KiB window (pair-stages 0-1,
    // pair-stage 2) and per half h of the pair; its fragments 16 rows apart
    // differ by an immediate.  Single operand: one window over its 4 stages,
    // one register per fragment (its swizzle mixes the fragment's columns).
    constexpr int NPF = AKC ? FM : FN, NSF = AKC ? FN : FM;  // paired / single fragments
    const int prow0 = AKC ? grp * P::TM : wn * P::TN;
    const int srow0 = AKC ? wn * P::TN : grp * P::TM;
    uint32_t rp[2][2], rs[NSF];
    {
        const int x = (lane & 15) >> 1, qd = lane >> 4;
        const int r = prow0 + (lane & 15);
#pragma unroll
        for (int w = 0; w < 2; ++w)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                rp[w][h] = lds0 + (uint32_t)(w * 2 * P::PAIR_BYTES) + (uint32_t)(r * 128 + (((h << 2) | qd) ^ x) * 16);
                opaque(rp[w][h]);
            }
#pragma unroll
        for (int f = 0; f < NSF; ++f) {
            rs[f] = lds0 + (uint32_t)P::SINGLE_REGION + frag16_offset<SKC, 256, BK>(srow0 + f * 16, lane);
            opaque(rs[f]);
        }
    }

    v4f acc[FM][FN];
    auto zero_acc = [&]() {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = v4f{};
    };
    v8bf fa[FM], fb[FN];

    // M phase of k-tile u (ST = u % 12): fragments, then the copies, then the wait.
    auto m_phase = [&](auto phase, int u) {
        constexpr int ST = decltype(phase)::value;
        constexpr int H = ST % 2, PS = (ST / 2) % PAIRS, SS = ST % SINGLES, W = PS / 2;
        constexpr uint32_t PO = (uint32_t)((PS - 2 * W) * P::PAIR_BYTES);
#pragma unroll
        for (int f = 0; f < NPF; ++f) {
            const v8bf v = read16_kc_at(rp[W][H] + PO + (uint32_t)(f * 16 * 128));
            if constexpr (AKC) fa[f] = v;
            else fb[f] = v;
        }
#pragma unroll
        for (int f = 0; f < NSF; ++f) {
            v8bf v;
            if constexpr (SKC) v = read16_kc_at(rs[f] + (uint32_t)(SS * P::SINGLE_BYTES));
            else v = read16_mn_at<256>(rs[f] + (uint32_t)(SS * P::SINGLE_BYTES));
            if constexpr (AKC) fb[f] = v;
            else fa[f] = v;
        }
        issue_pair_half(std::integral_constant<int, (ST / 2 + 2) % PAIRS>{}, std::integral_constant<int, H>{},
                        u / 2 + 2);
        issue_single(std::integral_constant<int, (ST + 3) % SINGLES>{}, u + 3);
        asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
    };
    auto c_phase = [&](int) {
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        __builtin_amdgcn_s_setprio(0);
    };
    // Prologue: pair 0, single 0, pair 1, single 1, single 2; k-tiles 0 and 1
    // have landed once only single 2's 2 instructions remain.
    auto prologue = [&]() {
        issue_pair(std::integral_constant<int, 0>{}, 0);
        issue_single(std::integral_constant<int, 0>{}, 0);
        issue_pair(std::integral_constant<int, 1>{}, 1);
        issue_single(std::integral_constant<int, 1>{}, 1);
        issue_single(std::integral_constant<int, 2>{}, 2);
    };

    // Tiles blockIdx.x, + gridDim.x, ...: a grid of fewer workgroups than
    // tiles keeps each workgroup on its CU from one tile to the next.  Between
    // tiles, the next tile's prologue copies go out before this tile's C
    // stores, so their latency overlaps the stores' drain, and no workgroup
    // is torn down and launched again.  (gridDim.x is a multiple of 8, so
    // every tile of a workgroup falls to the XCD block_coords planned for it.)
    const int total = tiles_m * tiles_n * batch;
    int tile = blockIdx.x;
    set_tile(tile);
    zero_acc();
    prologue();
    asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    auto store_c = [&](float* Cdone, int r0, int c0) {
        if constexpr (EDGE) store_acc16_lines_masked<FM, FN, NTC>(Cdone, N, r0, c0, acc, lane, M, N);
        else store_acc16_lines<FM, FN, NTC>(Cdone, N, r0, c0, acc, lane);
    };
    auto next_tile = [&]() {
        float* const Cdone = Ct;
        const int r0 = m0 + grp * P::TM, c0 = n0 + wn * P::TN;
        tile += (int)gridDim.x;
        if (tile >= total) {
            store_c(Cdone, r0, c0);
            return false;
        }
        // every wave's copies have landed (each waited for its own) before
        // the ring takes the next tile
        asm volatile("s_barrier" ::: "memory");
        set_tile(tile);
        prologue();
        store_c(Cdone, r0, c0);
        zero_acc();
        // everything but the last 8 stores has landed: the whole prologue,
        // so k-tile 0 of the next tile (the next M phase waits for the rest)
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        return true;
    };
    pingpong_schedule_tiles<P::PERIOD>(nk, grp, m_phase, c_phase, next_tile);
}

}  // namespace ch
