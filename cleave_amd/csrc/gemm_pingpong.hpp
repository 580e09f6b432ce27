// gemm_pingpong.hpp -- the ping-pong schedule shared by the f32 and bf16
// GEMM kernels of gemm_f32_pingpong.hpp and gemm_bf16_pingpong.hpp.
//
// Eight waves in two groups of four, one wave of each group per SIMD.  The
// groups alternate between
//   C phase: one k-tile's MFMAs back to back, operands already in registers;
//   M phase: read the next k-tile's operand fragments from LDS, issue this
//            wave's share of the global -> LDS copy S-1 k-tiles ahead, wait
//            for its own copy of the k-tile after the one just read, and for
//            the reads.
// A workgroup barrier closes every phase and group 1 runs one phase behind
// group 0, so on every SIMD one wave feeds the matrix core while the other
// moves data.  The k-tiles sit in a ring of S LDS stages (4 or 5); the copy
// of tile u+S-1 goes into the stage of tile u-1, which both groups finished
// reading a phase earlier.
//
// Group 0: M(0) in the prologue, then per k-tile s: C(s) | M(s+1).
// Group 1: per k-tile s: M(s) | C(s).
//
// The loops are unrolled over the S stages, so the M phase is handed its
// stage as a compile-time constant and can address every fragment as a
// loop-invariant register plus an immediate offset.  That keeps the M phase
// free of VALU instructions, which matters: a VALU instruction of the M wave
// does not issue while the C wave of its SIMD keeps the matrix core busy,
// and one such instruction ahead of the fragment reads held them back for
// most of a C phase (f32 at 4096^3: 0.857 of peak with the stage computed
// at run time, 0.912 unrolled).
#pragma once

#include <type_traits>
#include <utility>

namespace ch {

constexpr int kPingPongStages = 4;
template <int ST>
using PingPongStage = std::integral_constant<int, ST>;

// The copy half of an M phase for k-tile u: issue tile u+S-1, then wait for
// this wave's copy of tile u+1 -- the S-2 tiles issued after it may stay in
// flight -- and for the LDS reads already issued.  LPW is the number of copy
// instructions a wave issues per k-tile.  The copy is unconditional: issue()
// clamps its source to the last k-tile, so past the end it refills the stage
// of a tile both groups have finished with, which no later M phase reads.
// That keeps the M phase free of branches and its wait a constant (measured
// 0.5-3% faster for the bf16 kernel than issuing only real tiles and picking
// the wait count at run time).
template <int LPW, int S = kPingPongStages, class Issue>
__device__ __forceinline__ void pingpong_copy(int u, Issue&& issue) {
    static_assert(S >= 3 && (S - 2) * LPW < 64, "vmcnt counts up to 63");
    issue(u + S - 1);
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((S - 2) * LPW) : "memory");
}

// step(PingPongStage<(OFF + i) % S>{}, s + i) for i = 0, 1, ... while s + i < nk.
template <int S, int OFF, class Step, int... I>
__device__ __forceinline__ void pingpong_unrolled(int s, int nk, Step& step,
                                                  std::integer_sequence<int, I...>) {
    (void)((s + I < nk ? (step(PingPongStage<(OFF + I) % S>{}, s + I), true) : false) && ...);
}

// Runs the whole schedule over nk k-tiles.  issue(kt) copies this wave's
// share of k-tile min(kt, nk-1) into stage kt % S; m_phase(PingPongStage<ST>{}, u) is the
// M phase of k-tile u (stage ST = u % S), ending in pingpong_copy<LPW, S>;
// c_phase(u) is the C phase of k-tile u, on the fragments the wave's last M
// phase read.  With prologue_copies false the caller has already put tile 0 in
// stage 0 and started the copies of the next tiles, and issue is not called.
template <int LPW, int S = kPingPongStages, class Issue, class MPhase, class CPhase>
__device__ __forceinline__ void pingpong_schedule(int nk, int grp, Issue&& issue, MPhase&& m_phase,
                                                  CPhase&& c_phase, bool prologue_copies = true) {
    // Prologue: tiles 0..S-2 in flight; tile 0 landed everywhere; group 0
    // reads k-tile 0 (and issues tile S-1) so it can compute in phase 0.
    if (prologue_copies) {
#pragma unroll
        for (int t = 0; t < S - 1; ++t) issue(t);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((S - 2) * LPW) : "memory");  // tile 0 landed
    }
    asm volatile("s_barrier" ::: "memory");

    // Both groups execute 2*nk + 1 more barriers.  The compiler lays group
    // 1's branch out after group 0's, so a register group 1's loop reads on
    // entry would stay allocated through group 0's loop: group 0's first M
    // phase sits inside its own branch, and the prologue leaves no register
    // a group's loop reads before writing.  (The branch is uniform per wave,
    // and s_barrier counts waves, not program counters.)
    auto step0 = [&](auto next_stage, int s) {
        c_phase(s);
        asm volatile("s_barrier" ::: "memory");
        if (s + 1 < nk) m_phase(next_stage, s + 1);
        asm volatile("s_barrier" ::: "memory");
    };
    auto step1 = [&](auto stage, int s) {
        m_phase(stage, s);
        asm volatile("s_barrier" ::: "memory");
        c_phase(s);
        asm volatile("s_barrier" ::: "memory");
    };
    if (grp == 0) {
        m_phase(PingPongStage<0>{}, 0);
        asm volatile("s_barrier" ::: "memory");
        for (int s = 0; s < nk; s += S)
            pingpong_unrolled<S, 1>(s, nk, step0, std::make_integer_sequence<int, S>{});
    } else {
        asm volatile("s_barrier" ::: "memory");
        for (int s = 0; s < nk; s += S)
            pingpong_unrolled<S, 0>(s, nk, step1, std::make_integer_sequence<int, S>{});
    }
    // the copies past the last k-tile must land before the workgroup's LDS
    // is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// pingpong_schedule over a sequence of tiles, for a workgroup that stays on
// its CU from one tile to the next.  The caller has put the first tile's
// k-tile 0 in stage 0 and started the copies of its next tiles (as with
// prologue_copies false).  After each tile's last phase every wave waits for
// its copies (vmcnt(0)) and calls next_tile(), which returns false after the
// last tile; otherwise it must leave the next tile in the state the first one
// started in.  next_tile() may use barriers: both groups call it once per
// tile.  The tile loop sits inside each group's branch, so neither group's
// registers stay allocated through the other group's loop.
template <int S, class MPhase, class CPhase, class NextTile>
__device__ __forceinline__ void pingpong_schedule_tiles(int nk, int grp, MPhase&& m_phase, CPhase&& c_phase,
                                                        NextTile&& next_tile) {
    auto step0 = [&](auto next_stage, int s) {
        c_phase(s);
        asm volatile("s_barrier" ::: "memory");
        if (s + 1 < nk) m_phase(next_stage, s + 1);
        asm volatile("s_barrier" ::: "memory");
    };
    auto step1 = [&](auto stage, int s) {
        m_phase(stage, s);
        asm volatile("s_barrier" ::: "memory");
        c_phase(s);
        asm volatile("s_barrier" ::: "memory");
    };
    if (grp == 0) {
        do {
            asm volatile("s_barrier" ::: "memory");
            m_phase(PingPongStage<0>{}, 0);
            asm volatile("s_barrier" ::: "memory");
            for (int s = 0; s < nk; s += S)
                pingpong_unrolled<S, 1>(s, nk, step0, std::make_integer_sequence<int, S>{});
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } while (next_tile());
    } else {
        do {
            asm volatile("s_barrier" ::: "memory");
            asm volatile("s_barrier" ::: "memory");
            for (int s = 0; s < nk; s += S)
                pingpong_unrolled<S, 0>(s, nk, step1, std::make_integer_sequence<int, S>{});
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } while (next_tile());
    }
}

}  // namespace ch
