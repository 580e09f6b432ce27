// gemm_tiles.hpp -- LDS tile layouts and copy/read helpers for the bf16
// matrix-core GEMM on gfx950.
//
// Operands move global -> LDS with global_load_lds_dwordx4 (no VGPR staging):
// one instruction moves 16 bytes per lane, and lane l's bytes land at
// lds_base + 16*l, so a wave writes 1 KiB of LDS contiguously.  The LDS layout
// is therefore chosen by picking, per lane, WHICH 16-byte global chunk it
// fetches.  Two layouts, named by which index is contiguous in global memory:
//
//   KC ("k-contiguous", A stored M x K or B stored N x K):
//     LDS tile [R rows][BK], row pitch 2*BK bytes, CPR = BK/8 chunks per row.
//     Chunk c of row r is stored in slot kc_slot(r, c).  The MFMA operand
//     read (ds_read_b128) has 16 or 32 lanes read consecutive rows at one
//     logical chunk; the swizzle spreads the rows that share LDS banks.
//
//   MN ("m/n-contiguous", A stored K x M or B stored K x N):
//     LDS tile [BK][R], row pitch 2*R bytes, 16-byte chunk c of k-row kr in
//     slot mn_slot(kr, c).  The operand is read with ds_read_b64_tr_b16:
//     within each 16-lane group, result lane i, element j = the element
//     (i % 4) of source lane 4*j + i/4.  Source lane (4*j + q) points at
//     k-row kb + j, columns c0 + 4q .. c0 + 4q + 3, so result lane i receives
//     column c0 + i at k-rows kb .. kb + 3 -- exactly the k-contiguous
//     register layout the MFMA wants, with no register shuffles.
//
// LDS banks (gfx950, measured with the SQ_LDS_BANK_CONFLICT counter):
// ds_read_b64 and ds_read_b64_tr_b16 serve 32 lanes per cycle from 64 banks
// of 4 bytes, so the 32 lanes of a half-wave must cover 256 distinct bytes
// modulo 256.  ds_read_b128 takes 4 cycles per wave when conflict-free; a
// half-wave reading 16 B from rows 512 B apart pays a second pass.  Every
// swizzle below was checked pattern by pattern against that counter.
//
// v_mfma_f32_32x32x16_bf16 operand layout: lane l holds 8 bf16 of row
// (l % 32) at k = 8*(l / 32) .. +7 (both A and B, B indexed by column);
// the accumulator holds column (l % 32), rows 8*(v/4) + 4*(l/32) + v%4.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ch {
namespace tiles {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;
typedef __attribute__((address_space(3))) void lds_void;

// Slot of logical chunk c in KC row r (CPR chunks per row, ESZ-byte elements).
//   bf16, 4 chunks (BK = 32): the 16 x 16 x 32 read has a half-wave read rows
//     r0..r0+15 at chunks c, c+1; rows r and r+8 share banks, so bit 3 of the
//     row moves them two chunks apart (bit 4 does the same for the 32-row read).
//   bf16, 8 chunks (BK = 64) and f32: the 32-row read of the 32 x 32 MFMAs.
template <int CPR, int ESZ>
__device__ __forceinline__ int kc_slot(int r, int c) {
    static_assert(CPR == 4 || CPR == 8, "KC rows hold 4 or 8 chunks");
    if constexpr (CPR == 8) return c ^ ((r & 7) ^ ((r >> 3) & 1));
    else if constexpr (ESZ == 2) return c ^ (((r >> 3) & 1) << 1) ^ ((r >> 4) & 1);
    else return c ^ (((r >> 1) & 3) ^ ((r >> 3) & 1));
}
// Slot of chunk c in MN k-row kr, for the two MN read instructions:
//   bf16, ds_read_b64_tr_b16: a half-wave reads either 4 k-rows x 64 B
//     (32 x 32 x 16 operand) or k-rows kb..kb+3 and kb+8..kb+11 x 32 B
//     (16 x 16 x 32 operand).  XOR-ing 64 B blocks with kr & 3 separates the
//     4 rows of the first; flipping 32 B on bit 3 of kr separates the two row
//     quads of the second.  Needs 16 chunks (256 B) per k-row.
//   f32, ds_read_b32: the two half-waves read k-rows kr and kr + 4 at the same
//     128 B of columns; flipping 128 B on (kr >> 2) & 1 puts them in opposite
//     bank halves.
template <int ESZ>
__device__ __forceinline__ int mn_slot(int kr, int c) {
    static_assert(ESZ == 2 || ESZ == 4, "bf16 or f32 operands");
    if constexpr (ESZ == 2) return c ^ ((kr & 3) << 2) ^ (((kr >> 3) & 1) << 1);
    else return c ^ (((kr >> 2) & 1) << 3);
}

// Byte address (within the LDS window) of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const lds_void*)p;
}

// One global -> LDS copy instruction: 16 bytes per lane from sbase + voff
// (SGPR base, 32-bit per-lane byte offset) into LDS at lds_dst + 16*lane.
// Written as inline asm so the compiler does not see an outstanding LDS write:
// it would otherwise wait for every copy in flight before each ds_read, which
// serialises the copy of tile k+1 behind the math of tile k.  The caller
// orders copies and reads with s_waitcnt vmcnt + s_barrier.
// The LDS address goes in through an {m0} operand, so the compiler itself
// writes M0 and knows it did.
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds_dst) {
    asm volatile("global_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase), "{m0}"(lds_dst) : "memory");
}

// Per-lane byte offsets of this wave's NI/NW copy instructions for one
// operand tile, and the byte step that moves them to the next k-tile (added
// to the scalar base).
//   KC: tile [R rows][BK]; instruction q covers rows q*RPI .. +RPI-1.  The
//       offsets count from the tile's first row, which base_offset() puts in
//       the 64-bit scalar base: the 32-bit lane offsets then span R rows, so
//       an operand of any size is reached.
//   MN: tile [BK][R];      instruction q covers k-rows q*KPI .. +KPI-1, from
//       the tile's first column r0 (BK rows of the operand, whatever its size).
// Instruction q's LDS destination is tile_base + 1024*q.
template <bool KC, int R, int BK, int NW, int ESZ = 2>
struct TileCopy {
    static constexpr int EPC = 16 / ESZ;  // elements per 16-byte chunk
    static constexpr int NI = R * BK * ESZ / 1024, PER_WAVE = NI / NW;
    static_assert(NI % NW == 0, "tile copy must split evenly over the waves");
    uint32_t voff[PER_WAVE];

    __device__ __forceinline__ void init(int64_t ld, int r0, int wave, int lane) {
        if constexpr (KC) {
            constexpr int CPR = BK / EPC, RPI = 64 / CPR;
#pragma unroll
            for (int j = 0; j < PER_WAVE; ++j) {
                const int q = wave + NW * j;
                const int r = q * RPI + lane / CPR;
                const int c = kc_slot<CPR, ESZ>(r, lane % CPR);  // slot lane%CPR holds chunk c
                voff[j] = (uint32_t)(((int64_t)r * ld + EPC * c) * ESZ);
            }
        } else {
            constexpr int CPR = R / EPC, KPI = 64 / CPR;
            static_assert(CPR >= 16 && 64 % CPR == 0, "MN row too narrow for its swizzle");
#pragma unroll
            for (int j = 0; j < PER_WAVE; ++j) {
                const int q = wave + NW * j;
                const int kr = q * KPI + lane / CPR;
                const int c = mn_slot<ESZ>(kr, lane % CPR);
                voff[j] = (uint32_t)(((int64_t)kr * ld + r0 + EPC * c) * ESZ);
            }
        }
    }
    // Byte offset of the tile starting at row (KC) or column (MN) r0 from the
    // operand's base, to add to the scalar base (the MN column offset is in
    // the lane offsets already).
    static __device__ __forceinline__ int64_t base_offset(int64_t ld, int r0) {
        return KC ? (int64_t)r0 * ld * ESZ : 0;
    }
    // Byte step of the scalar base per k-tile.
    static __device__ __forceinline__ int64_t kstep(int64_t ld) {
        return KC ? (int64_t)BK * ESZ : (int64_t)BK * ld * ESZ;
    }

    __device__ __forceinline__ void issue(const char* sbase, uint32_t lds_tile, int wave) const {
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) dma16(sbase, voff[j], lds_tile + 1024u * (uint32_t)(wave + NW * j));
    }
};

// Copies for tiles that may cross the edge of the operand (M, N or K not a
// multiple of the tile).  A raw buffer load into LDS (buffer_load_dwordx4
// ... lds) range-checks voffset + soffset against the resource's byte count
// and writes zeros to LDS for a lane out of range; each lane whose 16-byte
// chunk lies outside the matrix is given an offset of kOutOfRange, so the
// tile arrives zero-padded without a padded copy of the operand.  Requires
// the operand's contiguous extent (K for a k-contiguous one, M or N
// otherwise) and its pitch to be multiples of the chunk (16 bytes), so a
// chunk is wholly inside or wholly outside, and the operand under 2 GiB, so
// kOutOfRange plus any k-tile step stays out of range.
constexpr uint32_t kOutOfRange = 0x80000000u;
typedef int v4i __attribute__((ext_vector_type(4)));

// Raw buffer resource over `bytes` bytes from `base` (stride 0; word 3 holds
// the 32-bit data format these loads need).
__device__ __forceinline__ v4i buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    v4i r;
    r[0] = (int)(uint32_t)a;
    r[1] = (int)((uint32_t)(a >> 32) & 0xFFFFu);
    r[2] = (int)bytes;
    r[3] = 0x00020000;
    return r;
}

// One buffer -> LDS copy instruction: 16 bytes per lane from the resource at
// voff + soff into LDS at lds_dst + 16*lane (inline asm for the reason dma16
// gives).
__device__ __forceinline__ void dma16_buf(v4i rsrc, uint32_t voff, uint32_t soff, uint32_t lds_dst) {
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" : : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_dst)
                 : "memory");
}

// TileCopy's instruction and lane layout, with per-lane masks: a chunk in a
// row (column) at or past `extent`, or at a k at or past K, loads zeros.
template <bool KC, int R, int BK, int NW, int ESZ = 2>
struct EdgeCopy {
    static constexpr int EPC = 16 / ESZ;
    static constexpr int NI = R * BK * ESZ / 1024, PER_WAVE = NI / NW;
    static_assert(NI % NW == 0, "tile copy must split evenly over the waves");
    uint32_t voff[PER_WAVE];  // byte offset from the operand base at k-tile 0, or kOutOfRange
    int k0[PER_WAVE];         // k of the lane's chunk (KC) or k-row (MN) at k-tile 0

    // r0: the tile's first row (KC) or column (MN); extent: the operand's rows
    // (KC) or columns (MN).
    __device__ __forceinline__ void init(int64_t ld, int r0, int extent, int wave, int lane) {
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) {
            const int q = wave + NW * j;
            if constexpr (KC) {
                constexpr int CPR = BK / EPC, RPI = 64 / CPR;
                const int r = q * RPI + lane / CPR;
                const int c = kc_slot<CPR, ESZ>(r, lane % CPR);
                voff[j] = r0 + r < extent ? (uint32_t)(((int64_t)(r0 + r) * ld + EPC * c) * ESZ) : kOutOfRange;
                k0[j] = EPC * c;
            } else {
                constexpr int CPR = R / EPC, KPI = 64 / CPR;
                static_assert(CPR >= 16 && 64 % CPR == 0, "MN row too narrow for its swizzle");
                const int kr = q * KPI + lane / CPR;
                const int c = mn_slot<ESZ>(kr, lane % CPR);
                voff[j] = r0 + EPC * c < extent ? (uint32_t)(((int64_t)kr * ld + r0 + EPC * c) * ESZ) : kOutOfRange;
                k0[j] = kr;
            }
        }
    }
    // Byte step of the scalar offset per k-tile.
    static __device__ __forceinline__ uint32_t kstep(int64_t ld) {
        return (uint32_t)(KC ? (int64_t)BK * ESZ : (int64_t)BK * ld * ESZ);
    }
    __device__ __forceinline__ void issue(v4i rsrc, int kt, int K, uint32_t soff, uint32_t lds_tile, int wave) const {
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j)
            dma16_buf(rsrc, k0[j] + kt * BK < K ? voff[j] : kOutOfRange, soff,
                      lds_tile + 1024u * (uint32_t)(wave + NW * j));
    }
};

// MFMA operand fragment (32 rows x 16 k) starting at tile row `row0`, k-step kk.
template <bool KC, int R, int BK>
__device__ __forceinline__ v8bf read_frag(const char* tile, int row0, int kk, int lane) {
    if constexpr (KC) {
        constexpr int CPR = BK / 8;
        const int r = row0 + (lane & 31);
        const int c = 2 * kk + (lane >> 5);
        return *reinterpret_cast<const v8bf*>(tile + r * (BK * 2) + kc_slot<CPR, 2>(r, c) * 16);
    } else {
        const int j = (lane & 15) >> 2, q = lane & 3;
        const int col = row0 + 16 * ((lane >> 4) & 1) + 4 * q;
        const int kb = kk * 16 + 8 * (lane >> 5) + j;
        v4s lo, hi;
        {
            const int kr = kb;
            const char* p = tile + kr * (R * 2) + mn_slot<2>(kr, col >> 3) * 16 + (col & 7) * 2;
            lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(const lds_void*)p);
        }
        {
            const int kr = kb + 4;
            const char* p = tile + kr * (R * 2) + mn_slot<2>(kr, col >> 3) * 16 + (col & 7) * 2;
            hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(const lds_void*)p);
        }
        typedef short v8s __attribute__((ext_vector_type(8)));
        v8s w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        return __builtin_bit_cast(v8bf, w);
    }
}

// MFMA operand fragment for v_mfma_f32_16x16x32_bf16: 16 rows starting at
// tile row `row0`, k-step kk of 32.  Lane l holds row (l % 16) at
// k = 32*kk + 8*(l / 16) .. +7 (A by row, B by column).
template <bool KC, int R, int BK>
__device__ __forceinline__ v8bf read_frag16(const char* tile, int row0, int kk, int lane) {
    if constexpr (KC) {
        constexpr int CPR = BK / 8;
        const int r = row0 + (lane & 15);
        const int c = 4 * kk + (lane >> 4);
        return *reinterpret_cast<const v8bf*>(tile + r * (BK * 2) + kc_slot<CPR, 2>(r, c) * 16);
    } else {
        // 16-lane group g reads k-rows 32*kk + 8*g + 4*h + (0..3) for h = 0, 1;
        // source lane 4*j + q points at k-row +j, columns row0 + 4*q .. +3.
        const int j = (lane & 15) >> 2, q = lane & 3;
        const int col = row0 + 4 * q;
        const int kb = kk * 32 + 8 * (lane >> 4) + j;
        v4s lo, hi;
        {
            const int kr = kb;
            const char* p = tile + kr * (R * 2) + mn_slot<2>(kr, col >> 3) * 16 + (col & 7) * 2;
            lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(const lds_void*)p);
        }
        {
            const int kr = kb + 4;
            const char* p = tile + kr * (R * 2) + mn_slot<2>(kr, col >> 3) * 16 + (col & 7) * 2;
            hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(const lds_void*)p);
        }
        typedef short v8s __attribute__((ext_vector_type(8)));
        v8s w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        return __builtin_bit_cast(v8bf, w);
    }
}

// The same 16 x 16 x 32 fragments, read at an address computed once.
// frag16_offset is the byte offset within a tile of the fragment
// read_frag16(tile, row0, 0, lane) reads (for an MN operand, its first k-row
// quad; the second quad is 4 k-rows on, with the same swizzle, since the
// quad's k-rows kb..kb+3 have kb % 8 <= 3).
template <bool KC, int R, int BK>
__device__ __forceinline__ uint32_t frag16_offset(int row0, int lane) {
    if constexpr (KC) {
        constexpr int CPR = BK / 8;
        const int r = row0 + (lane & 15), c = lane >> 4;
        return (uint32_t)(r * (BK * 2) + kc_slot<CPR, 2>(r, c) * 16);
    } else {
        const int j = (lane & 15) >> 2, q = lane & 3;
        const int col = row0 + 4 * q, kr = 8 * (lane >> 4) + j;
        return (uint32_t)(kr * (R * 2) + mn_slot<2>(kr, col >> 3) * 16 + (col & 7) * 2);
    }
}
typedef __attribute__((address_space(3))) v8bf lds_v8bf;
// KC fragment at LDS byte address a.
__device__ __forceinline__ v8bf read16_kc_at(uint32_t a) { return *(const lds_v8bf*)(uintptr_t)a; }
// MN fragment whose first k-row quad is at LDS byte address a (tile rows of R).
template <int R>
__device__ __forceinline__ v8bf read16_mn_at(uint32_t a) {
    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)a);
    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)(a + 4 * R * 2));
    typedef short v8s __attribute__((ext_vector_type(8)));
    const v8s w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(v8bf, w);
}

// Hide a value from the optimiser so it stays one register (the compiler
// would otherwise re-derive addresses from the lane id inside a loop).
template <class T>
__device__ __forceinline__ void opaque(T& v) { asm volatile("" : "+v"(v)); }

// f32 operand for four consecutive v_mfma_f32_32x32x2f32 steps over the
// 8-deep k-block kb (32 rows starting at tile row row0).  Lane-half h holds
// k = 8*kb + 4*h + s at step s (A and B agree, so the k-sum is complete).
typedef float v4f __attribute__((ext_vector_type(4)));
template <bool KC, int R, int BK>
__device__ __forceinline__ v4f read_frag_f32(const char* tile, int row0, int kb, int lane) {
    if constexpr (KC) {
        constexpr int CPR = BK / 4;
        const int r = row0 + (lane & 31);
        const int c = 2 * kb + (lane >> 5);
        return *reinterpret_cast<const v4f*>(tile + r * (BK * 4) + kc_slot<CPR, 4>(r, c) * 16);
    } else {
        const int col = row0 + (lane & 31);
        const int k0 = 8 * kb + 4 * (lane >> 5);
        v4f v;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kr = k0 + s;
            v[s] = *reinterpret_cast<const float*>(tile + kr * (R * 4) + mn_slot<4>(kr, col >> 2) * 16 + (col & 3) * 4);
        }
        return v;
    }
}

// Stores a wave's FM x FN blocks of 16 x 16 accumulators (v_mfma_f32_16x16x32
// layout: lane l holds column l%16, rows 4*(l/16) + v) to C at (r0, c0), ldc
// elements per row, as whole 128-byte rows.  Left as they are, a store
// instruction writes 16 columns (64 bytes) of 4 rows; v_permlane16_swap of
// blocks j and j+1 swaps the odd 16-lane rows of the first with the even rows
// of the second, after which lanes 0-31 hold 32 consecutive columns of one row
// and lanes 32-63 of another:
//   first  -> rows 8*(l/32) + v,     columns 32*(j/2) + l%32
//   second -> rows 8*(l/32) + 4 + v, columns 32*(j/2) + l%32
// Measured at 8192^3 bf16: every CU stores its 256 KiB at once at the end of a
// round of tiles, and whole lines drain ~25% faster than half lines.
//
// Values go in and out through __float_as_uint / __uint_as_float:
// __builtin_bit_cast of a vector subscript (acc[i][j][v], or the swap's
// result pair) reads element 0 whatever the index, in ROCm 7.2's clang.
//
// NT: non-temporal stores (`nt`), for a C larger than the MALL whose rows are
// whole 128-byte lines; the caller decides.
template <int FM, int FN, bool NT = false>
__device__ __forceinline__ void store_acc16_lines(float* __restrict__ C, int64_t ldc, int r0, int c0,
                                                  const v4f (&acc)[FM][FN], int lane) {
    static_assert(FN % 2 == 0, "blocks are paired along n");
    const int rl = 8 * (lane >> 5), cl = lane & 31;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; j += 2)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[i][j][v]),
                                                                __float_as_uint(acc[i][j + 1][v]), false, false);
                float* p = C + (int64_t)(r0 + i * 16 + rl + v) * ldc + (c0 + j * 16 + cl);
                if constexpr (NT) {
                    __builtin_nontemporal_store(__uint_as_float(s[0]), p);
                    __builtin_nontemporal_store(__uint_as_float(s[1]), p + 4 * ldc);
                } else {
                    p[0] = __uint_as_float(s[0]);
                    p[4 * ldc] = __uint_as_float(s[1]);
                }
            }
}
// The same stores, skipping elements at or past row M or column N (the
// guarded-edge kernels' last tiles), without branches: buffer stores over C
// from this wave's first row r0, sized to end at C's last element.  A row at
// or past M then lies past the resource's range (its offset is at least
// (M - r0) * ldc + c elements, and the range ends at (M - 1 - r0) * ldc + N,
// ldc >= N), so the hardware drops it; a column at or past N, which would
// land in the next row, gets an offset past the range (kOutOfRange).  The
// column test takes one value per pair of blocks and lane; testing every
// element's row and column instead kept 128 conditions live and spilled.
// Needs the block's rows of C (16 * FM of ldc floats) under 2 GiB.
template <int FM, int FN, bool NT = false>
__device__ __forceinline__ void store_acc16_lines_masked(float* __restrict__ C, int64_t ldc, int r0, int c0,
                                                         const v4f (&acc)[FM][FN], int lane, int M, int N) {
    constexpr int kAux = NT ? 2 : 0;  // cache policy: 2 = nt
    static_assert(FN % 2 == 0, "blocks are paired along n");
    if (r0 >= M) return;  // wave-uniform: the whole block lies past the last row
    const int64_t left = ((int64_t)(M - 1 - r0) * ldc + N) * 4;  // bytes from row r0 to C's last element
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        C + (int64_t)r0 * ldc, (short)0, (int)(left < 0x7FFFFFF0 ? left : 0x7FFFFFF0), 0x00020000);
    const int rl = 8 * (lane >> 5), cl = lane & 31;
    const uint32_t ld4 = (uint32_t)ldc * 4u;
#pragma unroll
    for (int j = 0; j < FN; j += 2) {
        const int c = c0 + j * 16 + cl;
        const bool col_ok = c < N;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[i][j][v]),
                                                                __float_as_uint(acc[i][j + 1][v]), false, false);
                const uint32_t o0 = (uint32_t)(i * 16 + rl + v) * ld4 + (uint32_t)c * 4u;
                __builtin_amdgcn_raw_buffer_store_b32(s[0], rsrc, (int)(col_ok ? o0 : kOutOfRange), 0, kAux);
                __builtin_amdgcn_raw_buffer_store_b32(s[1], rsrc, (int)(col_ok ? o0 + 4u * ld4 : kOutOfRange), 0,
                                                      kAux);
            }
    }
}

}  // namespace tiles
}  // namespace ch
