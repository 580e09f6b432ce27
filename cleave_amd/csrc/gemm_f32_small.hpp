// gemm_f32_small.hpp -- fp32 GEMM for small products on v_mfma_f32_32x32x2f32:
// one 32 x 32 tile of C per workgroup, its K range split over the
// workgroup's waves.
//
// A product with few tiles (config 1's 256^3 is 64 tiles of 32 x 32) leaves
// most CUs idle and each busy SIMD with a long serial MFMA chain: on 64 x 64
// tiles a wave of 256^3 runs 128 MFMAs one after the other.  Here wave w of
// the workgroup takes k in [64w, 64w + 64): 32 MFMAs, with all of its operand
// loads (8 k-blocks of 8) issued before the first one, so the product waits
// for memory once.  The W = K/64 partial tiles are added in LDS in wave order
// (wave 0 + wave 1 + ...), so the result does not depend on timing.
//
// Operand layout of the MFMA (as in gemm_f32_tiled.hpp): lane l feeds row
// (A) or column (B) l%32; over an 8-deep k-block, half-wave h = l/32 takes
// k = 4h + s at step s, for A and B alike, so all 8 k of the block are summed
// and a k-contiguous operand is one 16-byte load per lane per block.  An
// m/n-contiguous operand takes four 4-byte loads, each coalesced across the
// 32 lanes of a half-wave.
#pragma once

#include "gemm_common.hpp"

namespace ch {

struct F32Small {
    static constexpr int TILE = 32, KW = 64, KB = KW / 8, MAX_WAVES = 16;
    // Shapes this kernel takes without bounds checks: whole 32 x 32 tiles,
    // 64 k per wave and at most 16 waves, 16-byte aligned k-contiguous rows.
    static bool fits(int M, int N, int K, int64_t lda, int64_t ldb, bool akc, bool bkc) {
        return M % TILE == 0 && N % TILE == 0 && K % KW == 0 && K / KW <= MAX_WAVES &&
               (!akc || lda % 4 == 0) && (!bkc || ldb % 4 == 0);
    }
};

template <bool AKC, bool BKC>
__global__ __launch_bounds__(64 * F32Small::MAX_WAVES) void gemm_f32_small_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, int M, int N, int K,
    int64_t lda, int64_t ldb, int64_t strideA, int64_t strideB, int64_t strideC, int tiles_m, int tiles_n,
    int batch) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    typedef float v16f __attribute__((ext_vector_type(16)));
    constexpr int KB = F32Small::KB;
    __shared__ float red[F32Small::MAX_WAVES - 1][16][64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int waves = blockDim.x >> 6;
    const int r = lane & 31, h = lane >> 5;
    int bt, tm, tn;
    block_coords(blockIdx.x, tiles_m, tiles_n, batch, bt, tm, tn);
    const int m0 = tm * F32Small::TILE, n0 = tn * F32Small::TILE;
    A += (int64_t)bt * strideA;
    B += (int64_t)bt * strideB;
    C += (int64_t)bt * strideC;
    const int kw = wave * F32Small::KW;

    // Every operand load of this wave first: a[b][s] = A(m0 + r, kw + 8b + 4h + s),
    // bv[b][s] = B(kw + 8b + 4h + s, n0 + r).
    v4f a[KB], bv[KB];
#pragma unroll
    for (int b = 0; b < KB; ++b) {
        const int k = kw + 8 * b + 4 * h;
        if constexpr (AKC) {
            a[b] = *reinterpret_cast<const v4f*>(A + (int64_t)(m0 + r) * lda + k);
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) a[b][s] = A[(int64_t)(k + s) * lda + m0 + r];
        }
        if constexpr (BKC) {
            bv[b] = *reinterpret_cast<const v4f*>(B + (int64_t)(n0 + r) * ldb + k);
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) bv[b][s] = B[(int64_t)(k + s) * ldb + n0 + r];
        }
    }
    v16f acc = v16f{};
#pragma unroll
    for (int b = 0; b < KB; ++b)
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[b][s], bv[b][s], acc, 0, 0, 0);

    // Partial tiles of waves 1.. through LDS; wave 0 adds them in order.
    if (wave > 0) {
#pragma unroll
        for (int v = 0; v < 16; ++v) red[wave - 1][v][lane] = acc[v];
    }
    __syncthreads();
    if (wave != 0) return;
    for (int w = 1; w < waves; ++w) {
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[v] += red[w - 1][v][lane];
    }
    // 32 x 32 accumulator layout: lane holds column l%32, rows
    // 8*(v/4) + 4*(l/32) + v%4.
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = m0 + 8 * (v >> 2) + 4 * h + (v & 3);
        C[(int64_t)row * N + n0 + r] = acc[v];
    }
}

}  // namespace ch
