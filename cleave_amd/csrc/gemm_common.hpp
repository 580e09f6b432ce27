// gemm_common.hpp -- tile scheduling shared by the matrix-core kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace ch {

// MI355X dispatches consecutive workgroups round-robin over its 8 XCDs, each
// with a private L2.  Map the hardware order so XCD x receives a contiguous
// range [r*T/8, (r+1)*T/8) of logical tiles, r = xcd_range(x), then walk
// logical tiles in groups of GROUP_M tile-rows (column-major inside a group)
// so the tiles that run together share A row-panels and B column-panels.
constexpr int kXcds = 8;
constexpr int kGroupM = 8;

// The logical range XCD x takes.  With 8-row groups of 32 tile columns (8192
// outputs in 256 x 256 tiles), XCDs 2g and 2g+1 split group g's columns in
// halves.  Given in XCD order, every odd XCD took a right half; exchanging
// the two halves in every other pair (XCDs 2 and 3, 6 and 7) made the bf16
// 8192^3 product 1.5-1.8% faster (A.B 0.7232-0.7266 against 0.7368-0.7397
// ms, same box, three alternating runs; A.B^T and A^T.B^T 0.5-1%), and so
// did exchanging those of XCDs 4-7; exchanging all pairs, or reversing the
// order, changed nothing.  The f32 4096^3 headline was unchanged.
__device__ __forceinline__ int xcd_range(int x) { return x ^ ((x >> 1) & 1); }

__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm,
                                            int& tn) {
    const int total = tiles_m * tiles_n;
    int t = bid;
    if (total % kXcds == 0) t = xcd_range(bid % kXcds) * (total / kXcds) + bid / kXcds;
    const int per_group = kGroupM * tiles_n;
    const int group = t / per_group;
    const int first_m = group * kGroupM;
    const int gsize = min(tiles_m - first_m, kGroupM);
    const int in_group = t - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// Several products in one launch (a batch, or the K-slices of a split-K
// product): a 1-D grid of T*batch workgroups, T = tiles_m*tiles_n.  When the
// count divides by 8, XCD x takes the contiguous logical range
// [r*W/8, (r+1)*W/8), r = xcd_range(x), of (product, tile) pairs, so a
// product's operands are fetched into one or two L2s rather than all eight;
// inside a product the tiles are walked as in tile_coords.
__device__ __forceinline__ void block_coords(int bid, int tiles_m, int tiles_n, int batch, int& b,
                                             int& tm, int& tn) {
    const int T = tiles_m * tiles_n;
    const int W = T * batch;
    int g = bid;
    if (W % kXcds == 0) g = xcd_range(bid % kXcds) * (W / kXcds) + bid / kXcds;
    b = g / T;
    const int t = g - b * T;
    const int per_group = kGroupM * tiles_n;
    const int group = t / per_group;
    const int first_m = group * kGroupM;
    const int gsize = min(tiles_m - first_m, kGroupM);
    const int in_group = t - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// The guarded-edge kernels copy 16-byte chunks (Q elements) along each
// operand's contiguous extent, masking a chunk that starts past it.  A chunk
// that starts inside an m/n-contiguous row and runs past its extent reads
// columns that feed only entries of C outside the product, so that extent
// may be ragged when the memory the chunk reads exists: `padded` says every
// row holds its last chunk whole (an aligned copy, pitch at least the extent
// rounded up to Q).  A k-contiguous operand's extent is K and stays whole
// chunks: a chunk past K would multiply the other operand's zero k-rows by
// whatever it read, Inf and NaN included.
template <int Q>
__host__ __device__ constexpr int64_t chunk_up(int64_t x) {
    return (x + Q - 1) / Q * Q;
}
template <int Q>
inline bool edge_chunks(bool kc, int extent, int K, int64_t ld, bool padded) {
    if (ld % Q) return false;
    if (kc) return K % Q == 0;
    return extent % Q == 0 || (padded && ld >= chunk_up<Q>(extent));
}
// Bytes from an operand's base to the end of its last chunk: k-contiguous,
// `extent` rows of K; m/n-contiguous, K rows of `extent` (rounded up to a
// chunk).  The range of the operand's buffer resource.
template <int Q, int ESZ>
__host__ __device__ inline int64_t edge_bytes(bool kc, int extent, int K, int64_t ld) {
    return kc ? ((int64_t)(extent - 1) * ld + K) * ESZ : ((int64_t)(K - 1) * ld + chunk_up<Q>(extent)) * ESZ;
}

// Operands of the fused epilogues and operand transforms of the two GEMMs
// of the MLP step (mlp.hip); a plain GEMM passes {}.  The f32 kernels
// document what each MODE does with them.
struct MlpFuse {
    const float* w2 = nullptr;
    const float* d2 = nullptr;
    float* zpart = nullptr;
    float* dw2part = nullptr;
};

}  // namespace ch
