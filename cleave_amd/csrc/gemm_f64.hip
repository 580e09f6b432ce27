// gemm_f64.hip -- MatMul::matmul on Tensor<f64, ...> (stdlib/linalg/matrix.cleave:27-61
// with T = f64; Float covers f64, stdlib/num/num.cleave:50-51), single and
// batched, in all four trans_a / trans_b layouts, on the f64 matrix cores.
//
// v_mfma_f64_16x16x4f64: a wave multiplies a 16 x 4 block of A by a 4 x 16
// block of B into a 16 x 16 f64 accumulator, each lane supplying one double
// of each operand (A[l % 16][l / 16], B[l / 16][l % 16]) and holding four
// results, rows l / 16 + 4 v (v = 0..3) of column l % 16 (measured on
// gfx950: unlike the f32 16x16x4 form, whose lane holds four consecutive
// rows, the f64 form interleaves them).  On MI355X one such
// instruction keeps a SIMD's matrix core busy 64 cycles (FP64 matrix peak
// 78.6 TFLOP/s = 128 FLOP per CU-clock), so the kernel is matrix-core bound
// with little memory traffic per instruction: it needs enough independent
// accumulators per wave to issue back to back, not an elaborate copy
// pipeline.
//
// Tiles: a 256-thread workgroup computes a 128 x 128 block of C as 2 x 2 waves
// of 64 x 64 (4 x 4 MFMA tiles, 64 accumulator doubles per lane).  K advances
// 16 at a time through two LDS stages (2 x 32 KiB): the next tile's global
// loads are issued before the current tile's MFMAs and written to the other
// stage after them, one barrier per tile.  Both operands sit in LDS k-major
// ([k][m] and [k][n], rows padded to 144 doubles so the two 16-lane row
// groups of a half-wave read opposite bank halves, columns swizzled per k-row
// pair, lds_col).  Global loads are 16-byte
// vectors along whichever index is contiguous in memory when that extent is
// even, single doubles otherwise; out-of-range elements load as zero, so any
// M, N, K (K = 0 included: C = 0, the zero-filled accumulator of
// matrix.cleave:59) takes the same path.
#include "common.hpp"
#include "gemm_common.hpp"

namespace {

typedef double d4 __attribute__((ext_vector_type(4)));
typedef double d2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 16;
constexpr int kPitch = 144;  // LDS row pitch in doubles: 1152 B, 128 B mod 256

// LDS column of output index r in k-row k.  A k-contiguous operand is stored
// transposed: the 64 lanes of one store instruction cover 8 k-rows (8 lanes
// each) at 8 columns, and with a 144-double pitch every even k-row starts on
// the same bank, an 8-way conflict.  XOR-ing the column with 8 * ((k / 2) % 8)
// spreads those lanes over all 32 double slots of a 256-byte bank cycle (2
// passes for 512 bytes).  The XOR only moves 8-double groups, so the 16 lanes
// of an MFMA operand read still see one aligned 128-byte block per k-row, and
// k-rows 2j and 2j + 1 (one half-wave) share the XOR and stay 128 bytes apart
// modulo 256.  A 16-byte pair (r, r + 1), r even, stays adjacent.
__device__ __forceinline__ int lds_col(int k, int r) { return r ^ (((k >> 1) & 7) << 3); }

// Global -> register staging of one operand tile (R rows of the output
// dimension by BK along k).  KC: the operand is k-contiguous in memory (A
// stored M x K, B stored N x K); otherwise it is m/n-contiguous (A stored
// K x M, B stored K x N).  V doubles per load.
template <bool KC, int V>
struct TileLoad {
    static constexpr int kPer = (BM * BK) / (kThreads * V);  // loads per thread
    double v[kPer * V];

    // rows: extent of the output dimension (M or N); ld: row pitch in memory.
    __device__ __forceinline__ void load(const double* __restrict__ p, int64_t ld, int r0, int rows, int k0, int K) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = threadIdx.x + kThreads * i;
            int r, k;
            if constexpr (KC) {
                r = c / (BK / V);
                k = (c % (BK / V)) * V;
            } else {
                k = c / (BM / V);
                r = (c % (BM / V)) * V;
            }
            const bool ok = (r0 + r < rows) && (k0 + k < K);
            const int64_t off = KC ? (int64_t)(r0 + r) * ld + (k0 + k) : (int64_t)(k0 + k) * ld + (r0 + r);
            if constexpr (V == 2) {
                const d2 x = ok ? *reinterpret_cast<const d2*>(p + off) : d2{0.0, 0.0};
                v[2 * i] = x[0];
                v[2 * i + 1] = x[1];
            } else {
                v[i] = ok ? p[off] : 0.0;
            }
        }
    }

    // Into the k-major LDS stage s[BK][kPitch].
    __device__ __forceinline__ void store(double* s) const {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = threadIdx.x + kThreads * i;
            if constexpr (KC) {
                const int r = c / (BK / V), k = (c % (BK / V)) * V;
#pragma unroll
                for (int e = 0; e < V; ++e) s[(k + e) * kPitch + lds_col(k + e, r)] = v[V * i + e];
            } else {
                const int k = c / (BM / V), r = (c % (BM / V)) * V;
                if constexpr (V == 2)
                    *reinterpret_cast<d2*>(s + k * kPitch + lds_col(k, r)) = d2{v[2 * i], v[2 * i + 1]};
                else
                    s[k * kPitch + lds_col(k, r)] = v[i];
            }
        }
    }
};

// C[b] = op(A[b]) op(B[b]) for b < batch; a 1-D grid of tiles_m * tiles_n *
// batch workgroups in the XCD-aware order of block_coords.
template <bool TA, bool TB, int VA, int VB>
__global__ __launch_bounds__(kThreads) void gemm_f64_kernel(const double* __restrict__ A, const double* __restrict__ B,
                                                           double* __restrict__ C, int M, int N, int K, int batch,
                                                           int64_t sa, int64_t sb, int64_t sc) {
    __shared__ double As[2][BK * kPitch];
    __shared__ double Bs[2][BK * kPitch];

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int b, tm, tn;
    ch::block_coords(blockIdx.x, tiles_m, tiles_n, batch, b, tm, tn);
    A += (int64_t)b * sa;
    B += (int64_t)b * sb;
    C += (int64_t)b * sc;
    const int m0 = tm * BM, n0 = tn * BN;
    // A is k-contiguous unless stored K x M (trans_a); B is k-contiguous when stored N x K (trans_b).
    const int64_t lda = TA ? M : K, ldb = TB ? K : N;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int lr = lane & 15, lk = lane >> 4;

    d4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = d4{0.0, 0.0, 0.0, 0.0};

    TileLoad<!TA, VA> la;
    TileLoad<TB, VB> lb;
    const int tiles_k = (K + BK - 1) / BK;
    if (tiles_k > 0) {
        la.load(A, lda, m0, M, 0, K);
        lb.load(B, ldb, n0, N, 0, K);
        la.store(As[0]);
        lb.store(Bs[0]);
    }
    __syncthreads();
    for (int t = 0; t < tiles_k; ++t) {
        const int s = t & 1;
        const bool more = t + 1 < tiles_k;
        if (more) {
            la.load(A, lda, m0, M, (t + 1) * BK, K);
            lb.load(B, ldb, n0, N, (t + 1) * BK, K);
        }
        const double* as = As[s];
        const double* bs = Bs[s];
#pragma unroll
        for (int ks = 0; ks < BK; ks += 4) {
            double a[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = as[(ks + lk) * kPitch + lds_col(ks + lk, wm + 16 * i + lr)];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = bs[(ks + lk) * kPitch + lds_col(ks + lk, wn + 16 * j + lr)];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], bv[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            la.store(As[s ^ 1]);
            lb.store(Bs[s ^ 1]);
        }
        __syncthreads();
    }

    // acc[i][j][v] is C[m0 + wm + 16 i + lane / 16 + 4 v][n0 + wn + 16 j + lane % 16].
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = m0 + wm + 16 * i + lk + 4 * v;
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = n0 + wn + 16 * j + lr;
                if (n < N) C[(int64_t)m * N + n] = acc[i][j][v];
            }
        }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <bool TA, bool TB>
void launch_layout(const double* a, const double* b, double* c, int M, int N, int K, int batch, int64_t sa,
                   int64_t sb, int64_t sc, unsigned grid) {
    // 16-byte loads need every row of the contiguous index to start 16-byte aligned.
    const int contig_a = TA ? M : K, contig_b = TB ? K : N;
    const bool va = contig_a % 2 == 0 && aligned16(a) && sa % 2 == 0;
    const bool vb = contig_b % 2 == 0 && aligned16(b) && sb % 2 == 0;
    if (va && vb)
        gemm_f64_kernel<TA, TB, 2, 2><<<grid, kThreads, 0, ch::stream()>>>(a, b, c, M, N, K, batch, sa, sb, sc);
    else if (va)
        gemm_f64_kernel<TA, TB, 2, 1><<<grid, kThreads, 0, ch::stream()>>>(a, b, c, M, N, K, batch, sa, sb, sc);
    else if (vb)
        gemm_f64_kernel<TA, TB, 1, 2><<<grid, kThreads, 0, ch::stream()>>>(a, b, c, M, N, K, batch, sa, sb, sc);
    else
        gemm_f64_kernel<TA, TB, 1, 1><<<grid, kThreads, 0, ch::stream()>>>(a, b, c, M, N, K, batch, sa, sb, sc);
}

int32_t run_matmul_f64(const char* fn, const double* a, int64_t alen, const double* b, int64_t blen, double* c,
                       int64_t clen, int32_t batch, int32_t M, int32_t N, int32_t K, int32_t trans_a,
                       int32_t trans_b) {
    CH_REQUIRE(batch >= 1 && M >= 0 && N >= 0 && K >= 0, "%s: bad shape (batch %d, M %d, N %d, K %d)", fn, batch, M,
               N, K);
    CH_REQUIRE((trans_a == 0 || trans_a == 1) && (trans_b == 0 || trans_b == 1), "%s: trans flags must be 0 or 1",
               fn);
    const int64_t sa = (int64_t)M * K, sb = (int64_t)K * N, sc = (int64_t)M * N;
    const int64_t na = ch::count3(batch, M, K), nb = ch::count3(batch, K, N), nc = ch::count3(batch, M, N);
    CH_REQUIRE(na >= 0 && nb >= 0 && nc >= 0 && alen == na && blen == nb && clen == nc,
               "%s: lengths (%lld, %lld, %lld) do not match batch %d of %d x %d x %d", fn, (long long)alen,
               (long long)blen, (long long)clen, batch, M, N, K);
    if (clen == 0) return CLEAVE_HIP_OK;
    CH_REQUIRE(c && (K == 0 || (a && b)), "%s: null buffer", fn);
    CH_INIT_OR_RETURN();
    if (K > 0) {
        CH_DEVICE(fn, a, alen * 8);
        CH_DEVICE(fn, b, blen * 8);
    }
    CH_DEVICE(fn, c, clen * 8);
    const int64_t tiles = (int64_t)((M + BM - 1) / BM) * ((N + BN - 1) / BN) * batch;
    CH_REQUIRE(tiles <= 0x7FFFFFFF, "%s: %lld workgroups exceed the grid limit", fn, (long long)tiles);
    const unsigned grid = (unsigned)tiles;
    if (!trans_a && !trans_b) launch_layout<false, false>(a, b, c, M, N, K, batch, sa, sb, sc, grid);
    else if (!trans_a && trans_b) launch_layout<false, true>(a, b, c, M, N, K, batch, sa, sb, sc, grid);
    else if (trans_a && !trans_b) launch_layout<true, false>(a, b, c, M, N, K, batch, sa, sb, sc, grid);
    else launch_layout<true, true>(a, b, c, M, N, K, batch, sa, sb, sc, grid);
    CH_LAUNCHED(fn);
    return CLEAVE_HIP_OK;
}

}  // namespace

extern "C" {

int32_t cleave_hip_matmul_f64(const double* a, int64_t alen, const double* b, int64_t blen, double* c, int64_t clen,
                              int32_t M, int32_t N, int32_t K, int32_t trans_a, int32_t trans_b) {
    return run_matmul_f64("cleave_hip_matmul_f64", a, alen, b, blen, c, clen, 1, M, N, K, trans_a, trans_b);
}

int32_t cleave_hip_matmul_batched_f64(const double* a, int64_t alen, const double* b, int64_t blen, double* c,
                                      int64_t clen, int32_t batch, int32_t M, int32_t N, int32_t K, int32_t trans_a,
                                      int32_t trans_b) {
    return run_matmul_f64("cleave_hip_matmul_batched_f64", a, alen, b, blen, c, clen, batch, M, N, K, trans_a,
                          trans_b);
}

}  // extern "C"
