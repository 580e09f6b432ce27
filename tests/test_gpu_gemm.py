"""GEMM parity on the GPU, through the C ABI (cleave_hip_matmul_*).

Oracle: oracle/oracle.c's restated linalg.matmul loop (C = 0; C[i,j] += A[i,k]*B[k,j]).
Full-matrix comparison where the oracle finishes in seconds; at the BASELINE
sizes, sampled entries (each one an exact run of the reference loop) plus a
size-independent linearity property on every row: C 1 = A (B 1).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_gemm_close, sample_entries

pytestmark = pytest.mark.gpu


def _full_check(hip, oracle, A, B, ta, tb, what):
    a, b = hip.from_numpy(A), hip.from_numpy(B)
    c = hip.matmul(a, b, trans_a=ta, trans_b=tb)
    got = c.numpy()
    ref = oracle.matmul(A, B, trans_a=ta, trans_b=tb, threads=16)
    Af = np.abs(A.T if ta else A).astype(np.float64)
    Bf = np.abs(B.T if tb else B).astype(np.float64)
    K = Af.shape[1]
    return assert_gemm_close(got, ref, Af @ Bf, K, what)


def test_golden_vectors_exact(hip, golden):
    for case in golden["matmul"]:
        A = np.array(case["a"], np.float32)
        B = np.array(case["b"], np.float32)
        got = hip.matmul(hip.from_numpy(A), hip.from_numpy(B)).numpy()
        assert np.array_equal(got, np.array(case["c"], np.float32)), case["source"]


def test_matmul_against_ring_zero_is_exactly_zero(hip):
    # cleave/tests/mlir_lower.rs:2846-2858: the accumulator starts from a real zero.
    rng = np.random.default_rng(0)
    A = rng.standard_normal((256, 256)).astype(np.float32)
    c = hip.from_numpy(np.full((256, 256), np.nan, np.float32))  # garbage in the output buffer
    z = hip.zero((256, 256))
    hip.matmul(hip.from_numpy(A), z, out=c)
    assert np.array_equal(c.numpy(), np.zeros((256, 256), np.float32))


def test_config1_256_cube_uniform_seed0(hip, oracle):
    # A and B are the first and second 256^2 draws of the seed-0 uniform[-1,1)
    # stream: one fill of 2 x 256^2 values, split in two
    n = 256
    ab = hip.fill_uniform(hip.empty(2 * n * n), seed=0)
    a, b = ab.sub(0, (n, n)), ab.sub(n * n, (n, n))
    A, B = a.numpy(), b.numpy()
    # the device generator is the oracle's generator, bit for bit
    assert np.array_equal(np.concatenate([A.ravel(), B.ravel()]), oracle.uniform(2 * n * n, seed=0))
    got = hip.matmul(a, b).numpy()
    ref = oracle.matmul(A, B, threads=16)
    assert_gemm_close(got, ref, np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64), n, "256^3")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (2, 3, 2), (127, 129, 33), (300, 200, 17),
                                   (130, 257, 1000), (128, 128, 16), (256, 384, 48)])
def test_shapes_and_layouts(hip, oracle, M, N, K, ta, tb):
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    _full_check(hip, oracle, A, B, bool(ta), bool(tb), f"{M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (32, 32, 64), (96, 160, 320), (512, 512, 1024),
                                   (192, 320, 48), (64, 64, 16), (64, 128, 1040)])
def test_small_products(hip, oracle, M, N, K, ta, tb):
    # Products with at most one 32 x 32 tile per CU and K a multiple of 64 up
    # to 1024 run one tile per workgroup with K split over K/64 waves (config
    # 1's 256^3: 64 tiles, 4 waves; 512^2 x 1024: 16 waves); the others with
    # few 128 x 128 tiles run 64 x 64 tiles and a 16-deep ring, which K = 1040
    # wraps four times.
    rng = np.random.default_rng(M * 7 + N * 3 + K + 10 * ta + tb)
    A = rng.uniform(-1, 1, (K, M) if ta else (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (N, K) if tb else (K, N)).astype(np.float32)
    _full_check(hip, oracle, A, B, ta, tb, f"{M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_config2_4096_cube_sampled_and_linearity(hip, oracle, ta, tb):
    n = 4096
    a = hip.fill_normal(hip.empty((n, n)), seed=11)
    b = hip.fill_normal(hip.empty((n, n)), seed=12)
    c = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb))
    A, B, C = a.numpy(), b.numpy(), c.numpy()
    ii, jj = sample_entries(n, n, 512, seed=ta * 2 + tb)
    ref, absden = oracle.matmul_entries(A, B, n, n, n, ii, jj, trans_a=bool(ta), trans_b=bool(tb))
    assert_gemm_close(C[ii, jj], ref, absden, n, f"4096^3 ta={ta} tb={tb}")
    # every row: C 1 = A (B 1), in float64, within the same normalised bound
    Ad = (A.T if ta else A).astype(np.float64)
    Bd = (B.T if tb else B).astype(np.float64)
    rows = Ad @ Bd.sum(axis=1)
    den = np.abs(Ad) @ np.abs(Bd).sum(axis=1)
    assert np.max(np.abs(C.astype(np.float64).sum(axis=1) - rows) / den) <= 1e-5 * np.sqrt(n)
    # every column: 1^T C = (1^T A) B, in float64, within the same bound; with
    # the row identity, an entry stored in the wrong column of its row (or
    # the wrong row of its column) moves a sum
    cols = Ad.sum(axis=0) @ Bd
    cden = np.abs(Ad).sum(axis=0) @ np.abs(Bd)
    assert np.max(np.abs(C.astype(np.float64).sum(axis=0) - cols) / cden) <= 1e-5 * np.sqrt(n)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_config2_4096_cube_every_entry(hip, oracle, ta, tb):
    # Config 2 in full: every entry of the 4096^3 product (A·B, A·Bᵀ, Aᵀ·B)
    # against the reference loop.  The oracle's A·Bᵀ loop, whose operands are
    # both k-contiguous, runs several times faster than its A·B loop and gives
    # the same bits -- each entry is the same k-ascending chain of unfused
    # mul/add however the operands are stored (test_oracle.py pins that) --
    # so the reference for every layout runs on k-contiguous copies.
    n = 4096
    a = hip.fill_normal(hip.empty((n, n)), seed=61 + 2 * ta + tb)
    b = hip.fill_normal(hip.empty((n, n)), seed=71 + 2 * ta + tb)
    c = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    A, B = a.numpy(), b.numpy()
    Ak = np.ascontiguousarray(A.T) if ta else A  # M x K
    Bk = B if tb else np.ascontiguousarray(B.T)  # N x K
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    assert_gemm_close(c, ref, den, n, f"4096^3 every entry ta={ta} tb={tb}")


def test_deterministic(hip):
    n = 1024
    a = hip.fill_normal(hip.empty((n, n)), seed=3)
    b = hip.fill_normal(hip.empty((n, n)), seed=4)
    c1 = hip.matmul(a, b).numpy()
    c2 = hip.matmul(a, b).numpy()
    assert np.array_equal(c1, c2)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_batched_f32_small_products(hip, oracle, ta, tb):
    # 6 products of 64 x 96 x 192: 36 tiles of 32 x 32 over the batch, K split
    # over 3 waves; every entry of every product against the oracle.
    bsz, M, N, K = 6, 64, 96, 192
    rng = np.random.default_rng(90 + 2 * ta + tb)
    A = rng.uniform(-1, 1, (bsz, K, M) if ta else (bsz, M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (bsz, N, K) if tb else (bsz, K, N)).astype(np.float32)
    got = hip.matmul_batched(hip.from_numpy(A), hip.from_numpy(B), trans_a=bool(ta), trans_b=bool(tb)).numpy()
    for i in range(bsz):
        ref = oracle.matmul(A[i], B[i], trans_a=bool(ta), trans_b=bool(tb))
        den = np.abs(A[i].T if ta else A[i]).astype(np.float64) @ np.abs(B[i].T if tb else B[i]).astype(np.float64)
        assert_gemm_close(got[i], ref, den, K, f"batched small f32 ta={ta} tb={tb} #{i}")


def test_batched_f32(hip, oracle):
    rng = np.random.default_rng(5)
    bsz, M, N, K = 5, 96, 130, 70
    A = rng.standard_normal((bsz, M, K)).astype(np.float32)
    B = rng.standard_normal((bsz, K, N)).astype(np.float32)
    got = hip.matmul_batched(hip.from_numpy(A), hip.from_numpy(B)).numpy()
    for i in range(bsz):
        ref = oracle.matmul(A[i], B[i])
        assert_gemm_close(got[i], ref, np.abs(A[i]).astype(np.float64) @ np.abs(B[i]).astype(np.float64), K,
                          f"batch {i}")


# ---- bf16 in, f32 accumulate -------------------------------------------------------

def test_bf16_golden_vectors_exact(hip, golden, oracle):
    for case in golden["matmul"]:
        A = oracle.to_bf16(np.array(case["a"], np.float32))
        B = oracle.to_bf16(np.array(case["b"], np.float32))
        got = hip.matmul(hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16")).numpy()
        assert np.array_equal(got, np.array(case["c"], np.float32)), case["source"]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [
    (1, 1, 1), (3, 5, 7), (129, 131, 40), (200, 300, 100),  # general kernel (ragged)
    (256, 128, 64), (384, 128, 192),                         # 128 x 128 x 64 tiled kernel
    (256, 256, 64), (512, 768, 384), (768, 512, 640),        # 256 x 256 x 64 tiled kernel
])
def test_bf16_shapes_and_layouts(hip, oracle, M, N, K, ta, tb):
    rng = np.random.default_rng(M + N + K)
    A32 = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B32 = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    A, B = oracle.to_bf16(A32), oracle.to_bf16(B32)
    got = hip.matmul(hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16"), trans_a=bool(ta),
                     trans_b=bool(tb)).numpy()
    Au = oracle.bf16_to_f32(A).reshape(A.shape)
    Bu = oracle.bf16_to_f32(B).reshape(B.shape)
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb))
    Ad = np.abs(Au.T if ta else Au).astype(np.float64)
    Bd = np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, Ad @ Bd, K, f"bf16 {M}x{N}x{K}")


def test_bf16_batched_tiled_every_entry(hip, oracle):
    # batch entries back to back through the 256 x 256 x 64 kernel: each one
    # checked in full against the sequential loop on the upcast values
    rng = np.random.default_rng(9)
    bsz, M, N, K = 3, 256, 512, 128
    A = oracle.to_bf16(rng.standard_normal((bsz, M, K)).astype(np.float32))
    B = oracle.to_bf16(rng.standard_normal((bsz, K, N)).astype(np.float32))
    got = hip.matmul_batched(hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16")).numpy()
    for i in range(bsz):
        Au = oracle.bf16_to_f32(A[i]).reshape(M, K)
        Bu = oracle.bf16_to_f32(B[i]).reshape(K, N)
        ref = oracle.matmul(Au, Bu, threads=8)
        den = np.abs(Au).astype(np.float64) @ np.abs(Bu).astype(np.float64)
        assert_gemm_close(got[i], ref, den, K, f"batched bf16 entry {i}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("bsz,M,N,K", [(4, 256, 256, 128), (64, 512, 512, 512), (80, 512, 512, 1024)])
def test_bf16_batched_every_layout(hip, oracle, bsz, M, N, K, ta, tb):
    # The batched halves of the product rule (stdlib/linalg/matrix.cleave:24):
    # each batch entry stored K x M (trans_a) or N x K (trans_b).  4 x 256^2 runs
    # the 128 x 128 tiled kernel; 64 x 512^3 (config 5) the 256 x 256 one;
    # 80 x 512^2 x 1024 (320 tiles) a ping-pong kernel, whose paired-copy form
    # keeps 256 workgroups, 64 of them taking a tile of a second batch entry.
    # Three entries of each are checked in full against the oracle.
    a = hip.to_bf16(hip.fill_normal(hip.empty((bsz, K, M) if ta else (bsz, M, K)), seed=131 + 2 * ta + tb,
                                    std=0.02))
    b = hip.to_bf16(hip.fill_normal(hip.empty((bsz, N, K) if tb else (bsz, K, N)), seed=141 + 2 * ta + tb,
                                    std=0.02))
    got = hip.matmul_batched(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    A, B = a.numpy(), b.numpy()
    for i in (0, bsz // 2 + 1, bsz - 1):
        Au = oracle.bf16_to_f32(A[i]).reshape(A.shape[1:])
        Bu = oracle.bf16_to_f32(B[i]).reshape(B.shape[1:])
        ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb), threads=16)
        den = (np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64))
        assert_gemm_close(got[i], ref, den, K, f"batched bf16 ta={ta} tb={tb} #{i}")


def test_bf16_tiled_output_is_overwritten_and_deterministic(hip):
    # C is written, not accumulated into (the reference zero-fills its
    # accumulator), and two runs agree bit for bit
    n = 512
    a = hip.to_bf16(hip.fill_normal(hip.empty((n, n)), seed=5, std=0.02))
    b = hip.to_bf16(hip.fill_normal(hip.empty((n, n)), seed=6, std=0.02))
    c = hip.fill_normal(hip.empty((n, n)), seed=7)
    first = hip.matmul(a, b, out=c).numpy()
    second = hip.matmul(a, b, out=c).numpy()
    assert np.array_equal(first, second)


def test_config5_bf16_8192_cube(hip, oracle):
    n = 8192
    a32 = hip.fill_normal(hip.empty((n, n)), seed=21, std=0.02)
    b32 = hip.fill_normal(hip.empty((n, n)), seed=22, std=0.02)
    a, b = hip.to_bf16(a32), hip.to_bf16(b32)
    # the device cast is RNE, bit for bit with the oracle's
    A32 = a32.numpy()
    A = a.numpy()
    assert np.array_equal(A[:64], oracle.to_bf16(A32[:64]))
    del a32, b32
    c = hip.matmul(a, b)
    B = b.numpy()
    C = c.numpy()
    ii, jj = sample_entries(n, n, 384, seed=5)
    ref, absden = oracle.matmul_entries(A, B, n, n, n, ii, jj, bf16=True)
    assert_gemm_close(C[ii, jj], ref, absden, n, "bf16 8192^3")
    # the stated bf16 tolerance: rel <= 1e-2 against the f32 loop on upcast values
    assert np.all(np.abs(C[ii, jj] - ref) <= 1e-2 * np.abs(ref) + 1e-2 * absden / np.sqrt(n))
    Ad = oracle.bf16_to_f32(A).reshape(n, n).astype(np.float64)
    Bd = oracle.bf16_to_f32(B).reshape(n, n).astype(np.float64)
    rows = Ad @ Bd.sum(axis=1)
    den = np.abs(Ad) @ np.abs(Bd).sum(axis=1)
    assert np.max(np.abs(C.astype(np.float64).sum(axis=1) - rows) / den) <= 1e-5 * np.sqrt(n)
    del Ad, Bd
    # Every entry: the oracle's f32 loop on the upcast values, run as its
    # k-contiguous (A·Bᵀ) loop on a transposed copy of B, which gives the same
    # bits as its A·B loop (pinned in test_oracle.py) several times faster.
    Au = oracle.bf16_to_f32(A).reshape(n, n)
    Bt = np.ascontiguousarray(oracle.bf16_to_f32(B).reshape(n, n).T)
    full = oracle.matmul(Au, Bt, trans_b=True, threads=16)
    den = np.abs(Au) @ np.abs(Bt).T  # f32 is ample for a tolerance's scale
    assert_gemm_close(C, full, den, n, "bf16 8192^3 every entry")
    assert np.all(np.abs(C - full) <= 1e-2 * np.abs(full) + 1e-2 * den / np.sqrt(n))


def test_config5_batched_bf16_64x512(hip, oracle):
    bsz, n = 64, 512
    a32 = hip.fill_normal(hip.empty((bsz, n, n)), seed=31, std=0.02)
    b32 = hip.fill_normal(hip.empty((bsz, n, n)), seed=32, std=0.02)
    a, b = hip.to_bf16(a32), hip.to_bf16(b32)
    c = hip.matmul_batched(a, b)
    A, B, C = a.numpy(), b.numpy(), c.numpy()
    for i in [0, 1, 17, 63]:
        ii, jj = sample_entries(n, n, 128, seed=i)
        ref, absden = oracle.matmul_entries(A[i], B[i], n, n, n, ii, jj, bf16=True)
        assert_gemm_close(C[i][ii, jj], ref, absden, n, f"batched bf16 #{i}")
    # every entry of every product (the oracle's k-contiguous loop on a
    # transposed copy of B: the same bits as its A·B loop)
    for i in range(bsz):
        Au = oracle.bf16_to_f32(A[i]).reshape(n, n)
        Bt = np.ascontiguousarray(oracle.bf16_to_f32(B[i]).reshape(n, n).T)
        ref = oracle.matmul(Au, Bt, trans_b=True, threads=16)
        den = np.abs(Au).astype(np.float64) @ np.abs(Bt).astype(np.float64).T
        assert_gemm_close(C[i], ref, den, n, f"batch {i} every entry")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_big_tile_path_every_layout(hip, oracle, dtype, ta, tb):
    # 4096 x 4096 outputs give the 256 x 256 tiled kernels a tile per CU, so
    # every layout of that path runs here; a short K keeps the oracle cheap
    M = N = 4096
    K = 128
    a32 = hip.fill_normal(hip.empty((K, M) if ta else (M, K)), seed=61 + 2 * ta + tb)
    b32 = hip.fill_normal(hip.empty((N, K) if tb else (K, N)), seed=71 + 2 * ta + tb)
    if dtype == "bf16":
        a, b = hip.to_bf16(a32), hip.to_bf16(b32)
    else:
        a, b = a32, b32
    c = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    A, B = a.numpy(), b.numpy()
    ii, jj = sample_entries(M, N, 1024, seed=5 + ta + 2 * tb)
    ref, absden = oracle.matmul_entries(A, B, M, N, K, ii, jj, trans_a=bool(ta), trans_b=bool(tb),
                                        bf16=(dtype == "bf16"))
    assert_gemm_close(c[ii, jj], ref, absden, K, f"{dtype} big tile ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bf16_pingpong_every_layout(hip, oracle, ta, tb):
    # 8192 x 8192 outputs are four rounds of 256 x 256 tiles, which take the
    # bf16 ping-pong kernel at any K; K = 96 is three of its k-tiles
    M = N = 8192
    K = 96
    a = hip.to_bf16(hip.fill_normal(hip.empty((K, M) if ta else (M, K)), seed=31 + 2 * ta + tb, std=0.02))
    b = hip.to_bf16(hip.fill_normal(hip.empty((N, K) if tb else (K, N)), seed=41 + 2 * ta + tb, std=0.02))
    c = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    A, B = a.numpy(), b.numpy()
    ii, jj = sample_entries(M, N, 1024, seed=7 + ta + 2 * tb)
    ref, absden = oracle.matmul_entries(A, B, M, N, K, ii, jj, trans_a=bool(ta), trans_b=bool(tb), bf16=True)
    assert_gemm_close(c[ii, jj], ref, absden, K, f"bf16 ping-pong ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("K", [16, 48, 80])
def test_f32_pingpong_short_k(hip, oracle, K, ta, tb):
    # 4096 x 4096 outputs: the f32 ping-pong kernel of the headline, one tile
    # per CU.  1, 3 and 5 k-tiles of 16: the ring of four LDS stages is never
    # filled, or wraps once, so the copies past the last k-tile (clamped to
    # it) and the prologue's two tiles are all exercised.  EVERY entry of C is
    # compared with the oracle's sequential loop: an epilogue that stores a
    # value in the wrong column of its row would keep every row sum.
    M = N = 4096
    a = hip.fill_normal(hip.empty((K, M) if ta else (M, K)), seed=81 + K + 2 * ta + tb)
    b = hip.fill_normal(hip.empty((N, K) if tb else (K, N)), seed=91 + K + 2 * ta + tb)
    c = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    A, B = a.numpy(), b.numpy()
    ref = oracle.matmul(A, B, trans_a=bool(ta), trans_b=bool(tb), threads=16)
    Aa = np.abs(A.T if ta else A).astype(np.float64)
    Ba = np.abs(B.T if tb else B).astype(np.float64)
    assert_gemm_close(c, ref, Aa @ Ba, K, f"f32 short K={K} ta={ta} tb={tb}, every entry")
    # every row sum, in float64
    Ad = (A.T if ta else A).astype(np.float64)
    Bd = (B.T if tb else B).astype(np.float64)
    rows = Ad @ Bd.sum(axis=1)
    den = np.abs(Ad) @ np.abs(Bd).sum(axis=1)
    assert np.max(np.abs(c.astype(np.float64).sum(axis=1) - rows) / den) <= 1e-5 * np.sqrt(K)


def test_f32_batched_through_pingpong(hip, oracle):
    # 16 products of 1024 x 1024 (16 tiles of 256 x 256 each, 256 in all):
    # the batch strides go through the ping-pong kernel
    bsz, M, N, K = 16, 1024, 1024, 64
    rng = np.random.default_rng(17)
    A = rng.standard_normal((bsz, M, K)).astype(np.float32)
    B = rng.standard_normal((bsz, K, N)).astype(np.float32)
    got = hip.matmul_batched(hip.from_numpy(A), hip.from_numpy(B)).numpy()
    for i in (0, 7, 15):
        ii, jj = sample_entries(M, N, 256, seed=i)
        ref, absden = oracle.matmul_entries(A[i], B[i], M, N, K, ii, jj)
        assert_gemm_close(got[i][ii, jj], ref, absden, K, f"batched f32 entry {i}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(4096, 8192, 320), (3840, 5120, 320), (4096, 8192, 128), (3840, 5120, 128)])
def test_bf16_pingpong_every_entry(hip, oracle, M, N, K, ta, tb):
    # Two rounds of 256 x 256 tiles (512, or 300: 44 workgroups of 256 take a
    # second tile) with K = 320 go to a ping-pong kernel (the paired-copy one,
    # which keeps one workgroup per CU looping over its tiles, for A·B, A·Bᵀ
    # and Aᵀ·Bᵀ).  Its epilogue swaps 16-lane rows between accumulator blocks
    # to store whole 128-byte rows; every entry of C is checked, since a value
    # stored in the wrong column of its row would keep the row sums the
    # sampled tests also check.  With K = 128 the same shapes go to 128 x 128
    # tiles, two workgroups per CU (a short K over several rounds).
    rng = np.random.default_rng(40 + 2 * ta + tb + M)
    A = oracle.to_bf16(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = oracle.to_bf16(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
    got = hip.matmul(hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16"), trans_a=bool(ta),
                     trans_b=bool(tb)).numpy()
    Au = oracle.bf16_to_f32(A).reshape(A.shape)
    Bu = oracle.bf16_to_f32(B).reshape(B.shape)
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb), threads=16)
    Ad = np.abs(Au.T if ta else Au).astype(np.float64)
    Bd = np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, Ad @ Bd, K, f"bf16 ping-pong every entry ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("K", [32, 64, 128, 160, 192, 352, 384, 832])
def test_bf16_pingpong_ring_depths(hip, oracle, K, ta, tb):
    # 4096 x 8192 outputs are two rounds of 256 x 256 tiles.  From K = 320
    # the dispatch gives them to a ping-pong kernel: with K a multiple of 64,
    # A·B and Aᵀ·Bᵀ take the kernel that copies the k-contiguous operand in
    # pairs of k-tiles (a ring of 3 pairs beside a ring of 4 single k-tiles):
    # K = 384 and 832 are 6 and 13 pairs (filled, wrapping).  The other K, and
    # the other layouts, take the kernel with a ring of five single k-tiles:
    # 1, 5 and 11 k-tiles for K = 32, 160, 352.  K = 64, 128 and 192 (a short
    # K over several rounds) go to 128 x 128 tiles, two workgroups per CU,
    # with 1 - 3 k-tiles of 64.
    M, N = 4096, 8192
    a = hip.to_bf16(hip.fill_normal(hip.empty((K, M) if ta else (M, K)), seed=101 + K + 2 * ta + tb, std=0.02))
    b = hip.to_bf16(hip.fill_normal(hip.empty((N, K) if tb else (K, N)), seed=111 + K + 2 * ta + tb, std=0.02))
    c = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    A, B = a.numpy(), b.numpy()
    ii, jj = sample_entries(M, N, 1024, seed=3 * K + ta + 2 * tb)
    ref, absden = oracle.matmul_entries(A, B, M, N, K, ii, jj, trans_a=bool(ta), trans_b=bool(tb), bf16=True)
    assert_gemm_close(c[ii, jj], ref, absden, K, f"bf16 ring K={K} ta={ta} tb={tb}")
    # every row sum, in float64 on the upcast operands
    Ad = oracle.bf16_to_f32(A).reshape(A.shape).astype(np.float64)
    Bd = oracle.bf16_to_f32(B).reshape(B.shape).astype(np.float64)
    Ad = Ad.T if ta else Ad
    Bd = Bd.T if tb else Bd
    rows = Ad @ Bd.sum(axis=1)
    den = np.abs(Ad) @ np.abs(Bd).sum(axis=1)
    assert np.max(np.abs(c.astype(np.float64).sum(axis=1) - rows) / den) <= 1e-5 * np.sqrt(K)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_infinities_and_nans_propagate_like_the_loop(hip, oracle, dtype):
    # The reference loop is IEEE arithmetic without reassociation, so an Inf
    # or NaN in an operand reaches exactly the entries whose k-sum touches it:
    # NaN stays NaN, an Inf with finite partners stays an Inf of the product's
    # sign, and Inf meeting -Inf in one sum (or Inf times 0) is NaN.  The
    # sum's order does not change any of that, so float64 products pin it.
    # 4096 x 4096 outputs take the 256 x 256 kernels (f32 ping-pong, bf16 tiled).
    M = N = 4096
    K = 64
    rng = np.random.default_rng(23)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    A[3, 5] = np.inf
    A[7, 9] = np.nan
    A[11, 2] = -np.inf
    A[11, 3] = np.inf           # row 11: -Inf and +Inf, NaN or an Inf by the signs of their partners
    B[10, 20] = -np.inf
    B[5, 600] = 0.0             # A[3,5] = Inf times 0 -> NaN at (3, 600)
    B[33, 4000] = np.nan
    if dtype == "bf16":
        a = hip.from_numpy(oracle.to_bf16(A))
        b = hip.from_numpy(oracle.to_bf16(B))
        Au, Bu = oracle.bf16_to_f32(a.numpy()), oracle.bf16_to_f32(b.numpy())
    else:
        a, b = hip.from_numpy(A), hip.from_numpy(B)
        Au, Bu = A, B
    got = hip.matmul(a, b).numpy()
    rows = [3, 7, 11, 100]
    cols = [20, 600, 4000, 17]
    with np.errstate(invalid="ignore", over="ignore"):
        ref_rows = Au[rows].astype(np.float64) @ Bu.astype(np.float64)
        ref_cols = Au.astype(np.float64) @ Bu[:, cols].astype(np.float64)
    for g, r in ((got[rows], ref_rows), (got[:, cols], ref_cols)):
        assert np.array_equal(np.isnan(g), np.isnan(r))
        assert np.array_equal(np.isposinf(g), np.isposinf(r))
        assert np.array_equal(np.isneginf(g), np.isneginf(r))
    # the special entries are where they should be, and nowhere else
    assert np.isnan(got[7]).all() and np.isnan(got[:, 4000]).all()
    assert np.isnan(got[3, 600])
    clean = np.ones((M, N), bool)
    clean[[3, 7, 11]] = False
    clean[:, [20, 4000]] = False
    assert np.isfinite(got[clean]).all()


@pytest.mark.parametrize("dtype,off", [("f32", 1), ("f32", 2), ("bf16", 1), ("bf16", 4)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_misaligned_operand_views(hip, oracle, dtype, off, ta, tb):
    # Operands starting `off` elements into their buffers (4 or 8 bytes for
    # f32, 2 or 8 bytes for bf16) at a shape the fast kernels would otherwise
    # take (multiples of 128 and 256): the launchers check the base pointers'
    # 16-byte alignment and send such views to the guarded general kernel.
    M, N, K = 256, 256, 128
    rng = np.random.default_rng(7 * off + 2 * ta + tb)
    A32 = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B32 = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    if dtype == "bf16":
        A, B = oracle.to_bf16(A32), oracle.to_bf16(B32)
        Au, Bu = oracle.bf16_to_f32(A).reshape(A.shape), oracle.bf16_to_f32(B).reshape(B.shape)
    else:
        A, B, Au, Bu = A32, B32, A32, B32
    abuf = hip.from_numpy(np.concatenate([np.zeros(off, A.dtype), A.ravel()]), dtype)
    bbuf = hip.from_numpy(np.concatenate([np.zeros(off, B.dtype), B.ravel()]), dtype)
    a, b = abuf.sub(off, A.shape), bbuf.sub(off, B.shape)
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb))
    den = np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, den, K, f"{dtype} view at +{off} ta={ta} tb={tb}")


def _operands(oracle, dtype, M, N, K, ta, tb, seed, batch=None):
    rng = np.random.default_rng(seed)
    lead = () if batch is None else (batch,)
    A32 = rng.standard_normal(lead + ((K, M) if ta else (M, K))).astype(np.float32)
    B32 = rng.standard_normal(lead + ((N, K) if tb else (K, N))).astype(np.float32)
    if dtype == "bf16":
        A, B = oracle.to_bf16(A32), oracle.to_bf16(B32)
        return A, B, oracle.bf16_to_f32(A).reshape(A.shape), oracle.bf16_to_f32(B).reshape(B.shape)
    return A32, B32, A32, B32


# Ragged shapes past the general kernel: every dimension ragged, K alone
# ragged, M alone ragged, N alone ragged.  They run the guarded-edge kernels
# (below) on the operands in place when each operand's rows are whole 16-byte
# chunks, else on aligned copies of the operands that are not (C in place
# either way); the zero-padded route (padded copies of the operands, the
# valid corner of C copied out) takes f32 with K past 512 over more than
# four 64 x 64 tiles per CU.
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(1000, 1000, 1000), (640, 2048, 520), (1031, 768, 512), (2048, 1100, 256)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_padded_ragged_every_entry(hip, oracle, dtype, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=M + 3 * N + 7 * K + 2 * ta + tb)
    got = hip.matmul(hip.from_numpy(A, dtype), hip.from_numpy(B, dtype), trans_a=bool(ta),
                     trans_b=bool(tb)).numpy()
    assert got.shape == (M, N)
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb), threads=16)
    den = np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, den, K, f"padded {dtype} {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_padded_large_ragged_every_entry(hip, oracle, dtype):
    # 3000 x 5000 x 2000: M, N and K all ragged (bf16 on the 256 x 256
    # kernels with guarded edges, f32 on the 128 x 128 tiled kernel's); every
    # entry against the loop (its A·Bᵀ form on a transposed copy of B, bit
    # for bit its A·B loop)
    M, N, K = 3000, 5000, 2000
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, 0, 0, seed=41)
    got = hip.matmul(hip.from_numpy(A, dtype), hip.from_numpy(B, dtype)).numpy()
    Bt = np.ascontiguousarray(Bu.T)
    ref = oracle.matmul(Au, Bt, trans_b=True, threads=16)
    den = np.abs(Au) @ np.abs(Bt).T
    assert_gemm_close(got, ref, den, K, f"padded {dtype} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,ta,tb", [(3000, 5000, 600, 0, 0), (3001, 4200, 520, 0, 1), (4100, 3000, 700, 1, 0),
                                         (3000, 4100, 600, 1, 1)])
def test_f32_edge128_every_entry(hip, oracle, M, N, K, ta, tb):
    # f32 ragged products past four 64 x 64 tiles per CU with K over 512 and
    # at least three 128 x 128 tiles per CU: the 128 x 128 tiled kernel with
    # guarded edges on the operands in place (K ragged to the 16-deep
    # k-tile).  C pre-filled with NaN; every entry against the loop.
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, ta, tb, seed=7 * M + N + K + 2 * ta + tb)
    out = hip.from_numpy(np.full((M, N), np.nan, np.float32))
    got = hip.matmul(hip.from_numpy(A), hip.from_numpy(B), trans_a=bool(ta), trans_b=bool(tb), out=out).numpy()
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    assert_gemm_close(got, ref, den, K, f"f32 edge128 {M}x{N}x{K} ta={ta} tb={tb}")


def test_f32_edge128_batched_every_entry(hip, oracle):
    # four 1500 x 2100 x 520 products: 816 tiles of 128 x 128 over the batch
    bs, M, N, K = 4, 1500, 2100, 520
    rng = np.random.default_rng(88)
    A = rng.uniform(-1, 1, (bs, M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (bs, K, N)).astype(np.float32)
    out = hip.from_numpy(np.full((bs, M, N), np.nan, np.float32))
    got = hip.matmul_batched(hip.from_numpy(A), hip.from_numpy(B), out=out).numpy()
    for i in range(bs):
        Bt = np.ascontiguousarray(B[i].T)
        ref = oracle.matmul(A[i], Bt, trans_b=True, threads=16)
        den = np.abs(A[i]).astype(np.float64) @ np.abs(Bt).astype(np.float64).T
        assert_gemm_close(got[i], ref, den, K, f"f32 edge128 batched {i}")


@pytest.mark.parametrize("dtype,off", [("f32", 1), ("bf16", 1), ("bf16", 4)])
def test_padded_misaligned_views(hip, oracle, dtype, off):
    # Views starting `off` elements into their buffers at an aligned shape
    # large enough for the padded route: the operands are copied (element by
    # element, the source rows not being 16-byte aligned) into aligned buffers.
    M, N, K = 1024, 1024, 512
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, 0, 1, seed=77 + off)
    abuf = hip.from_numpy(np.concatenate([np.zeros(off, A.dtype), A.ravel()]), dtype)
    bbuf = hip.from_numpy(np.concatenate([np.zeros(off, B.dtype), B.ravel()]), dtype)
    a, b = abuf.sub(off, A.shape), bbuf.sub(off, B.shape)
    got = hip.matmul(a, b, trans_b=True).numpy()
    ref = oracle.matmul(Au, Bu, trans_b=True, threads=16)
    den = np.abs(Au).astype(np.float64) @ np.abs(Bu.T).astype(np.float64)
    assert_gemm_close(got, ref, den, K, f"padded {dtype} view at +{off}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_padded_batched_every_entry(hip, oracle, dtype, ta, tb):
    bsz, M, N, K = 5, 700, 900, 300
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=5 + ta + tb, batch=bsz)
    got = hip.matmul_batched(hip.from_numpy(A, dtype), hip.from_numpy(B, dtype), trans_a=bool(ta),
                             trans_b=bool(tb)).numpy()
    assert got.shape == (bsz, M, N)
    for i in range(bsz):
        ref = oracle.matmul(Au[i], Bu[i], trans_a=bool(ta), trans_b=bool(tb), threads=16)
        den = np.abs(Au[i].T if ta else Au[i]).astype(np.float64) @ \
            np.abs(Bu[i].T if tb else Bu[i]).astype(np.float64)
        assert_gemm_close(got[i], ref, den, K, f"padded batched {dtype} entry {i}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_padded_infinities_and_nans(hip, oracle, dtype):
    # The padded rows, columns and k add zeros only: an Inf or NaN reaches
    # exactly the entries its row or column feeds, and 0 * Inf = NaN of a
    # padded partner never lands in a valid entry.
    M, N, K = 1000, 1001, 70
    rng = np.random.default_rng(29)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    A[999, 69] = np.inf          # last row, last k: its padded neighbours are zeros
    A[5, 3] = np.nan
    B[69, 1000] = -np.inf        # last k, last column
    B[2, 7] = 0.0
    A[9, 2] = np.inf             # Inf times 0 -> NaN at (9, 7)
    if dtype == "bf16":
        a, b = hip.from_numpy(oracle.to_bf16(A)), hip.from_numpy(oracle.to_bf16(B))
        Au, Bu = oracle.bf16_to_f32(a.numpy()).reshape(M, K), oracle.bf16_to_f32(b.numpy()).reshape(K, N)
    else:
        a, b = hip.from_numpy(A), hip.from_numpy(B)
        Au, Bu = A, B
    got = hip.matmul(a, b).numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        ref = Au.astype(np.float64) @ Bu.astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    assert np.isnan(got[9, 7]) and np.isnan(got[5]).all()
    fin = np.isfinite(ref)
    den = np.abs(Au).astype(np.float64) @ np.abs(Bu).astype(np.float64)
    assert np.all(np.abs(got[fin] - ref[fin]) <= 1e-5 * np.sqrt(K) * den[fin])


# f32 ragged shapes with up to 4 tiles of 64 x 64 per CU run the 64 x 64
# kernel with guarded edges on the operands in place: the copies are buffer
# loads that read zeros outside the matrix, the stores are masked.  It needs
# each operand's contiguous extent to be a multiple of 4 (whole 16-byte
# chunks): K for a k-contiguous operand, M or N for an m/n-contiguous one.
# Per layout: all three dimensions ragged against the tile (64 x 64 x 16), a
# tile row or column mostly outside, K below one k-tile, and products of a
# few tiles.  Every entry against the loop.
_EDGE_CASES = [
    (1001, 1000, 996, 0, 0), (100, 104, 52, 0, 0), (200, 300, 12, 0, 0), (1000, 1000, 1000, 0, 0),
    (999, 1001, 1000, 0, 1), (130, 97, 44, 0, 1), (65, 1000, 4, 0, 1),
    (1000, 1004, 999, 1, 0), (132, 100, 45, 1, 0), (1000, 1000, 1000, 1, 0),
    (1000, 999, 1004, 1, 1), (100, 131, 48, 1, 1), (1448, 1448, 1448, 1, 1),
    # a short K over many tiles (past four per CU)
    (5000, 5000, 252, 0, 0), (3000, 3000, 500, 1, 1), (6000, 4000, 128, 1, 0), (4100, 4000, 300, 0, 1),
]


@pytest.mark.parametrize("M,N,K,ta,tb", _EDGE_CASES)
def test_f32_edge_tiles_every_entry(hip, oracle, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, ta, tb, seed=M + 5 * N + 11 * K + 2 * ta + tb)
    a, b = hip.from_numpy(A), hip.from_numpy(B)
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert got.shape == (M, N)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "repeat"
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb), threads=16)
    den = np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, den, K, f"f32 edge {M}x{N}x{K} ta={ta} tb={tb}")


# f32 ragged products of one or two rounds of 128 x 128 tiles (M, N and K
# ragged against 128 x 128 x 16, all four layouts, batched): the 64 x 64
# guarded-edge tiles or the padded route.  C pre-filled with NaN.
_F32_RAGGED_ROUND_CASES = [
    (2000, 2000, 1000, 0, 0), (2000, 2000, 1004, 0, 1), (1900, 2100, 996, 1, 0), (2000, 2000, 2004, 1, 1),
    (2500, 2500, 600, 0, 0), (2540, 2532, 100, 1, 1),
]


@pytest.mark.parametrize("M,N,K,ta,tb", _F32_RAGGED_ROUND_CASES)
def test_f32_ragged_rounds_every_entry(hip, oracle, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, ta, tb, seed=M + 3 * N + 5 * K + 2 * ta + tb)
    a, b = hip.from_numpy(A), hip.from_numpy(B)
    out = hip.from_numpy(np.full((M, N), np.nan, np.float32))
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb), out=out).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "repeat"
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb), threads=16)
    den = np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, den, K, f"f32 ragged rounds {M}x{N}x{K} ta={ta} tb={tb}")


def test_f32_ragged_rounds_batched_every_entry(hip, oracle):
    bsz, M, N, K = 4, 1000, 1000, 500  # 256 tiles of 128 x 128 over four products
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, 0, 1, seed=61, batch=bsz)
    got = hip.matmul_batched(hip.from_numpy(A), hip.from_numpy(B), trans_b=True).numpy()
    for i in range(bsz):
        ref = oracle.matmul(Au[i], Bu[i], trans_b=True, threads=16)
        den = np.abs(Au[i]).astype(np.float64) @ np.abs(Bu[i]).astype(np.float64).T
        assert_gemm_close(got[i], ref, den, K, f"f32 ragged rounds batched entry {i}")


def test_f32_ragged_rounds_infinities_and_nans(hip):
    # the zeros read past the operands add 0 * 0 only (2000 x 2000 x 1000)
    M, N, K = 2000, 2000, 1000
    rng = np.random.default_rng(67)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    A[M - 1, K - 1] = np.inf
    A[7, 3] = np.nan
    B[K - 1, N - 1] = -np.inf
    B[K - 2, 11] = np.inf
    got = hip.matmul(hip.from_numpy(A), hip.from_numpy(B)).numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        ref = A.astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_f32_edge_tiles_batched_every_entry(hip, oracle, ta, tb):
    # 3 x 700 x 900 x 300: 495 tiles of 64 x 64 over three products
    bsz, M, N, K = 3, 700, 900, 300
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, ta, tb, seed=17 + ta + tb, batch=bsz)
    got = hip.matmul_batched(hip.from_numpy(A), hip.from_numpy(B), trans_a=bool(ta), trans_b=bool(tb)).numpy()
    for i in range(bsz):
        ref = oracle.matmul(Au[i], Bu[i], trans_a=bool(ta), trans_b=bool(tb), threads=16)
        den = np.abs(Au[i].T if ta else Au[i]).astype(np.float64) @ \
            np.abs(Bu[i].T if tb else Bu[i]).astype(np.float64)
        assert_gemm_close(got[i], ref, den, K, f"f32 edge batched entry {i}")


# bf16 ragged products that the padded route would run on 128 x 128 tiles
# (fewer 256 x 256 tiles than half a round) run those tiles with guarded
# edges (64 x 128 tiles up to a round with a k-contiguous A; three stages up
# to a round, two beyond), the operands in place.  Contiguous extents are
# multiples of 8 (whole 16-byte chunks).
_BF16_EDGE_CASES = [
    (1001, 1000, 1000, 0, 0), (2000, 2400, 520, 0, 0), (104, 200, 264, 0, 0),
    (999, 1001, 1000, 0, 1), (2001, 2399, 512, 0, 1),
    (1000, 1008, 999, 1, 0), (2000, 2400, 333, 1, 0),
    (1000, 999, 1000, 1, 1), (136, 150, 200, 1, 1),
]


@pytest.mark.parametrize("M,N,K,ta,tb", _BF16_EDGE_CASES)
def test_bf16_edge_tiles_every_entry(hip, oracle, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, "bf16", M, N, K, ta, tb, seed=3 * M + N + 7 * K + 2 * ta + tb)
    a, b = hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16")
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert got.shape == (M, N)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "repeat"
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb), threads=16)
    den = np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, den, K, f"bf16 edge {M}x{N}x{K} ta={ta} tb={tb}")


def test_bf16_edge_tiles_batched_every_entry(hip, oracle):
    bsz, M, N, K = 3, 700, 904, 296
    A, B, Au, Bu = _operands(oracle, "bf16", M, N, K, 0, 0, seed=23, batch=bsz)
    got = hip.matmul_batched(hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16")).numpy()
    for i in range(bsz):
        ref = oracle.matmul(Au[i], Bu[i], threads=16)
        den = np.abs(Au[i]).astype(np.float64) @ np.abs(Bu[i]).astype(np.float64)
        assert_gemm_close(got[i], ref, den, K, f"bf16 edge batched entry {i}")


# At least half a round of 256 x 256 tiles with K past the short-K kernels:
# the paired-copy kernel's guarded-edge form (A.B, A.B^T, A^T.B^T) reads the
# ragged operands in place, and for A^T.B (no k-contiguous operand) the
# single-ring ping-pong kernel's.  Ragged M, N and K (K % 64 != 0: a pair of
# k-tiles half past K).
_BF16_PAIRS_EDGE_CASES = [
    (3000, 3000, 1000, 0, 0), (2600, 4100, 520, 0, 1), (3000, 2900, 1000, 1, 1), (300, 30000, 700, 0, 0),
    (4000, 3000, 2056, 0, 0), (3000, 3000, 1000, 1, 0), (3000, 5000, 2000, 1, 0), (2900, 4100, 1000, 1, 0),
    (40000, 200, 1000, 0, 0), (40000, 200, 1000, 1, 0),  # one partial column of tiles
    # a short K over as many tiles: 128 x 128 tiles with guarded edges
    (5000, 5000, 248, 0, 0), (3000, 3000, 504, 0, 1), (6000, 5000, 128, 1, 0), (4100, 4000, 200, 1, 1),
]


@pytest.mark.parametrize("M,N,K,ta,tb", _BF16_PAIRS_EDGE_CASES)
def test_bf16_pairs_edge_every_entry(hip, oracle, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, "bf16", M, N, K, ta, tb, seed=5 * M + N + 3 * K + 2 * ta + tb)
    a, b = hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16")
    out = hip.from_numpy(np.full((M, N), np.nan, np.float32))  # every entry must be written
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb), out=out).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert got.shape == (M, N)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "repeat"
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb), threads=16)
    den = np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, den, K, f"bf16 pairs edge {M}x{N}x{K} ta={ta} tb={tb}")


def test_bf16_pairs_edge_batched_every_entry(hip, oracle):
    bsz, M, N, K = 3, 1800, 2000, 600
    A, B, Au, Bu = _operands(oracle, "bf16", M, N, K, 0, 1, seed=29, batch=bsz)
    got = hip.matmul_batched(hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16"), trans_b=True).numpy()
    for i in range(bsz):
        ref = oracle.matmul(Au[i], Bu[i], trans_b=True, threads=16)
        den = np.abs(Au[i]).astype(np.float64) @ np.abs(Bu[i]).astype(np.float64).T
        assert_gemm_close(got[i], ref, den, K, f"bf16 pairs edge batched entry {i}")


# Rows that are not whole 16-byte chunks (an extent not a multiple of 8 in
# bf16 or 4 in f32): the operands that need it are copied with their
# contiguous extent rounded up (and K rounded up in both when K itself is
# ragged), and the guarded-edge kernels run on the copies with C written in
# place.  One case per route: fewer 256 x 256 tiles than half a round, a
# short K over many tiles, the paired-copy kernel (K ragged to 8 too), A^T.B's
# single-ring kernel; f32's 64 x 64 kernels.  C pre-filled with NaN.
_ALIGN_CASES = [
    ("bf16", 1500, 1500, 1500, 0, 0), ("bf16", 1500, 1500, 1500, 0, 1), ("bf16", 1500, 1500, 1500, 1, 0),
    ("bf16", 1500, 1500, 1500, 1, 1), ("bf16", 2048, 1100, 256, 0, 0), ("bf16", 5000, 5004, 200, 0, 0),
    ("bf16", 5004, 5000, 202, 1, 1), ("bf16", 3000, 3004, 1000, 0, 0), ("bf16", 3000, 3000, 1002, 0, 1),
    ("bf16", 3001, 3000, 1000, 1, 0), ("bf16", 3000, 2999, 998, 1, 1),
    ("f32", 1001, 1001, 1001, 0, 0), ("f32", 1001, 1001, 1001, 0, 1), ("f32", 1001, 1001, 1001, 1, 0),
    ("f32", 1001, 1001, 1001, 1, 1), ("f32", 3000, 3001, 501, 0, 0), ("f32", 2999, 3000, 250, 1, 1),
]


@pytest.mark.parametrize("dtype,M,N,K,ta,tb", _ALIGN_CASES)
def test_aligned_copies_every_entry(hip, oracle, dtype, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=7 * M + 3 * N + K + 2 * ta + tb)
    a, b = hip.from_numpy(A, dtype), hip.from_numpy(B, dtype)
    out = hip.from_numpy(np.full((M, N), np.nan, np.float32))  # every entry must be written
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb), out=out).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "repeat"
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb), threads=16)
    den = np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, den, K, f"aligned copies {dtype} {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_aligned_copies_batched_every_entry(hip, oracle, dtype):
    bsz, M, N, K = 3, 701, 899, 301
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, 1, 0, seed=43, batch=bsz)
    got = hip.matmul_batched(hip.from_numpy(A, dtype), hip.from_numpy(B, dtype), trans_a=True).numpy()
    for i in range(bsz):
        ref = oracle.matmul(Au[i], Bu[i], trans_a=True, threads=16)
        den = np.abs(Au[i].T).astype(np.float64) @ np.abs(Bu[i]).astype(np.float64)
        assert_gemm_close(got[i], ref, den, K, f"aligned copies batched {dtype} entry {i}")


def test_bf16_pairs_edge_infinities_and_nans(hip):
    # the zeros read past the operands add 0 * 0 only: an Inf or NaN in the
    # last row, column or k reaches exactly the entries it feeds
    M, N, K = 3000, 3000, 1000
    rng = np.random.default_rng(37)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    A[M - 1, K - 1] = np.inf
    A[7, 3] = np.nan
    B[K - 1, N - 1] = -np.inf
    B[K - 2, 11] = np.inf
    a = hip.to_bf16(hip.from_numpy(A))
    b = hip.to_bf16(hip.from_numpy(B))
    got = hip.matmul(a, b).numpy()
    Ab = a.numpy().astype(np.uint32) << 16
    Bb = b.numpy().astype(np.uint32) << 16
    Af, Bf = Ab.view(np.float32).astype(np.float64), Bb.view(np.float32).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = Af @ Bf
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))


def test_f32_edge_tiles_infinities_and_nans(hip, oracle):
    # The zeros the edge copies read outside the matrix add 0 * 0 = +0 only:
    # an Inf or NaN in the last row, column or k reaches exactly the entries
    # it feeds (1000 x 1000 x 70: every dimension ragged against the tile).
    M, N, K = 1000, 1000, 70
    rng = np.random.default_rng(31)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    A[999, 69] = np.inf
    A[5, 3] = np.nan
    B[69, 999] = -np.inf
    B[2, 7] = 0.0
    A[9, 2] = np.inf
    got = hip.matmul(hip.from_numpy(A), hip.from_numpy(B)).numpy()
    with np.errstate(invalid="ignore", over="ignore"):
        ref = A.astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    assert np.isnan(got[9, 7]) and np.isnan(got[5]).all()
    fin = np.isfinite(ref)
    den = np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)
    assert np.all(np.abs(got[fin] - ref[fin]) <= 1e-5 * np.sqrt(K) * den[fin])


# The aligned kernels are chosen by tile count (on a 256-CU MI355X): f32 runs
# the small kernel up to 512 tiles of 32 x 32 (640^3), 64 x 64 tiles below
# 256 tiles of 128 x 128 (1024^2 x 512, 1280^2 x 256), the ping-pong kernel on
# 128 x 128 tiles where their last round is at least 77% full (2048^2 x 128;
# x 16, one k-tile; 2048 x 4096 x 48; 2560^2 x 64; three rounds at 3072 x 4096
# x 32), 128 x 64 tiles where the last round of four workgroups per CU would
# be under 70% full and K is too short to split it (2304^2 x 128); bf16 runs 64 x 128
# tiles for up to a round of 128 x 128 (1024^2 x 512; 128 x 128 with an
# m-contiguous A), two-stage 128 x 128 tiles for several rounds
# (2304^2 x 128), and 256 x 256 tiles from 128 of them (3072^2 x 128 tiled,
# 3072^2 x 640 ping-pong).  Every entry, every layout.
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("dtype,M,N,K", [
    ("f32", 640, 640, 640), ("f32", 1024, 1024, 512), ("f32", 1280, 1280, 256),
    ("f32", 2304, 2304, 128), ("f32", 2048, 2048, 128), ("f32", 2048, 2048, 16), ("f32", 2048, 4096, 48),
    ("f32", 2560, 2560, 64), ("f32", 3072, 4096, 32),
    ("bf16", 1024, 1024, 512), ("bf16", 2304, 2304, 128), ("bf16", 3072, 3072, 128),
    ("bf16", 3072, 3072, 640),
])
def test_tile_choices_every_entry(hip, oracle, dtype, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=M + N + K + 2 * ta + tb)
    got = hip.matmul(hip.from_numpy(A, dtype), hip.from_numpy(B, dtype), trans_a=bool(ta),
                     trans_b=bool(tb)).numpy()
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb), threads=16)
    den = np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, den, K, f"{dtype} {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_f32_batched_products_on_the_128_tile_ping_pong(hip, oracle, ta, tb):
    # four 1024^2 x 80 products: one round of 256 tiles of 128 x 128 over the batch
    bsz, M, N, K = 4, 1024, 1024, 80
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, ta, tb, seed=91 + ta, batch=bsz)
    got = hip.matmul_batched(hip.from_numpy(A), hip.from_numpy(B), trans_a=bool(ta), trans_b=bool(tb)).numpy()
    for i in range(bsz):
        ref = oracle.matmul(Au[i], Bu[i], trans_a=bool(ta), trans_b=bool(tb), threads=16)
        den = np.abs(Au[i].T if ta else Au[i]).astype(np.float64) @ np.abs(Bu[i].T if tb else Bu[i]).astype(np.float64)
        assert_gemm_close(got[i], ref, den, K, f"batched 128-tile ping-pong product {i}")


@pytest.mark.parametrize("dtype,bsz,M,N,K,ta,tb", [
    # f32, 64 tiles of 128 x 128 over the batch: 4 K slices of 512 (a round
    # of 256 tiles on the 128 x 128 ping-pong kernel, each slice at its
    # product's k-offset), added in order
    *[("f32", 16, 256, 256, 2048, ta, tb) for ta in (0, 1) for tb in (0, 1)],
    # 64 products of one tile: 4 slices of 1024
    ("f32", 64, 128, 128, 4096, 0, 0),
    # 48 tiles: 5 slices of 768 (240 tiles)
    ("f32", 3, 512, 512, 3840, 1, 0),
    # bf16 on the 128 x 128 tiled kernel: 64 tiles as 4 slices of 1024
    *[("bf16", 16, 256, 256, 4096, ta, tb) for ta in (0, 1) for tb in (0, 1)],
    # 32 tiles as 8 slices of 1024
    ("bf16", 2, 512, 512, 8192, 0, 1),
])
def test_batched_k_slices_every_entry(hip, oracle, dtype, bsz, M, N, K, ta, tb):
    # Every entry of every product against the loop, and bitwise the same on
    # a second call.
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=97 + 2 * ta + tb, batch=bsz)
    a, b = hip.from_numpy(A, dtype), hip.from_numpy(B, dtype)
    got = hip.matmul_batched(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    again = hip.matmul_batched(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    for i in range(bsz):
        Ak = np.ascontiguousarray(Au[i].T if ta else Au[i])
        Bk = np.ascontiguousarray(Bu[i] if tb else Bu[i].T)
        ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
        den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
        assert_gemm_close(got[i], ref, den, K, f"{dtype} batched K slices {i}/{bsz} {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_many_tiny_products_stay_on_the_general_kernel(hip, oracle, dtype):
    # 2048 products of 16 x 24 x 20: above the padded route's size threshold
    # in total, but padding each to whole tiles would multiply the work, so
    # they run the guarded general kernel; every entry of every product.
    bsz, M, N, K = 2048, 16, 24, 20
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, 0, 1, seed=61, batch=bsz)
    got = hip.matmul_batched(hip.from_numpy(A, dtype), hip.from_numpy(B, dtype), trans_b=True).numpy()
    den = np.einsum("bmk,bnk->bmn", np.abs(Au).astype(np.float64), np.abs(Bu).astype(np.float64))
    for i in range(bsz):
        ref = oracle.matmul(Au[i], Bu[i], trans_b=True)
        assert_gemm_close(got[i], ref, den[i], K, f"tiny {dtype} product {i}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(1024, 4096, 8192), (1024, 2048, 16384), (2048, 2048, 8192),
                                   (64, 64, 65536), (512, 512, 16384), (192, 320, 8192),
                                   (1024, 1024, 4096), (768, 768, 8192)])
def test_f32_k_split_every_entry(hip, oracle, M, N, K, ta, tb):
    # Few tiles and a long K: the product runs as K slices (4 or 8 on the
    # ping-pong kernel for 256 x 256 tiles; 4 to 16 that fill a round of
    # 128 x 128 tiles; 8 to 128 on the small-product or 64 x 64 kernels
    # otherwise), then the slices are added in order.
    # Every entry against the loop (its A.B^T form on transposed copies, bit
    # for bit its A.B loop), and bitwise the same on a second call.
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, ta, tb, seed=M + N + K + 2 * ta + tb)
    a, b = hip.from_numpy(A), hip.from_numpy(B)
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak) @ np.abs(Bk).T
    assert_gemm_close(got, ref, den, K, f"k-split {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("M,N,K,ta,tb", [
    # 324 tiles of 128 x 128: rows 0-1791 a whole round on the ping-pong
    # kernel, rows 1792-2303 a product of their own
    *[(2304, 2304, 768, ta, tb) for ta in (0, 1) for tb in (0, 1)],
    # 272 tiles of 256 x 256: rows 0-4095 a round of them, rows 4096-4351 on
    # 64 x 64 tiles
    *[(4352, 4096, 256, ta, tb) for ta in (0, 1) for tb in (0, 1)],
    # 352 tiles of 256 x 256, whose remaining 768 rows (384 tiles of 128 x
    # 128) split again: rows 0-2047, 2048-2559, 2560-2815
    (2816, 8192, 512, 0, 0), (2816, 8192, 512, 1, 1),
])
def test_f32_ragged_round_split_every_entry(hip, oracle, M, N, K, ta, tb):
    # A product whose last round of tiles is ragged runs as bands of rows:
    # whole rounds, then the rest on its own kernels.  Every entry against the
    # loop (A.B^T form on transposed copies), and bitwise the same on a second
    # call.
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, ta, tb, seed=5 + 2 * ta + tb)
    a, b = hip.from_numpy(A), hip.from_numpy(B)
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    assert_gemm_close(got, ref, den, K, f"round split {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("M,N,K,ta,tb", [
    # 384 tiles of 128 x 128 (a round and a half): two K slices of 1024 fill
    # three whole rounds on the ping-pong kernel, added in order
    *[(2048, 3072, 2048, ta, tb) for ta in (0, 1) for tb in (0, 1)],
    # the same on zero-padded copies (2048 x 3072 x 2048)
    (2000, 3000, 2040, 0, 0),
])
def test_f32_k_slices_at_ragged_round_every_entry(hip, oracle, M, N, K, ta, tb):
    # Every entry against the loop (A.B^T form on transposed copies), and
    # bitwise the same on a second call.
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, ta, tb, seed=41 + 2 * ta + tb)
    a, b = hip.from_numpy(A), hip.from_numpy(B)
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    assert_gemm_close(got, ref, den, K, f"K slices {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bf16_ragged_round_split_every_entry(hip, oracle, ta, tb):
    # 272 tiles of 256 x 256: rows 0-4095 a round of them, rows 4096-4351 a
    # product of their own.  Every entry against the loop on the upcast values,
    # and bitwise the same on a second call.
    M, N, K = 4352, 4096, 512
    A, B, Au, Bu = _operands(oracle, "bf16", M, N, K, ta, tb, seed=31 + 2 * ta + tb)
    a, b = hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16")
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    assert_gemm_close(got, ref, den, K, f"bf16 round split {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(100, 100, 100000), (70, 300, 30000), (1000, 1000, 32768), (1001, 1003, 20000),
                                   (1001, 1003, 32768), (2048, 200, 2000)])
def test_f32_ragged_long_k_every_entry(hip, oracle, M, N, K, ta, tb):
    # Ragged M or N, few tiles and a long K: K slices on the 64 x 64 kernel's
    # guarded-edge form (1000^2 x 32768 and 1001 x 1003 x 32768 on the 128 x
    # 128 kernel's, 16 slices), on the operands in place (1000^2 x 32768, 100^2 x
    # 100000 as 125 slices, 70 x 300 x 30000, 2048 x 200 x 2000), on aligned
    # copies of the operands whose rows are not whole chunks (1001 x 1003 x
    # 32768), or on aligned copies of both with K rounded up to 2048 (1001 x
    # 1003 x 20000).  1001 x 1003 is odd for the slice sum's tail.  C
    # pre-filled with NaN; every entry against the loop.
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, ta, tb, seed=M + N + K + ta)
    out = hip.from_numpy(np.full((M, N), np.nan, np.float32))
    got = hip.matmul(hip.from_numpy(A), hip.from_numpy(B), trans_a=bool(ta), trans_b=bool(tb), out=out).numpy()
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    assert_gemm_close(got, ref, den, K, f"ragged long-K {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("M,N,K,ta,tb", [(2500, 640, 16384, 1, 1), (1536, 1100, 8192, 0, 0), (1200, 1100, 12000, 0, 1),
                                         (1500, 1500, 8192, 1, 0), (1201, 1103, 8192, 0, 0), (2000, 2000, 8192, 1, 0)])
def test_f32_balanced_slices_every_entry(hip, oracle, M, N, K, ta, tb):
    # Ragged products with more 64 x 64 tiles than CUs and a long K: K
    # slices that even out the tiles per CU (2500 x 640 x 16384, 400 tiles,
    # in 8 slices; 1536 x 1100 x 8192 and 1500^2 x 8192 in 4; 1200 x 1100 x
    # 12000 in 5, slices of 2400; 1201 x 1103 x 8192 on aligned copies, odd
    # M*N for the slice sum's tail; 2000^2 x 8192 in 4 slices of 128 x 128
    # tiles).  C pre-filled with NaN; every entry against the loop, and a
    # second call bit for bit.
    A, B, Au, Bu = _operands(oracle, "f32", M, N, K, ta, tb, seed=M + N + K + 2 * ta + tb)
    ha, hb = hip.from_numpy(A), hip.from_numpy(B)
    out = hip.from_numpy(np.full((M, N), np.nan, np.float32))
    got = hip.matmul(ha, hb, trans_a=bool(ta), trans_b=bool(tb), out=out).numpy()
    again = hip.matmul(ha, hb, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    assert_gemm_close(got, ref, den, K, f"balanced slices {M}x{N}x{K} ta={ta} tb={tb}")
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


@pytest.mark.parametrize("M,N,K,ta,tb", [(1500, 1500, 8192, 1, 1), (1200, 1100, 12000, 0, 1), (900, 900, 20000, 1, 0),
                                         (1152, 1152, 8192, 0, 0), (1024, 1024, 16384, 1, 0)])
def test_bf16_slices_past_one_round_every_entry(hip, oracle, M, N, K, ta, tb):
    # bf16 products with a partial round of 128 x 128 tiles and a long K: K
    # slices past one round of tiles, up to 4 per CU.  Ragged, on the
    # guarded-edge kernels: 1500^2 x 8192 (144 tiles) in 4 slices; 1200 x
    # 1100 x 12000 in 5, slices of 2400, ragged to the 64-deep k-tile; 900^2 x
    # 20000 in 10.  Aligned, on the tiled kernels: 1152^2 x 8192 in 4, 1024^2
    # x 16384 A^T.B in 8.  C pre-filled with NaN; every entry against the
    # loop, and a second call bit for bit.
    A, B, Au, Bu = _operands(oracle, "bf16", M, N, K, ta, tb, seed=3 * M + N + K + 2 * ta + tb)
    a, b = hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16")
    out = hip.from_numpy(np.full((M, N), np.nan, np.float32))
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb), out=out).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    assert_gemm_close(got, ref, den, K, f"bf16 slices past a round {M}x{N}x{K} ta={ta} tb={tb}")
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(64, 64, 65536), (128, 128, 65536), (512, 1024, 16384), (100, 100, 100000),
                                   (256, 8448, 4096), (1000, 1000, 32768), (1001, 1001, 32768),
                                   (704, 896, 30000), (128, 300, 5000), (300, 400, 20024)])
def test_bf16_k_split_every_entry(hip, oracle, M, N, K, ta, tb):
    # bf16 products with few 128 x 128 tiles and a long K run as K slices:
    # on the tiled kernels; on their guarded-edge forms for a ragged M, N or
    # K, as many slices as whole 16-byte chunks allow (64 x 64, 1000^2, 704 x
    # 896 x 30000, 128 x 300 x 5000 in place; 1001^2 and 100^2 on aligned
    # copies, 1001^2 odd so the slice sum has a tail); on aligned copies with
    # K rounded up to 2048 where no slice count divides K in whole chunks
    # (300 x 400 x 20024, 20024 = 8 x 2503); with fewer 256 x 256 tiles than
    # half a round as slices of those (256 x 8448: 33 tiles, 4 slices).
    # Added in order; C pre-filled with NaN; every entry against the f32 loop
    # on the upcast values, and a second call gives the same bits.
    A, B, Au, Bu = _operands(oracle, "bf16", M, N, K, ta, tb, seed=M + N + K + 2 * ta + tb)
    a, b = hip.from_numpy(A, "bf16"), hip.from_numpy(B, "bf16")
    out = hip.from_numpy(np.full((M, N), np.nan, np.float32))
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb), out=out).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    assert_gemm_close(got, ref, den, K, f"bf16 k-split {M}x{N}x{K} ta={ta} tb={tb}")
