"""Matmul shapes with a dimension of 1 on the GPU (gemv.hip), through the C ABI:
matrix-vector products (N = 1 or M = 1) and outer products (K = 1), every entry
against the oracle's sequential loop (oracle/oracle.c, linalg.matmul of
/root/reference/stdlib/linalg/matrix.cleave:27-61).  These are the shapes of
examples/xor_tensor.cleave:44-49 (matmul by an n x 1 weight) and of its reverse
rule (stdlib/linalg/matrix.cleave:24): G W2^T is an outer product, H^T G a
product over the batch.

Bars: sums within the GEMM bound |C - C_ref| <= 1e-5 sqrt(K) sum|A||B| (their
order differs from the loop's); outer products bit for bit (the loop adds one
product to a zero, and so does the kernel).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_gemm_close

pytestmark = pytest.mark.gpu


def _operands(oracle, dtype, M, N, K, ta, tb, seed, batch=None):
    rng = np.random.default_rng(seed)
    lead = () if batch is None else (batch,)
    A32 = rng.standard_normal(lead + ((K, M) if ta else (M, K))).astype(np.float32)
    B32 = rng.standard_normal(lead + ((N, K) if tb else (K, N))).astype(np.float32)
    if dtype == "bf16":
        A, B = oracle.to_bf16(A32), oracle.to_bf16(B32)
        return A, B, oracle.bf16_to_f32(A).reshape(A.shape), oracle.bf16_to_f32(B).reshape(B.shape)
    return A32, B32, A32, B32


def _check(got, Au, Bu, oracle, ta, tb, K, what):
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb), threads=16)
    if K == 1:
        assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32)), what
        return
    den = np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(got, ref, den, K, what)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [
    (1000, 1, 777), (1024, 1, 4096), (3, 1, 2), (65536, 1, 512),   # N = 1
    (1, 1000, 777), (1, 4096, 1024), (1, 5, 3), (1, 512, 65536),   # M = 1
    (700, 900, 1), (4096, 4096, 1), (1, 7, 1), (9, 1, 1),          # K = 1
    (1, 1, 5000), (1, 1, 1), (1, 1, 2),                             # dot products
    (1, 1, 300000), (3, 1, 100003), (1, 40, 200000),                # few long rows: k cut in slices
])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_vector_shapes_every_entry(hip, oracle, dtype, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=M + 3 * N + 7 * K + 2 * ta + tb)
    got = hip.matmul(hip.from_numpy(A, dtype), hip.from_numpy(B, dtype), trans_a=bool(ta),
                     trans_b=bool(tb)).numpy()
    assert got.shape == (M, N)
    _check(got, Au, Bu, oracle, ta, tb, K, f"{dtype} {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(300, 1, 257), (1, 300, 257), (300, 200, 1)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_vector_shapes_batched(hip, oracle, dtype, M, N, K, ta, tb):
    bsz = 6
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=5 * M + N + K, batch=bsz)
    got = hip.matmul_batched(hip.from_numpy(A, dtype), hip.from_numpy(B, dtype), trans_a=bool(ta),
                             trans_b=bool(tb)).numpy()
    assert got.shape == (bsz, M, N)
    for i in range(bsz):
        _check(got[i], Au[i], Bu[i], oracle, ta, tb, K, f"batched {dtype} {M}x{N}x{K} entry {i}")


@pytest.mark.parametrize("dtype,off", [("f32", 1), ("bf16", 1), ("bf16", 3)])
@pytest.mark.parametrize("M,N,K,ta,tb", [(513, 1, 640, 0, 0), (513, 1, 640, 1, 0), (1, 640, 512, 0, 1),
                                         (1, 640, 512, 0, 0), (64, 96, 1, 0, 0)])
def test_vector_shapes_misaligned_views(hip, oracle, dtype, off, M, N, K, ta, tb):
    # operands starting `off` elements into their buffers: the element-wise
    # (unvectorised) paths
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=17 + off)
    abuf = hip.from_numpy(np.concatenate([np.zeros(off, A.dtype), A.ravel()]), dtype)
    bbuf = hip.from_numpy(np.concatenate([np.zeros(off, B.dtype), B.ravel()]), dtype)
    a, b = abuf.sub(off, A.shape), bbuf.sub(off, B.shape)
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    _check(got, Au, Bu, oracle, ta, tb, K, f"{dtype} view at +{off} {M}x{N}x{K}")


def test_vector_shapes_deterministic_and_special_values(hip, oracle):
    M, K = 2048, 3000
    rng = np.random.default_rng(3)
    A = rng.standard_normal((M, K)).astype(np.float32)
    x = rng.standard_normal((K, 1)).astype(np.float32)
    A[5, 7] = np.inf
    A[9, 2] = np.nan
    x[11, 0] = 0.0
    A[13, 11] = np.inf  # Inf times 0 -> NaN
    a, b = hip.from_numpy(A), hip.from_numpy(x)
    g1 = hip.matmul(a, b).numpy()
    g2 = hip.matmul(a, b).numpy()
    assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32))
    assert np.isinf(g1[5, 0]) and np.sign(g1[5, 0]) == np.sign(x[7, 0])  # Inf times a finite nonzero
    assert np.isnan(g1[9, 0]) and np.isnan(g1[13, 0])
    clean = np.ones(M, bool)
    clean[[5, 9, 13]] = False
    ref = oracle.matmul(A[clean], x)
    den = np.abs(A[clean]).astype(np.float64) @ np.abs(x).astype(np.float64)
    assert_gemm_close(g1[clean], ref, den, K, "gemv with special rows elsewhere")


def test_negative_zero_products_become_positive_zero(hip):
    # K = 1: the loop computes 0 + a*b, which turns a -0 product into +0
    a = np.array([[-0.0], [1.0], [-2.0]], np.float32)
    b = np.array([[0.0, -0.0, 3.0]], np.float32)
    got = hip.matmul(hip.from_numpy(a), hip.from_numpy(b)).numpy()
    want = (np.float32(0.0) + a @ b).astype(np.float32)
    assert np.array_equal(np.signbit(got), np.signbit(want)) and not np.signbit(got[0, 0])


# One output dimension of at most 32 (the skinny kernels of gemv.hip, on the
# matrix cores): the matrix operand along the long output dimension streams
# once, 32 of its rows per wave (16 x 16 tiles up to 16 vectors, 32 x 32 from
# 17), staged through LDS when its rows are k-contiguous; long K in groups
# whose partial tiles are added in order.
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [
    (1000, 10, 777), (4096, 3, 4096), (513, 32, 100), (2000, 17, 1),     # N small
    (10, 4096, 1000), (5, 777, 65536), (31, 2000, 33), (2, 3, 2),        # M small
    (32, 32, 1000), (7, 9, 300000),                                       # both small, long K
    (20000, 20, 3), (30000, 8, 5), (16, 700, 4100),                       # K under one block; K tail
])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_skinny_shapes_every_entry(hip, oracle, dtype, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=2 * M + 5 * N + K + 2 * ta + tb)
    got = hip.matmul(hip.from_numpy(A, dtype), hip.from_numpy(B, dtype), trans_a=bool(ta),
                     trans_b=bool(tb)).numpy()
    assert got.shape == (M, N)
    _check(got, Au, Bu, oracle, ta, tb, K, f"{dtype} {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(300, 7, 257), (7, 300, 257)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_skinny_shapes_batched(hip, oracle, dtype, M, N, K, ta, tb):
    bsz = 5
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=3 * M + N + K, batch=bsz)
    got = hip.matmul_batched(hip.from_numpy(A, dtype), hip.from_numpy(B, dtype), trans_a=bool(ta),
                             trans_b=bool(tb)).numpy()
    for i in range(bsz):
        _check(got[i], Au[i], Bu[i], oracle, ta, tb, K, f"batched {dtype} {M}x{N}x{K} entry {i}")


@pytest.mark.parametrize("dtype,off", [("f32", 1), ("bf16", 1)])
@pytest.mark.parametrize("M,N,K,ta,tb", [(600, 12, 640, 0, 0), (600, 12, 640, 1, 1), (12, 600, 640, 0, 1),
                                         (12, 600, 640, 1, 0)])
def test_skinny_shapes_misaligned_views(hip, oracle, dtype, off, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=29 + off)
    abuf = hip.from_numpy(np.concatenate([np.zeros(off, A.dtype), A.ravel()]), dtype)
    bbuf = hip.from_numpy(np.concatenate([np.zeros(off, B.dtype), B.ravel()]), dtype)
    a, b = abuf.sub(off, A.shape), bbuf.sub(off, B.shape)
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    _check(got, Au, Bu, oracle, ta, tb, K, f"{dtype} view at +{off} {M}x{N}x{K}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(700, 10, 300), (10, 700, 300), (450, 24, 200), (712, 12, 300), (20, 712, 260)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_skinny_clamped_rows_and_columns_stay_apart(hip, oracle, dtype, M, N, K, ta, tb):
    # Rows past the long dimension read its last row, and columns past the
    # short one read its last column: an Inf in op(A)'s last row and a NaN in
    # op(B)'s last column (the clamp targets in either orientation) must reach
    # only the entries the loop gives them.
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=7 * M + N + ta + 2 * tb)
    Af = (Au.T if ta else Au).copy()  # op(A), op(B) as float32
    Bf = (Bu.T if tb else Bu).copy()
    Af[M - 1, 5] = np.inf
    Bf[7, N - 1] = np.nan
    As, Bs = (Af.T if ta else Af).copy(), (Bf.T if tb else Bf).copy()
    if dtype == "bf16":
        As, Bs = oracle.to_bf16(As), oracle.to_bf16(Bs)
    got = hip.matmul(hip.from_numpy(As, dtype), hip.from_numpy(Bs, dtype), trans_a=bool(ta),
                     trans_b=bool(tb)).numpy()
    ref = oracle.matmul(Af, Bf, threads=16)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isinf(got), np.isinf(ref))
    inf = np.isinf(ref)
    assert inf.any() and np.isnan(ref).any()
    assert np.array_equal(np.sign(got[inf]), np.sign(ref[inf]))
    # the rest: rows 0 .. M-2 and columns 0 .. N-2 are untouched by either value
    ca, cb = Af[:M - 1], Bf[:, :N - 1]
    den = np.abs(ca).astype(np.float64) @ np.abs(cb).astype(np.float64)
    assert_gemm_close(got[:M - 1, :N - 1], ref[:M - 1, :N - 1], den, K, f"{dtype} {M}x{N}x{K} away from the specials")
