"""Matmul dispatch over many shapes on the GPU, through the C ABI.

The aligned kernels are chosen by shape: the small-product kernel, 64 x 64 and
128 x 128 tiles, the 128 x 128 and 256 x 256 ping-pong kernels, K slices,
bands of rows at a ragged round of tiles, zero-padded copies for ragged
shapes, the skinny kernels (an output dimension of 2-32), matrix-vector and
outer products, and the guarded general kernel.  This file draws shapes
around those thresholds (tile multiples and their neighbours, short and long
K, one-row outputs) from a fixed seed, in both dtypes and random layouts, and
checks every entry against the oracle's loop (oracle/oracle.c, linalg.matmul
of /root/reference/stdlib/linalg/matrix.cleave:27-61) under the GEMM bound
|C - C_ref| <= 1e-5 sqrt(K) sum|A||B|, and that a second call repeats bit for
bit (every path sums in an order fixed by the shape).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_gemm_close

pytestmark = pytest.mark.gpu

_DIMS = [1, 2, 17, 31, 32, 33, 64, 100, 127, 128, 129, 255, 256, 257, 384, 512, 640, 1000, 1024,
         1536, 1920, 2048, 2304, 2816, 3072, 4352]
_KS = [1, 2, 15, 16, 17, 48, 64, 100, 256, 512, 768, 1024, 2048, 4100]
_MAX_MAC = 4e9  # oracle work per case


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M, N = int(rng.choice(_DIMS)), int(rng.choice(_DIMS))
        K = int(rng.choice(_KS))
        if M * N * K > _MAX_MAC:
            continue
        dtype = "bf16" if rng.random() < 0.4 else "f32"
        out.append((dtype, M, N, K, int(rng.integers(2)), int(rng.integers(2))))
    return out


def _operands(oracle, dtype, M, N, K, ta, tb, seed):
    rng = np.random.default_rng(seed)
    A32 = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B32 = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    if dtype == "bf16":
        A, B = oracle.to_bf16(A32), oracle.to_bf16(B32)
        return A, B, oracle.bf16_to_f32(A).reshape(A.shape), oracle.bf16_to_f32(B).reshape(B.shape)
    return A32, B32, A32, B32


@pytest.mark.parametrize("dtype,M,N,K,ta,tb", _cases(160, seed=2024))
def test_shape_every_entry(hip, oracle, dtype, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=M * 7 + N * 3 + K + 2 * ta + tb)
    a, b = hip.from_numpy(A, dtype), hip.from_numpy(B, dtype)
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert got.shape == (M, N)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "repeat"
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    if K == 1:  # one product added to a zero: exact
        assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))
    else:
        assert_gemm_close(got, ref, den, K, f"{dtype} {M}x{N}x{K} ta={ta} tb={tb}")


# Ragged shapes for the routes past the aligned kernels: extents that are not
# whole 16-byte chunks (aligned copies of those operands), few tiles with a
# long K (K slices on the guarded-edge kernels, K rounded up where no slice
# count divides it), and rows of C that are whole 128-byte lines or not (the
# non-temporal C stores).  C pre-filled with NaN.
_RDIMS = [33, 100, 300, 700, 900, 1000, 1001, 1500, 2047, 2500, 3001]
_RKS = [100, 300, 1000, 1002, 3000, 5000, 8192, 20000, 20024, 30000]


def _ragged_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M, N = int(rng.choice(_RDIMS)), int(rng.choice(_RDIMS))
        K = int(rng.choice(_RKS))
        if M * N * K > _MAX_MAC:
            continue
        dtype = "bf16" if rng.random() < 0.5 else "f32"
        out.append((dtype, M, N, K, int(rng.integers(2)), int(rng.integers(2))))
    return out


@pytest.mark.parametrize("dtype,M,N,K,ta,tb", _ragged_cases(60, seed=31))
def test_ragged_shape_every_entry(hip, oracle, dtype, M, N, K, ta, tb):
    A, B, Au, Bu = _operands(oracle, dtype, M, N, K, ta, tb, seed=M * 5 + N * 11 + K + 2 * ta + tb)
    a, b = hip.from_numpy(A, dtype), hip.from_numpy(B, dtype)
    out = hip.from_numpy(np.full((M, N), np.nan, np.float32))
    got = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb), out=out).numpy()
    again = hip.matmul(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "repeat"
    Ak = np.ascontiguousarray(Au.T if ta else Au)
    Bk = np.ascontiguousarray(Bu if tb else Bu.T)
    ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
    assert_gemm_close(got, ref, den, K, f"{dtype} {M}x{N}x{K} ta={ta} tb={tb}")


def _batched_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        M, N = int(rng.choice(_DIMS[:19])), int(rng.choice(_DIMS[:19]))
        K = int(rng.choice(_KS[:12]))
        bsz = int(rng.choice([2, 3, 7, 16, 64]))
        if bsz * M * N * K > _MAX_MAC / 2:
            continue
        dtype = "bf16" if rng.random() < 0.4 else "f32"
        out.append((dtype, bsz, M, N, K, int(rng.integers(2)), int(rng.integers(2))))
    return out


@pytest.mark.parametrize("dtype,bsz,M,N,K,ta,tb", _batched_cases(48, seed=7))
def test_batched_shape_every_entry(hip, oracle, dtype, bsz, M, N, K, ta, tb):
    rng = np.random.default_rng(bsz * 1000 + M + N + K)
    A32 = rng.standard_normal((bsz,) + ((K, M) if ta else (M, K))).astype(np.float32)
    B32 = rng.standard_normal((bsz,) + ((N, K) if tb else (K, N))).astype(np.float32)
    if dtype == "bf16":
        A, B = oracle.to_bf16(A32), oracle.to_bf16(B32)
        Au, Bu = oracle.bf16_to_f32(A).reshape(A.shape), oracle.bf16_to_f32(B).reshape(B.shape)
    else:
        A, B, Au, Bu = A32, B32, A32, B32
    a, b = hip.from_numpy(A, dtype), hip.from_numpy(B, dtype)
    got = hip.matmul_batched(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    again = hip.matmul_batched(a, b, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert got.shape == (bsz, M, N)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "repeat"
    for i in range(bsz):
        Ak = np.ascontiguousarray(Au[i].T if ta else Au[i])
        Bk = np.ascontiguousarray(Bu[i] if tb else Bu[i].T)
        ref = oracle.matmul(Ak, Bk, trans_b=True, threads=16)
        if K == 1:
            assert np.array_equal(got[i].view(np.uint32), ref.astype(np.float32).view(np.uint32))
        else:
            den = np.abs(Ak).astype(np.float64) @ np.abs(Bk).astype(np.float64).T
            assert_gemm_close(got[i], ref, den, K, f"{dtype} batch {i}/{bsz} {M}x{N}x{K} ta={ta} tb={tb}")
