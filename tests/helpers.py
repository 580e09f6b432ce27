"""Tolerances and small utilities shared by the GPU parity tests.

Tolerances (from the path's specification):
  GEMM   |C_gpu - C_ref| <= 1e-5 * sqrt(K) * sum_k |A_ik||B_kj|   per entry
  maps   |y_gpu - y_ref| <= 1e-5 * |y_ref|   (exp/tanh); bit-exact for IEEE ops
  sums   |s_gpu - s_ref| <= 1e-5 * sum_i |x_i|
  integer outputs (escape counts, u64 sums, argmax): bit-exact
"""
from __future__ import annotations

import numpy as np


def gemm_normalised_error(got, ref, absden) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    absden = np.asarray(absden, np.float64)
    diff = np.abs(got - ref)
    zero = absden == 0
    if np.any(diff[zero] != 0):
        return np.inf
    return float(np.max(diff[~zero] / absden[~zero])) if np.any(~zero) else 0.0


def assert_gemm_close(got, ref, absden, K, what=""):
    err = gemm_normalised_error(got, ref, absden)
    tol = 1e-5 * np.sqrt(K)
    assert err <= tol, f"{what}: normalised error {err:.3e} > {tol:.3e}"
    return err


def rel_close(got, ref, rtol=1e-5, atol=0.0):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    both_nan = np.isnan(got) & np.isnan(ref)
    ok = both_nan | (np.abs(got - ref) <= rtol * np.abs(ref) + atol)
    return bool(np.all(ok))


def sample_entries(M, N, n, seed):
    rng = np.random.default_rng(seed)
    ii = rng.integers(0, M, n).astype(np.int32)
    jj = rng.integers(0, N, n).astype(np.int32)
    # always include the four corners and the tile seams around the middle
    extra_i = np.array([0, 0, M - 1, M - 1, M // 2, M // 2 - 1, min(M - 1, 127), min(M - 1, 128)], np.int32)
    extra_j = np.array([0, N - 1, 0, N - 1, N // 2 - 1, N // 2, min(N - 1, 128), min(N - 1, 127)], np.int32)
    return np.concatenate([ii, extra_i]), np.concatenate([jj, extra_j])


def view(t, offset_elems, n):
    """Unowned sub-view of a device tensor (for misaligned-pointer paths)."""
    import cleave_amd as ca

    esize = {"f32": 4, "u32": 4, "bf16": 2}[t.dtype]
    return ca.Tensor(t.ptr + offset_elems * esize, (n,), t.dtype, owned=False)
