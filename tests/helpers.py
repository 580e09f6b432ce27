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


def mlp_grad_scales(X, y, W1, W2):
    """Per-entry scales of the MLP step's gradient contractions, in float64.

    dW1 = X^T d1 and dW2 = H^T d2 are K = B contractions, so each entry gets
    the GEMM bound 1e-5 * sqrt(B) * sum_m |a_m||b_m|; these are those sums:
    |X|^T |d1| with |d1| = |W2| * H(1-H) * |d2|, and |H|^T |d2|, where
    d2 = (2/B)(yhat - y) yhat (1 - yhat) from a float64 forward pass (ample for
    a tolerance's scale)."""
    X64 = np.asarray(X, np.float64)
    B = X64.shape[0]
    H = 1.0 / (1.0 + np.exp(-(X64 @ np.asarray(W1, np.float64))))
    W2v = np.asarray(W2, np.float64).ravel()
    yh = 1.0 / (1.0 + np.exp(-(H @ W2v)))
    d2 = np.abs((2.0 / B) * (yh - np.asarray(y, np.float64).ravel()) * yh * (1.0 - yh))
    a1 = np.abs(X64).T @ (np.abs(W2v)[None, :] * (H * (1.0 - H)) * d2[:, None])
    a2 = np.abs(H).T @ d2
    return a1, a2


def assert_mlp_grads_close(got1, got2, ref1, ref2, X, y, W1, W2, what=""):
    """Every dW1 / dW2 entry within the GEMM bound of the oracle's entry."""
    B = np.asarray(X).shape[0]
    a1, a2 = mlp_grad_scales(X, y, W1, W2)
    tol = 1e-5 * np.sqrt(B)
    e1 = gemm_normalised_error(np.asarray(got1).reshape(a1.shape), np.asarray(ref1).reshape(a1.shape), a1)
    e2 = gemm_normalised_error(np.asarray(got2).reshape(a2.shape), np.asarray(ref2).reshape(a2.shape), a2)
    assert e1 <= tol, f"{what} dW1 normalised error {e1:.3e} > {tol:.3e}"
    assert e2 <= tol, f"{what} dW2 normalised error {e2:.3e} > {tol:.3e}"
    return e1, e2
