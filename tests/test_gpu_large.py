"""Maximum sizes: arrays past 2^31 elements and GEMM operands past 4 GiB.

The maps, reductions, Index and the escape-count map index with 64-bit
integers; the fast GEMM kernels address a tile with 32-bit per-lane offsets
from a 64-bit per-tile base, so an operand spanning 4 GiB or more stays on
them.  Each case checks sampled entries against the oracle (or exact closed
forms) without copying the arrays back whole.
One MI355X holds 288 GB; the largest case here allocates 24 GiB.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_gemm_close, rel_close

pytestmark = pytest.mark.gpu

BIG = (1 << 31) + 37  # elements: past the int32 range


def _at(t, idx):
    """Values of device tensor t (flat) at the given indices, one small copy each."""
    return np.concatenate([t.sub(int(i), (1,)).numpy() for i in idx])


def _uniform_at(oracle, seed, i, lo=-1.0, hi=1.0):
    """Element i of the uniform fill: lo + (hi - lo) * u_i in f32 (the
    generator's definition, pinned in test_oracle.py), from one splitmix64 draw."""
    u = np.float32((oracle.splitmix64_at(seed, i) >> 40) * 2.0 ** -24)
    return np.float32(np.float32(lo) + np.float32(hi - lo) * u)


def _samples(n, seed, k=24):
    rng = np.random.default_rng(seed)
    edge = [0, 1, 3, (1 << 31) - 1, 1 << 31, (1 << 31) + 1, n - 5, n - 1]
    return np.unique(np.concatenate([rng.integers(0, n, k), [e for e in edge if e < n]]))


def test_maps_past_2pow31_elements(hip, oracle):
    print(f"maps over {BIG} f32 elements", flush=True)
    a = hip.fill_uniform(hip.empty(BIG), seed=11)
    b = hip.fill_uniform(hip.empty(BIG), seed=12, lo=0.5, hi=2.0)
    out = hip.add(a, b)
    idx = _samples(BIG, 1)
    A, B = _at(a, idx), _at(b, idx)
    assert np.array_equal(_at(out, idx), oracle.add(A, B))
    hip.div(a, b, out=out)
    assert np.array_equal(_at(out, idx), oracle.div(A, B))
    hip.sigmoid(a, out=out)
    assert rel_close(_at(out, idx), oracle.sigmoid(A), 1e-5)
    # 4 bytes past a 16-byte boundary: the scalar path of the maps
    va, vo = a.sub(1, (BIG - 1,)), out.sub(1, (BIG - 1,))
    hip.neg(va, out=vo)
    assert np.array_equal(_at(out, idx[idx >= 1]), -A[idx >= 1])


def test_reductions_past_2pow31_elements(hip, oracle):
    print(f"reductions over {BIG} f32 elements", flush=True)
    x = hip.zero((BIG,))
    far = (1 << 31) + 19
    x.sub(far, (1,)).upload(np.array([7.5], np.float32))
    assert hip.max_of(x) == 7.5
    assert hip.argmax(x) == far  # an index past the int32 range
    x.sub(far + 8, (1,)).upload(np.array([7.5], np.float32))
    assert hip.argmax(x) == far  # first of equal maxima, as the reference's strict > fold
    assert hip.sum(x) == 15.0
    x.sub(5, (1,)).upload(np.array([np.nan], np.float32))
    assert hip.argmax(x) == far  # a NaN after v[0] never wins (cmpf ogt)
    # ones: the f32 sum is n up to rounding, within the sum bound n * 1e-5
    hip.fill_uniform(x, seed=3, lo=1.0, hi=1.0)
    assert abs(hip.sum(x) - BIG) <= 1e-5 * BIG
    # u64 sum of u32 counts past 2^31 elements: zeros (the f32 zero fill's bits) plus planted counts
    c = hip.empty((BIG,), "u32")
    from cleave_amd import _lib
    _lib.call("cleave_hip_zero_f32", c.ptr, c.size)
    for i, v in [(0, 1000), ((1 << 31) + 3, 4000000000), (BIG - 1, 123456789)]:
        c.sub(i, (1,)).upload(np.array([v], np.uint32))
    assert hip.sum_u64(c) == 1000 + 4000000000 + 123456789


def test_index_past_2pow31(hip, oracle):
    shape = (1 << 16, (1 << 15) + 1)  # 2^31 + 2^16 elements
    n = shape[0] * shape[1]
    print(f"index into {shape}", flush=True)
    t = hip.fill_uniform(hip.empty(shape), seed=21)
    for idx in [(shape[0] - 1, shape[1] - 1), (65535, 1), (40000, 30000)]:
        flat = idx[0] * shape[1] + idx[1]
        assert flat >= 1 << 31 or idx == (40000, 30000)
        assert hip.index(t, idx) == float(t.view((n,)).sub(flat, (1,)).numpy()[0]) == float(
            _uniform_at(oracle, 21, flat))
    dt = hip.zero(shape)
    hip.index_bwd(2.5, dt, (shape[0] - 1, 7))
    assert hip.index(dt, (shape[0] - 1, 7)) == 2.5


@pytest.mark.parametrize("dtype,M,K,tb,N", [("f32", 1 << 20, 1024, 0, 256), ("f32", 1 << 20, 1024, 1, 256),
                                           ("bf16", 1 << 21, 1024, 0, 256), ("bf16", 1 << 21, 1024, 1, 256),
                                           ("bf16", (1 << 21) + 5, 1024, 0, 260)])
def test_gemm_operand_past_4gib(hip, oracle, dtype, M, K, tb, N):
    # A (M x K) spans exactly 4 GiB, one byte past what a 32-bit offset from
    # the operand's base reaches; with tb, B (N x K) is k-contiguous too.
    # The product must still be the reference loop's, within the GEMM bound.
    # The ragged case is past the guarded-edge kernels' 2 GiB per operand and
    # B's rows are not whole 16-byte chunks: zero-padded copies of both
    # operands, the valid corner of C copied out.
    print(f"{dtype} gemm {M}x{N}x{K} tb={tb}: A spans {M * K * (4 if dtype == 'f32' else 2) / 2**30:.1f} GiB",
          flush=True)
    a32 = hip.fill_normal(hip.empty((M, K)), seed=31)
    b32 = hip.fill_normal(hip.empty((N, K) if tb else (K, N)), seed=32)
    if dtype == "bf16":
        a, b = hip.to_bf16(a32), hip.to_bf16(b32)
        del a32
    else:
        a, b = a32, b32
    c = hip.matmul(a, b, trans_b=bool(tb))
    rows = _samples(M, 5, 12)
    rows = rows[rows < M]
    Bh = b.numpy()
    Ar = np.stack([a.sub(int(r) * K, (K,)).numpy() for r in rows])
    Cr = np.stack([c.sub(int(r) * N, (N,)).numpy() for r in rows])
    if dtype == "bf16":
        Ar = oracle.bf16_to_f32(Ar).reshape(Ar.shape)
        Bh = oracle.bf16_to_f32(Bh).reshape(Bh.shape)
    ref = oracle.matmul(Ar, Bh, trans_b=bool(tb))
    den = np.abs(Ar).astype(np.float64) @ np.abs(Bh.T if tb else Bh).astype(np.float64)
    assert_gemm_close(Cr, ref, den, K, f"{dtype} rows {rows[:4]}...")


def test_escape_counts_past_2pow31_pixels(hip, oracle):
    w, h = 65536, 32769  # 2^31 + 2^16 pixels, 8 GiB of u32 counts
    x0, y0, dx, dy, it = -2.0, -1.5, 3.0 / w, 3.0 / h, 24
    print(f"escape counts {w}x{h}", flush=True)
    cnt = hip.escape_counts(w, h, x0, y0, dx, dy, it)
    for r in [0, 16384, 32768, h - 1]:
        got = cnt.sub(r * w, (w,)).numpy()
        ref = oracle.mandelbrot(w, h, x0, y0, np.float32(dx), np.float32(dy), it, rows=(r, r + 1))[r]
        assert np.array_equal(got, ref), r
