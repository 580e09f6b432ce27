"""cleave_hip_reduce_sum_f32_noalloc: the Sum that allocates nothing.

It must give what cleave_hip_reduce_sum_f32 gives (same kernels and grid, so
the same bits), within the sum tolerance of the oracle's left fold
(stdlib/nn/nn.cleave:111-117), on consecutive calls that share its static
workspace, the later ones smaller, and at every alignment of the input.
Called through the C ABI.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _noalloc_sum(lib, x, out):
    from cleave_amd import _lib

    st = lib.cleave_hip_reduce_sum_f32_noalloc(x.ptr, x.size, out.ptr)
    if st != 0:
        raise _lib.CleaveHipError(st, _lib.last_error()[1])
    return float(out.numpy()[0])


def test_noalloc_sum_matches_the_allocating_entry_on_consecutive_calls(hip, oracle):
    from cleave_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(71)
    out_a, out_b = hip.empty(1), hip.empty(1)
    # large first (the most partial sums: 16 blocks per CU), then ever smaller,
    # so a later call finds the earlier call's partials in the workspace
    for n in (1 << 24, 1000003, 4099, 7, 1):
        X = rng.standard_normal(n).astype(np.float32)
        x = hip.from_numpy(X)
        got = _noalloc_sum(lib, x, out_b)
        hip.reduce_sum(x, out_a)
        want = float(out_a.numpy()[0])
        assert got == want or (np.isnan(got) and np.isnan(want)), (n, got, want)
        ref = oracle.sum_f32(X)
        assert abs(got - ref) <= 1e-5 * np.abs(X).sum(dtype=np.float64), (n, got, ref)


def test_noalloc_sum_on_unaligned_views(hip, oracle):
    from helpers import view
    from cleave_amd import _lib

    lib = _lib.load()
    X = np.random.default_rng(72).standard_normal(70001).astype(np.float32)
    base = hip.from_numpy(X)
    out_a, out_b = hip.empty(1), hip.empty(1)
    for off in (1, 2, 3):  # 4, 8 and 12 bytes past a 16-byte boundary: the scalar stage-1 path
        n = X.size - off
        v = view(base, off, n)
        got = _noalloc_sum(lib, v, out_b)
        hip.reduce_sum(v, out_a)
        assert got == float(out_a.numpy()[0])
        assert abs(got - oracle.sum_f32(X[off:])) <= 1e-5 * np.abs(X[off:]).sum(dtype=np.float64)


def test_noalloc_sum_argument_errors(hip):
    from cleave_amd import _lib

    lib = _lib.load()
    x, out = hip.empty(8), hip.empty(1)
    assert lib.cleave_hip_reduce_sum_f32_noalloc(x.ptr, 0, out.ptr) == _lib.ERR_ARG
    assert lib.cleave_hip_reduce_sum_f32_noalloc(x.ptr, 8, None) == _lib.ERR_ARG
    # a length beyond the buffer's allocation is refused before any launch;
    # the overrun is kept to 40 bytes of a 4000-byte allocation, inside the
    # allocation's own page, so even a missing check could not fault
    y = hip.empty(1000)
    assert lib.cleave_hip_reduce_sum_f32_noalloc(y.ptr, 1010, out.ptr) == _lib.ERR_ARG
    assert "allocation" in _lib.last_error()[1]
