"""The library's device buffers (cleave_hip_buf_alloc / cleave_hip_buf_free,
runtime.hip): freed buffers are cached and reused by later allocations of the
same size without a device synchronisation; the bytes a buffer was allocated
with still bound what a device entry point may read from it."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_a_freed_buffer_is_reused_for_the_same_size(hip):
    from cleave_amd._lib import load
    lib = load()
    size = (97 << 20) + 3  # a size class no other test uses
    p = lib.cleave_hip_buf_alloc(size)
    lib.cleave_hip_buf_free(p)
    q = lib.cleave_hip_buf_alloc(size)
    assert q == p
    r = lib.cleave_hip_buf_alloc(size)  # the cached block is taken: a new one
    assert r != q
    lib.cleave_hip_buf_free(q)
    lib.cleave_hip_buf_free(r)


def test_reuse_while_earlier_work_is_queued_stays_ordered(hip):
    # A buffer freed while queued work still reads it, then reallocated and
    # overwritten by later work: the stream runs the reads first.
    n = 1 << 24
    rng = np.random.default_rng(0)
    X = rng.standard_normal(n).astype(np.float32)
    Y = rng.standard_normal(n).astype(np.float32)
    outs = []
    for _ in range(4):
        a = hip.from_numpy(X)
        b = hip.empty(n)
        outs.append(hip.add(a, a, out=b))  # queued
        del a  # freed into the cache while the add may still be queued
        c = hip.from_numpy(Y)  # likely the same block, overwritten after the add
        outs.append(hip.neg(c))
        del c
    for i, o in enumerate(outs):
        want = (X + X) if i % 2 == 0 else -Y
        assert np.array_equal(o.numpy(), want)


def test_operands_are_bounded_by_the_bytes_asked_for(hip):
    # 1000 floats live in a block rounded up to 4096 bytes; an entry point told
    # the operand holds 1010 floats must refuse it, not read the padding.
    from cleave_amd._lib import load
    lib = load()
    t = hip.from_numpy(np.ones(1000, np.float32))
    o = hip.empty(1010)
    assert lib.cleave_hip_neg_f32(t.ptr, 1010, o.ptr, 1010) == -2  # CLEAVE_HIP_ERR_ARG
    assert "needs 4040 bytes" in lib.cleave_hip_last_error_message().decode()
    assert lib.cleave_hip_neg_f32(t.ptr, 1000, o.ptr, 1000) == 0
    hip.sync()
    assert np.array_equal(o.numpy()[:1000], -np.ones(1000, np.float32))
