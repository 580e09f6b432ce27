"""The library's device buffers (cleave_hip_buf_alloc / cleave_hip_buf_free,
runtime.hip): freed buffers are cached and reused by later allocations of the
same size without a device synchronisation; the bytes a buffer was allocated
with still bound what a device entry point may read from it; a pointer into a
freed block is refused; the cache goes back to the device on request and
before library scratch would fail to grow."""
from __future__ import annotations

import ctypes as C

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


def test_a_pointer_into_a_freed_buffer_is_refused(hip):
    from cleave_amd._lib import ERR_ARG, load
    lib = load()
    size = (3 << 20) + 4 * 7  # a size class no other test uses
    p = lib.cleave_hip_buf_alloc(size)
    o = lib.cleave_hip_buf_alloc(size)
    assert lib.cleave_hip_neg_f32(p, 1000, o, 1000) == 0
    hip.sync()
    lib.cleave_hip_buf_free(p)
    for ptr in (p, p + 4096):  # the block's base and a view inside it
        assert lib.cleave_hip_neg_f32(ptr, 100, o, 100) == ERR_ARG
        assert "freed" in lib.cleave_hip_last_error_message().decode()
    lib.cleave_hip_buf_free(o)


def test_trim_returns_the_cache_to_the_device(hip):
    from cleave_amd._lib import load
    lib = load()
    lib.cleave_hip_buf_trim()
    assert lib.cleave_hip_buf_cached_bytes() == 0
    size = (5 << 20) + 12
    p = lib.cleave_hip_buf_alloc(size)
    lib.cleave_hip_buf_free(p)
    held = lib.cleave_hip_buf_cached_bytes()
    assert held >= size
    assert lib.cleave_hip_buf_trim() == held
    assert lib.cleave_hip_buf_cached_bytes() == 0
    q = lib.cleave_hip_buf_alloc(size)  # a fresh block, usable
    assert q
    lib.cleave_hip_buf_free(q)


def test_scratch_growth_takes_back_the_cache_when_the_device_is_full(hip):
    # 8 GiB of freed buffers wait in the cache; the rest of the device is
    # taken by plain hipMalloc blocks until under 1.5 GiB is free.  A host-array
    # add whose staging needs 6 GiB of library scratch must then return the
    # cache to the device and succeed, instead of failing with ERR_OOM.
    from cleave_amd import host
    from cleave_amd._lib import load
    lib = load()
    hiprt = C.CDLL("libamdhip64.so")
    hiprt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    hiprt.hipFree.argtypes = [C.c_void_p]
    hiprt.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    GiB = 1 << 30
    free, total = C.c_size_t(), C.c_size_t()

    def free_now():
        assert hiprt.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
        return free.value

    lib.cleave_hip_buf_trim()
    blk = lib.cleave_hip_buf_alloc(8 * GiB)
    assert blk
    lib.cleave_hip_buf_free(blk)
    assert lib.cleave_hip_buf_cached_bytes() >= 8 * GiB
    hog = []
    try:
        while free_now() > 3 * GiB // 2:
            chunk = min(free.value - GiB, 32 * GiB) & ~((1 << 21) - 1)
            p = C.c_void_p()
            if chunk <= 0 or hiprt.hipMalloc(C.byref(p), chunk) != 0:
                break
            hog.append(p)
        assert free_now() <= 3 * GiB // 2, f"could not fill the device ({free.value} bytes free)"
        n = (2 * GiB) // 4  # a, b and the output: 6 GiB of staging
        a = np.full(n, 1.5, np.float32)
        b = np.full(n, 2.25, np.float32)
        out = host.add(a, b)  # raises CleaveHipError on ERR_OOM
        assert out[0] == 3.75 and out[-1] == 3.75 and out[n // 2] == 3.75
        assert lib.cleave_hip_buf_cached_bytes() == 0
    finally:
        for p in hog:
            hiprt.hipFree(p)
