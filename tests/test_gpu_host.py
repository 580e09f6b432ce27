"""The host-array entry points (`cleave_hip_*_host`) on the GPU, against the oracle.

These are the entry points an `extern(...)` declaration binds: cleave passes an
array as the aligned pointer of a host memref plus its length
(/root/reference/cleave/src/mlir_lower.rs:1720-1751) and cleave-rt reads host
memory (/root/reference/cleave-rt/src/lib.rs:86-90).  Every call here hands
numpy host arrays straight to the C ABI (through cleave_amd.host) and compares
the result with the oracle's restated loops.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from helpers import assert_gemm_close, assert_mlp_grads_close, rel_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def host(hip):
    from cleave_amd import host as h
    return h


def _absden(A, B, ta=False, tb=False):
    Ad = np.abs(A.T if ta else A).astype(np.float64)
    Bd = np.abs(B.T if tb else B).astype(np.float64)
    return Ad @ Bd


def test_config1_matmul_256_seed0_host_arrays(host, oracle):
    # A and B are the first and second 256^2 draws of the
    # seed-0 uniform[-1,1) stream, held in host memory as cleave holds them.
    n = 256
    ab = oracle.uniform(2 * n * n, seed=0)
    A, B = ab[:n * n].reshape(n, n), ab[n * n:].reshape(n, n)
    got = host.matmul(A, B)
    ref = oracle.matmul(A, B)
    assert_gemm_close(got, ref, _absden(A, B), n, "host 256^3")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_matmul_f32_host_layouts(host, oracle, ta, tb):
    rng = np.random.default_rng(10 + 2 * ta + tb)
    M, N, K = 300, 260, 70
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    got = host.matmul(A, B, trans_a=bool(ta), trans_b=bool(tb))
    ref = oracle.matmul(A, B, trans_a=bool(ta), trans_b=bool(tb))
    assert_gemm_close(got, ref, _absden(A, B, ta, tb), K, f"host f32 ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_matmul_bf16_host(host, oracle, ta, tb):
    rng = np.random.default_rng(20 + ta)
    M, N, K = 256, 384, 128
    A = oracle.to_bf16(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    B = oracle.to_bf16(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
    got = host.matmul(A, B, trans_a=bool(ta), trans_b=bool(tb))
    Au, Bu = oracle.bf16_to_f32(A).reshape(A.shape), oracle.bf16_to_f32(B).reshape(B.shape)
    ref = oracle.matmul(Au, Bu, trans_a=bool(ta), trans_b=bool(tb))
    assert_gemm_close(got, ref, _absden(Au, Bu, ta, tb), K, "host bf16")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_matmul_batched_host_transposed(host, oracle, dtype):
    rng = np.random.default_rng(30)
    bsz, M, N, K = 3, 128, 96, 64
    A = rng.standard_normal((bsz, K, M)).astype(np.float32)  # trans_a: entries stored K x M
    B = rng.standard_normal((bsz, N, K)).astype(np.float32)  # trans_b: entries stored N x K
    if dtype == "bf16":
        A, B = oracle.to_bf16(A), oracle.to_bf16(B)
    got = host.matmul_batched(A, B, trans_a=True, trans_b=True)
    for i in range(bsz):
        Ai, Bi = A[i], B[i]
        if dtype == "bf16":
            Ai, Bi = oracle.bf16_to_f32(Ai).reshape(K, M), oracle.bf16_to_f32(Bi).reshape(N, K)
        ref = oracle.matmul(Ai, Bi, trans_a=True, trans_b=True)
        assert_gemm_close(got[i], ref, _absden(Ai, Bi, True, True), K, f"host batched {dtype} #{i}")


def test_maps_host_bit_exact(host, oracle):
    rng = np.random.default_rng(40)
    a = rng.standard_normal(4099).astype(np.float32)
    b = rng.standard_normal(4099).astype(np.float32)
    s = oracle.sigmoid(a)
    for name in ("add", "sub", "mul", "div"):
        assert np.array_equal(getattr(host, name)(a, b), getattr(oracle, name)(a, b)), name
    for name in ("neg", "relu"):
        assert np.array_equal(getattr(host, name)(a), getattr(oracle, name)(a)), name
    for name, x in (("sigmoid_bwd", s), ("tanh_bwd", np.tanh(a).astype(np.float32)), ("relu_bwd", a)):
        assert np.array_equal(getattr(host, name)(x, b), getattr(oracle, name)(x, b)), name
    assert rel_close(host.sigmoid(a), oracle.sigmoid(a), 1e-5)
    assert rel_close(host.tanh(a), oracle.tanh(a), 1e-5, 1e-7)
    da, db = host.div_bwd(a, b, s)
    rda, rdb = oracle.div_bwd(a, b, s)
    assert np.array_equal(da, rda) and np.array_equal(db, rdb)
    assert np.array_equal(host.zero(17), np.zeros(17, np.float32))


def test_sgd_and_bias_host(host, oracle):
    rng = np.random.default_rng(41)
    w = rng.standard_normal(1000).astype(np.float32)
    g = rng.standard_normal(1000).astype(np.float32)
    expect = (w - np.float32(0.01) * g).astype(np.float32)
    host.sgd_update(w, g, 0.01)
    assert np.array_equal(w, expect)
    m = rng.standard_normal((37, 64)).astype(np.float32)
    bias = rng.standard_normal(64).astype(np.float32)
    assert np.array_equal(host.add_row_bias(m, bias), oracle.add_row_bias(m, bias))
    got = host.sum_rows(m)
    ref = oracle.sum_rows(m)
    assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(m).sum(axis=0))


def test_reductions_host(host, oracle):
    rng = np.random.default_rng(42)
    v = rng.standard_normal(100003).astype(np.float32)
    assert abs(host.sum(v) - oracle.sum_f32(v)) <= 1e-5 * np.abs(v).sum()
    assert abs(host.mean(v) - oracle.mean_f32(v)) <= 1e-5 * np.abs(v).sum() / v.size
    assert host.max_of(v) == oracle.max_of(v)
    assert host.argmax(v) == oracle.argmax(v)
    # the reference's own vector (cleave/tests/mlir_lower.rs:2441-2451)
    t = np.array([1, 5, 3], np.float32)
    assert (host.sum(t), host.mean(t), host.max_of(t)) == (9.0, 3.0, 5.0)
    counts = rng.integers(0, 1001, 77777, dtype=np.uint32)
    assert host.sum_u64(counts) == oracle.sum_u64(counts)


def test_index_host(host, oracle):
    rng = np.random.default_rng(43)
    t = rng.standard_normal((3, 5, 7)).astype(np.float32)
    for idx in [(0, 0, 0), (2, 4, 6), (1, 3, 2)]:
        assert host.index(t, idx) == oracle.index(t, idx)
    dt = np.zeros((3, 5, 7), np.float32)
    host.index_bwd(2.5, dt, (1, 2, 3))
    ref = np.zeros((3, 5, 7), np.float32)
    oracle.index_bwd(2.5, ref, (1, 2, 3))
    assert np.array_equal(dt, ref)


def test_escape_counts_host_bit_exact(host, oracle):
    w, h = 128, 96
    got = host.escape_counts(w, h, -2.0, -1.5, 3.0 / w, 3.0 / h, 200)
    assert np.array_equal(got, oracle.mandelbrot(w, h, -2.0, -1.5, 3.0 / w, 3.0 / h, 200))


def test_mlp_step_host(host, oracle):
    rng = np.random.default_rng(44)
    B, D, Hd = 64, 32, 48
    X = rng.standard_normal((B, D)).astype(np.float32)
    y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = rng.uniform(-0.3, 0.3, (D, Hd)).astype(np.float32)
    W2 = rng.uniform(-0.3, 0.3, Hd).astype(np.float32)
    lossr, dW1r, dW2r, W1r, W2r = oracle.mlp_step(X, y, W1, W2, lr=0.01)
    w1, w2 = W1.copy(), W2.copy()
    loss, dw1, dw2 = host.mlp_step(X, y, w1, w2, 0.01)
    assert abs(loss - lossr) <= 1e-5 * abs(lossr)
    assert_mlp_grads_close(dw1, dw2, dW1r, dW2r, X, y, W1, W2, "host")
    assert np.array_equal(w1, W1 - np.float32(0.01) * dw1)
    assert np.array_equal(w2, W2 - np.float32(0.01) * dw2)


def test_large_host_arrays_through_the_bounce_buffers(host, oracle):
    # Copies above 4 MiB go through two pinned 16 MiB bounce buffers in
    # chunks, host threads copying one while the DMA engine moves the other.
    # Lengths with a ragged last chunk, an exact multiple of the chunk, several
    # operands per call, in place (sgd_update), and an output-only array.
    rng = np.random.default_rng(123)
    n = (1 << 24) + 13  # 64 MiB + 52 B: five chunks, the last one short
    a = rng.standard_normal(n, dtype=np.float32)
    b = rng.standard_normal(n, dtype=np.float32)
    assert np.array_equal(host.add(a, b), oracle.add(a, b))
    assert np.array_equal(host.sub(a, b), oracle.sub(a, b))
    s = host.sum(a)
    assert abs(s - oracle.sum_f32(a)) <= 1e-5 * float(np.sum(np.abs(a), dtype=np.float64))
    assert host.max_of(a) == oracle.max_of(a)
    w = b.copy()
    host.sgd_update(w, a, 0.01)
    assert np.array_equal(w, b - np.float32(0.01) * a)
    m = 2048  # 16 MiB operands: exactly one chunk each
    A = rng.standard_normal((m, 256), dtype=np.float32)
    B = rng.standard_normal((256, m), dtype=np.float32)
    got = host.matmul(A, B)  # 16 MiB output
    ref = oracle.matmul(A, B, threads=16)
    assert_gemm_close(got, ref, _absden(A, B), 256, "host matmul with 16 MiB output")
    w_, h_ = 4096, 4097  # 64 MiB of counts, output only
    cnt = host.escape_counts(w_, h_, -2.0, -1.5, 3.0 / w_, 3.0 / h_, 64)
    ref = oracle.mandelbrot(w_, h_, -2.0, -1.5, np.float32(3.0 / w_), np.float32(3.0 / h_), 64, threads=16)
    assert np.array_equal(cnt.reshape(h_, w_), ref)


def test_host_copies_whose_split_leaves_a_tail(host, oracle):
    # 2,621,441 floats = 10,485,764 bytes: one bounce chunk split over up to 5
    # copying threads.  A split that rounded n / parts down to 64 bytes left
    # the last 4 bytes uncopied here (stale input on the way in, an unwritten
    # output element on the way out).
    rng = np.random.default_rng(321)
    n = 2621441
    a = rng.standard_normal(n, dtype=np.float32)
    b = rng.standard_normal(n, dtype=np.float32)
    got = host.add(a, b)
    assert np.array_equal(got, oracle.add(a, b))
    assert got[-1] == a[-1] + b[-1]
    s = host.sum(a)
    assert abs(s - oracle.sum_f32(a)) <= 1e-5 * float(np.sum(np.abs(a), dtype=np.float64))
    for m in (n - 1, n + 1, 3 * 1048576 + 5, 4 * 1048576 - 3):  # other ragged splits around it
        x = rng.standard_normal(m, dtype=np.float32)
        assert np.array_equal(host.neg(x), -x), m


def test_host_forms_take_empty_arrays(host):
    e = np.empty(0, np.float32)
    assert host.add(e, e).size == 0 and host.relu(e).size == 0


def test_device_entries_refuse_host_arrays_on_copy_only_paths(hip):
    # The device entry points check every operand's memory kind before any
    # device work.  Exercised only where the entry point would do no more than
    # a copy without the check (Index reads one element with a copy; upload
    # and download are copies), so no kernel can see a host address.
    from cleave_amd import _lib

    lib = _lib.load()
    t = np.arange(12, dtype=np.float32).reshape(3, 4)
    dims = np.array([3, 4], np.int32)
    idx = np.array([1, 2], np.int32)
    v = lib.cleave_hip_index_f32(t.ctypes.data, t.size, dims.ctypes.data, 2, idx.ctypes.data, 2)
    code, msg = _lib.last_error()
    assert v != v and code == _lib.ERR_ARG and "not device memory" in msg, msg
    other = np.zeros(16, np.float32)
    n = lib.cleave_hip_upload(other.ctypes.data, t.ctypes.data, 16)
    code, msg = _lib.last_error()
    assert n == _lib.ERR_ARG and "not device memory" in msg, msg
    # device memory, and views inside it, pass
    d = hip.from_numpy(t.ravel())
    assert hip.index(d.view((3, 4)), (1, 2)) == 6.0
    out = np.zeros(4, np.float32)
    assert lib.cleave_hip_download(out.ctypes.data, d.ptr + 16, 16) == 16
    assert np.array_equal(out, t.ravel()[4:8])
