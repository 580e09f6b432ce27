"""The memref-descriptor entry points on the GPU, each compared with the oracle
directly (never with another HIP entry point).  Transposed operands reach the
A B^T / A^T B products through the descriptor's strides alone
(/root/reference/cleave/src/mlir_lower.rs:1702-1713 is where a Tensor would
cross `extern` as a memref)."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_gemm_close, assert_mlp_grads_close, rel_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mr(hip):
    from cleave_amd import memref
    return memref


def _np(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def _dev(hip, oracle, arr, dtype="f32"):
    """Device copy of arr; for bf16, the RNE bit patterns and their upcast values."""
    if dtype == "bf16":
        bits = oracle.to_bf16(arr)
        return hip.from_numpy(bits, "bf16"), oracle.bf16_to_f32(bits).reshape(arr.shape)
    return hip.from_numpy(arr), arr


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(96, 80, 64), (256, 256, 128), (33, 17, 9)])
def test_matmul_strides_select_the_transposed_forms(hip, mr, oracle, dtype, ta, tb, M, N, K):
    A = _np((K, M) if ta else (M, K), 1 + M)
    B = _np((N, K) if tb else (K, N), 2 + N)
    a, Au = _dev(hip, oracle, A, dtype)
    b, Bu = _dev(hip, oracle, B, dtype)
    c = hip.empty((M, N))
    da = mr.transposed(a) if ta else mr.of(a)
    db = mr.transposed(b) if tb else mr.of(b)
    mr.call("cleave_hip_matmul_" + dtype, da, db, mr.of(c))
    ref = oracle.matmul(Au, Bu, trans_a=ta, trans_b=tb)
    den = np.abs(Au.T if ta else Au).astype(np.float64) @ np.abs(Bu.T if tb else Bu).astype(np.float64)
    assert_gemm_close(c.numpy(), ref, den, K, f"memref {dtype} {M}x{N}x{K} ta={ta} tb={tb}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_batched_matmul_rank3(hip, mr, oracle, dtype, ta, tb):
    bs, M, N, K = 3, 64, 48, 32
    A = _np((bs, K, M) if ta else (bs, M, K), 3)
    B = _np((bs, N, K) if tb else (bs, K, N), 4)
    a, Au = _dev(hip, oracle, A, dtype)
    b, Bu = _dev(hip, oracle, B, dtype)
    c = hip.empty((bs, M, N))
    mr.call("cleave_hip_matmul_" + dtype, mr.transposed(a) if ta else mr.of(a),
            mr.transposed(b) if tb else mr.of(b), mr.of(c))
    got = c.numpy()
    for i in range(bs):
        ref = oracle.matmul(Au[i], Bu[i], trans_a=ta, trans_b=tb)
        den = (np.abs(Au[i].T if ta else Au[i]).astype(np.float64)
               @ np.abs(Bu[i].T if tb else Bu[i]).astype(np.float64))
        assert_gemm_close(got[i], ref, den, K, f"memref batched {dtype} #{i}")


@pytest.mark.parametrize("name", ["add", "sub", "mul", "div", "sigmoid_bwd", "tanh_bwd", "relu_bwd"])
def test_binary_maps_bit_exact(hip, mr, oracle, name):
    shape = (5, 7, 9)
    A, B = _np(shape, 7), _np(shape, 8)
    if name == "sigmoid_bwd":
        A = oracle.sigmoid(A)
    elif name == "tanh_bwd":
        A = oracle.tanh(A)
    a, b = hip.from_numpy(A), hip.from_numpy(B)
    out = hip.empty(shape)
    mr.call(f"cleave_hip_{name}_f32", mr.of(a), mr.of(b), mr.of(out))
    assert np.array_equal(out.numpy(), getattr(oracle, name)(A, B))


@pytest.mark.parametrize("name", ["neg", "relu", "sigmoid", "tanh"])
def test_unary_maps(hip, mr, oracle, name):
    X = _np((33, 17), 9) * 4
    x = hip.from_numpy(X)
    out = hip.empty((33, 17))
    mr.call(f"cleave_hip_{name}_f32", mr.of(x), mr.of(out))
    ref = getattr(oracle, name)(X)
    if name in ("neg", "relu"):
        assert np.array_equal(out.numpy(), ref)
    else:  # device expf/tanhf against libm: rel 1e-5
        assert rel_close(out.numpy(), ref, 1e-5, 1e-7)


def test_div_bwd_zero_and_sgd(hip, mr, oracle):
    A, B, G = _np((4, 6), 10), _np((4, 6), 11), _np((4, 6), 12)
    a, b, g = (hip.from_numpy(v) for v in (A, B, G))
    da, db = hip.empty((4, 6)), hip.empty((4, 6))
    mr.call("cleave_hip_div_bwd_f32", mr.of(a), mr.of(b), mr.of(g), mr.of(da), mr.of(db))
    rda, rdb = oracle.div_bwd(A, B, G)
    assert np.array_equal(da.numpy(), rda) and np.array_equal(db.numpy(), rdb)
    # SGD is the oracle MLP step's update, w - lr * g in f32 (pinned in test_oracle.py)
    w = hip.from_numpy(A)
    mr.call("cleave_hip_sgd_update_f32", mr.of(w), mr.of(g), 0.25)
    assert np.array_equal(w.numpy(), A - np.float32(0.25) * G)
    mr.call("cleave_hip_zero_f32", mr.of(w))
    assert np.array_equal(w.numpy(), np.zeros((4, 6), np.float32))


def test_row_bias_and_its_reverse_rule(hip, mr, oracle):
    A, Bv = _np((40, 24), 16), _np((24,), 17)
    a, b = hip.from_numpy(A), hip.from_numpy(Bv)
    out = hip.empty((40, 24))
    mr.call("cleave_hip_add_row_bias_f32", mr.of(a), mr.of(b, (1, 24)), mr.of(out))
    assert np.array_equal(out.numpy(), oracle.add_row_bias(A, Bv))
    s = hip.empty((24,))
    mr.call("cleave_hip_sum_rows_f32", mr.of(a), mr.of(s))
    assert np.all(np.abs(s.numpy() - oracle.sum_rows(A)) <= 1e-5 * np.abs(A).sum(axis=0))


def test_reductions(hip, mr, oracle):
    X = _np((64, 129), 13)
    x = hip.from_numpy(X)
    scale = np.abs(X).sum(dtype=np.float64)
    assert abs(mr.call("cleave_hip_sum_f32", mr.of(x)) - oracle.sum_f32(X)) <= 1e-5 * scale
    assert abs(mr.call("cleave_hip_mean_f32", mr.of(x)) - oracle.mean_f32(X)) <= 1e-5 * scale / X.size
    assert mr.call("cleave_hip_max_of_f32", mr.of(x)) == oracle.max_of(X)
    assert mr.call("cleave_hip_argmax_f32", mr.of(x)) == oracle.argmax(X)
    C = np.random.default_rng(18).integers(0, 1001, (10, 100), dtype=np.uint32)
    counts = hip.from_numpy(C)
    assert mr.call("cleave_hip_sum_u32_u64", mr.of(counts)) == oracle.sum_u64(C)


def test_index_and_its_reverse_rule(hip, mr, oracle):
    T = _np((3, 4, 5), 14)
    t = hip.from_numpy(T)
    for idx in [(0, 0, 0), (2, 3, 4), (1, 2, 3)]:
        assert mr.call("cleave_hip_index_f32", mr.of(t), mr.host(np.array(idx, np.int32))) == oracle.index(T, idx)
    dt = hip.zero((4, 6))
    want = np.zeros((4, 6), np.float32)
    for g, idx in [(2.5, (1, 2)), (0.5, (1, 2)), (-1.0, (3, 5))]:
        mr.call("cleave_hip_index_bwd_f32", g, mr.of(dt), mr.host(np.array(idx, np.int32)))
        oracle.index_bwd(g, want, idx)
    assert np.array_equal(dt.numpy(), want)


def test_mandelbrot(hip, mr, oracle):
    w, h = 96, 64
    d = np.float32(3.0 / w)
    out = hip.empty((h, w), "u32")
    mr.call("cleave_hip_mandelbrot_u32", mr.of(out), -2.0, -1.5, float(d), float(d), 200)
    assert np.array_equal(out.numpy(), oracle.mandelbrot(w, h, -2.0, -1.5, d, d, 200))


@pytest.mark.parametrize("B,D,H", [(256, 64, 128), (512, 256, 512)])  # unfused, fused
def test_mlp_step(hip, mr, oracle, B, D, H):
    rng = np.random.default_rng(15 + B)
    X = rng.standard_normal((B, D)).astype(np.float32)
    Y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = rng.uniform(-0.1, 0.1, (D, H)).astype(np.float32)
    W2 = rng.uniform(-0.1, 0.1, H).astype(np.float32)
    lr = 0.05
    loss_r, dW1_r, dW2_r, W1_r, W2_r = oracle.mlp_step(X, Y, W1, W2, lr=lr, threads=16)
    x, y, w1, w2 = (hip.from_numpy(v) for v in (X, Y, W1, W2))
    dw1, dw2, loss = hip.empty((D, H)), hip.empty(H), hip.empty(1)
    mr.call("cleave_hip_mlp_step_f32", mr.of(x), mr.of(y), mr.of(w1), mr.of(w2), mr.of(dw1), mr.of(dw2),
            mr.of(loss), lr)
    assert abs(loss.numpy()[0] - loss_r) <= 1e-5 * abs(loss_r)
    g1, g2 = dw1.numpy(), dw2.numpy()
    assert_mlp_grads_close(g1, g2, dW1_r, dW2_r, X, Y, W1, W2, f"memref B={B}")
    assert np.array_equal(w1.numpy(), W1 - np.float32(lr) * g1)
    assert np.array_equal(w2.numpy(), W2 - np.float32(lr) * g2)


def test_broadcast_forms(hip, oracle):
    # the _bcast maps and sum_to_shape on descriptors: each operand keeps its
    # own sizes, out holds the broadcast shape
    import cleave_amd.memref as mr

    rng = np.random.default_rng(61)
    A = rng.standard_normal((6, 1, 40)).astype(np.float32)
    B = (rng.standard_normal((5, 1)) + 3).astype(np.float32)
    a, b, out = hip.from_numpy(A), hip.from_numpy(B), hip.empty((6, 5, 40))
    for op in ("add", "sub", "mul", "div"):
        mr.call(f"cleave_hip_{op}_bcast_f32", mr.of(a), mr.of(b), mr.of(out))
        assert np.array_equal(out.numpy(), oracle.bcast(op, A, B)), op
    with pytest.raises(Exception, match="broadcast"):
        mr.call("cleave_hip_add_bcast_f32", mr.of(a), mr.of(b), mr.of(hip.empty((6, 40, 5))))
    s = hip.empty((1, 5, 1))
    mr.call("cleave_hip_sum_to_shape_f32", mr.of(out), mr.of(s))
    O = out.numpy()
    want = O.astype(np.float64).sum(axis=(0, 2), keepdims=True)
    assert np.all(np.abs(s.numpy() - want) <= 1e-6 * 240 * np.abs(O).astype(np.float64).sum(axis=(0, 2),
                                                                                              keepdims=True))
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    a64, b64, o64 = hip.from_numpy(A64), hip.from_numpy(B64), hip.empty((6, 5, 40), "f64")
    mr.call("cleave_hip_mul_bcast_f64", mr.of(a64), mr.of(b64), mr.of(o64))
    assert np.array_equal(o64.numpy(), oracle.bcast("mul", A64, B64, f64=True))
