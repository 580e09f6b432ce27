"""The memref-descriptor entry points on the GPU: each must give exactly the
pointer form's result (the same kernels run), with transposed operands taken
from the descriptor's strides instead of flags."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mr(hip):
    from cleave_amd import memref
    return memref


def _rand(hip, shape, seed, dtype="f32"):
    a = np.random.default_rng(seed).standard_normal(shape).astype(np.float32)
    t = hip.from_numpy(a)
    return hip.to_bf16(t) if dtype == "bf16" else t


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_matmul_strides_select_the_transposed_forms(hip, mr, dtype, ta, tb):
    M, N, K = 96, 80, 64
    a = _rand(hip, (K, M) if ta else (M, K), 1, dtype)
    b = _rand(hip, (N, K) if tb else (K, N), 2, dtype)
    want = hip.matmul(a, b, trans_a=ta, trans_b=tb).numpy()
    c = hip.empty((M, N))
    da = mr.transposed(a) if ta else mr.of(a)
    db = mr.transposed(b) if tb else mr.of(b)
    mr.call("cleave_hip_matmul_" + dtype, da, db, mr.of(c))
    assert np.array_equal(c.numpy(), want)


def test_batched_matmul_rank3(hip, mr):
    bs, M, N, K = 3, 64, 48, 32
    a = _rand(hip, (bs, K, M), 3)  # transposed per entry
    b = _rand(hip, (bs, K, N), 4)
    want = hip.matmul_batched(a, b, trans_a=True).numpy()
    c = hip.empty((bs, M, N))
    mr.call("cleave_hip_matmul_f32", mr.transposed(a), mr.of(b), mr.of(c))
    assert np.array_equal(c.numpy(), want)
    ab, bb = _rand(hip, (bs, M, K), 5, "bf16"), _rand(hip, (bs, K, N), 6, "bf16")
    want = hip.matmul_batched(ab, bb).numpy()
    mr.call("cleave_hip_matmul_bf16", mr.of(ab), mr.of(bb), mr.of(c))
    assert np.array_equal(c.numpy(), want)


@pytest.mark.parametrize("name", ["add", "sub", "mul", "div", "sigmoid_bwd", "tanh_bwd", "relu_bwd"])
def test_binary_maps_match_pointer_forms(hip, mr, name):
    shape = (5, 7, 9)
    a, b = _rand(hip, shape, 7), _rand(hip, shape, 8)
    want = getattr(hip, name)(a, b).numpy()
    out = hip.empty(shape)
    mr.call(f"cleave_hip_{name}_f32", mr.of(a), mr.of(b), mr.of(out))
    assert np.array_equal(out.numpy(), want)


@pytest.mark.parametrize("name", ["neg", "relu", "sigmoid", "tanh"])
def test_unary_maps_match_pointer_forms(hip, mr, name):
    x = _rand(hip, (33, 17), 9)
    want = getattr(hip, name)(x).numpy()
    out = hip.empty((33, 17))
    mr.call(f"cleave_hip_{name}_f32", mr.of(x), mr.of(out))
    assert np.array_equal(out.numpy(), want)


def test_div_bwd_zero_and_sgd(hip, mr):
    a, b, g = _rand(hip, (4, 6), 10), _rand(hip, (4, 6), 11), _rand(hip, (4, 6), 12)
    wa, wb = (t.numpy() for t in hip.div_bwd(a, b, g))
    da, db = hip.empty((4, 6)), hip.empty((4, 6))
    mr.call("cleave_hip_div_bwd_f32", mr.of(a), mr.of(b), mr.of(g), mr.of(da), mr.of(db))
    assert np.array_equal(da.numpy(), wa) and np.array_equal(db.numpy(), wb)
    w = hip.from_numpy(a.numpy())
    mr.call("cleave_hip_sgd_update_f32", mr.of(w), mr.of(g), 0.25)
    assert np.array_equal(w.numpy(), hip.sgd_update(hip.from_numpy(a.numpy()), g, 0.25).numpy())
    mr.call("cleave_hip_zero_f32", mr.of(w))
    assert not w.numpy().any()


def test_row_bias_and_its_reverse_rule(hip, mr):
    a, b = _rand(hip, (40, 24), 16), _rand(hip, (24,), 17)
    want = hip.add_row_bias(a, b).numpy()
    out = hip.empty((40, 24))
    mr.call("cleave_hip_add_row_bias_f32", mr.of(a), mr.of(b, (1, 24)), mr.of(out))
    assert np.array_equal(out.numpy(), want)
    s = hip.empty((24,))
    mr.call("cleave_hip_sum_rows_f32", mr.of(a), mr.of(s))
    assert np.array_equal(s.numpy(), hip.sum_rows(a).numpy())


def test_reductions_match_pointer_forms(hip, mr):
    x = _rand(hip, (64, 129), 13)
    assert mr.call("cleave_hip_sum_f32", mr.of(x)) == hip.sum(x)
    assert mr.call("cleave_hip_mean_f32", mr.of(x)) == hip.mean(x)
    assert mr.call("cleave_hip_max_of_f32", mr.of(x)) == hip.max_of(x)
    assert mr.call("cleave_hip_argmax_f32", mr.of(x)) == hip.argmax(x)
    counts = hip.from_numpy(np.arange(1000, dtype=np.uint32).reshape(10, 100))
    assert mr.call("cleave_hip_sum_u32_u64", mr.of(counts)) == 999 * 1000 // 2


def test_index_and_its_reverse_rule(hip, mr, oracle):
    T = np.random.default_rng(14).standard_normal((3, 4, 5)).astype(np.float32)
    t = hip.from_numpy(T)
    for idx in [(0, 0, 0), (2, 3, 4), (1, 2, 3)]:
        assert mr.call("cleave_hip_index_f32", mr.of(t), mr.host(np.array(idx, np.int32))) == oracle.index(T, idx)
    dt = hip.zero((4, 6))
    want = np.zeros((4, 6), np.float32)
    for g, idx in [(2.5, (1, 2)), (0.5, (1, 2)), (-1.0, (3, 5))]:
        mr.call("cleave_hip_index_bwd_f32", g, mr.of(dt), mr.host(np.array(idx, np.int32)))
        oracle.index_bwd(g, want, idx)
    assert np.array_equal(dt.numpy(), want)


def test_mandelbrot_and_mlp_step(hip, mr):
    w, h = 96, 64
    d = np.float32(3.0 / w)
    want = hip.escape_counts(w, h, -2.0, -1.5, d, d, 200).numpy()
    out = hip.empty((h, w), "u32")
    mr.call("cleave_hip_mandelbrot_u32", mr.of(out), -2.0, -1.5, float(d), float(d), 200)
    assert np.array_equal(out.numpy(), want)
    B, D, H = 256, 64, 128
    rng = np.random.default_rng(15)
    X = rng.standard_normal((B, D)).astype(np.float32)
    Y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = rng.uniform(-0.1, 0.1, (D, H)).astype(np.float32)
    W2 = rng.uniform(-0.1, 0.1, H).astype(np.float32)
    x, y = hip.from_numpy(X), hip.from_numpy(Y)
    w1a, w2a, w1b, w2b = (hip.from_numpy(v) for v in (W1, W2, W1, W2))
    la, lb = hip.empty(1), hip.empty(1)
    hip.mlp_step(x, y, w1a, w2a, 0.05, loss=la)
    mr.call("cleave_hip_mlp_step_f32", mr.of(x), mr.of(y), mr.of(w1b), mr.of(w2b), None, None, mr.of(lb), 0.05)
    assert la.numpy()[0] == lb.numpy()[0]
    assert np.array_equal(w1a.numpy(), w1b.numpy()) and np.array_equal(w2a.numpy(), w2b.numpy())
