"""Elementwise maps and backward ops on the GPU vs the oracle.

IEEE ops (add/sub/mul/div/neg/relu and the backward forms built from them)
are bit-exact; sigmoid/tanh use the device exp/tanh and are within rel 1e-5.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import rel_close, view

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 5, 1023, 4097, (1 << 20) + 3]


def _rand(n, seed, lo=None):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32) * 3
    return x


def test_golden(hip, golden):
    for case in golden["elementwise_add"]:
        got = hip.add(hip.from_numpy(np.array(case["a"], np.float32)),
                      hip.from_numpy(np.array(case["b"], np.float32))).numpy()
        assert np.array_equal(got, np.array(case["out"], np.float32))
    act = golden["activations"]
    for fn in ("relu", "sigmoid", "tanh"):
        got = getattr(hip, fn)(hip.from_numpy(np.array(act[fn + "_in"], np.float32))).numpy()
        assert np.array_equal(got, np.array(act[fn + "_out"], np.float32)), fn


@pytest.mark.parametrize("n", SIZES)
def test_binary_ops_bit_exact(hip, oracle, n):
    a, b = _rand(n, 1), _rand(n, 2)
    b[b == 0] = 1.0
    da, db = hip.from_numpy(a), hip.from_numpy(b)
    for name in ("add", "sub", "mul", "div"):
        got = getattr(hip, name)(da, db).numpy()
        ref = getattr(oracle, name)(a, b)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (name, n)


@pytest.mark.parametrize("n", SIZES)
def test_unary_ops(hip, oracle, n):
    a = _rand(n, 3)
    da = hip.from_numpy(a)
    for name in ("neg", "relu"):
        got = getattr(hip, name)(da).numpy()
        assert np.array_equal(got.view(np.uint32), getattr(oracle, name)(a).view(np.uint32)), name
    assert rel_close(hip.sigmoid(da).numpy(), oracle.sigmoid(a), 1e-5)
    assert rel_close(hip.tanh(da).numpy(), oracle.tanh(a), 1e-5, atol=1e-30)


def test_special_values(hip, oracle):
    x = np.array([-0.0, 0.0, -2.0, 3.0, -np.inf, np.inf, np.nan, 1e-45, -1e-45, 88.0, -88.0, 104.0, -104.0],
                 np.float32)
    d = hip.from_numpy(x)
    r = hip.relu(d).numpy()
    ro = oracle.relu(x)
    assert np.array_equal(np.isnan(r), np.isnan(ro))
    m = ~np.isnan(ro)
    assert np.array_equal(r[m].view(np.uint32), ro[m].view(np.uint32))  # incl. +0 for -0
    assert rel_close(hip.sigmoid(d).numpy(), oracle.sigmoid(x), 1e-5, atol=1e-38)
    assert rel_close(hip.tanh(d).numpy(), oracle.tanh(x), 1e-5, atol=1e-38)


def test_backward_ops_bit_exact(hip, oracle):
    n = 100_003
    x = _rand(n, 4)
    g = _rand(n, 5)
    s = oracle.sigmoid(x)
    t = oracle.tanh(x)
    dx, dg, ds, dt = (hip.from_numpy(v) for v in (x, g, s, t))
    assert np.array_equal(hip.sigmoid_bwd(ds, dg).numpy(), oracle.sigmoid_bwd(s, g))
    assert np.array_equal(hip.tanh_bwd(dt, dg).numpy(), oracle.tanh_bwd(t, g))
    assert np.array_equal(hip.relu_bwd(dx, dg).numpy(), oracle.relu_bwd(x, g))
    b = np.abs(g) + 0.5
    da_, db_ = hip.div_bwd(dx, hip.from_numpy(b), dg)
    ra, rb = oracle.div_bwd(x, b, g)
    assert np.array_equal(da_.numpy(), ra) and np.array_equal(db_.numpy(), rb)


def test_sgd_update_and_zero(hip):
    n = 4099
    w = _rand(n, 6)
    g = _rand(n, 7)
    dw = hip.from_numpy(w)
    hip.sgd_update(dw, hip.from_numpy(g), 0.01)
    assert np.array_equal(dw.numpy(), w - np.float32(0.01) * g)
    z = hip.from_numpy(np.full(n, np.nan, np.float32))
    hip.zero(z)
    assert np.array_equal(z.numpy(), np.zeros(n, np.float32))


def test_misaligned_pointers_take_the_scalar_path(hip, oracle):
    n = 1001
    a, b = _rand(n + 1, 8), _rand(n + 1, 9)
    da, db = hip.from_numpy(a), hip.from_numpy(b)
    out = hip.empty(n + 1)
    hip.add(view(da, 1, n), view(db, 1, n), out=view(out, 1, n))
    assert np.array_equal(out.numpy()[1:], oracle.add(a[1:], b[1:]))
    hip.sigmoid(view(da, 1, n), out=view(out, 1, n))
    assert rel_close(out.numpy()[1:], oracle.sigmoid(a[1:]), 1e-5)


def test_hbm_sized_map(hip, oracle):
    n = (1 << 26) + 5  # 256 MiB per operand
    x = hip.fill_normal(hip.empty(n), seed=10)
    y = hip.sigmoid(x)
    X, Y = x.numpy(), y.numpy()
    idx = np.random.default_rng(0).integers(0, n, 1 << 20)
    assert rel_close(Y[idx], oracle.sigmoid(X[idx]), 1e-5)
    assert rel_close(Y[-5:], oracle.sigmoid(X[-5:]), 1e-5)
    z = hip.add(x, y).numpy()
    assert np.array_equal(z[idx], X[idx] + Y[idx]) and np.array_equal(z[-5:], X[-5:] + Y[-5:])


def test_index_reads_row_major_elements(hip, oracle):
    # Index::index over a rank-3 tensor (tensor.extract, row-major flattening)
    rng = np.random.default_rng(21)
    T = rng.standard_normal((3, 4, 5)).astype(np.float32)
    t = hip.from_numpy(T)
    for idx in [(0, 0, 0), (2, 3, 4), (1, 2, 3), (0, 3, 1), (2, 0, 4)]:
        assert hip.index(t, idx) == oracle.index(T, idx)
    with pytest.raises(hip.CleaveHipError):
        hip.index(t, (3, 0, 0))


def test_index_bwd_is_the_reverse_of_the_index_rule(hip, oracle):
    # derivative index(c, idx): index(d(c), idx) -> dL/dc = g at idx, 0 elsewhere;
    # repeated reads of one element accumulate
    dt = hip.zero((4, 6))
    want = np.zeros((4, 6), np.float32)
    for g, idx in [(2.5, (1, 2)), (0.5, (1, 2)), (-1.0, (3, 5))]:
        hip.index_bwd(g, dt, idx)
        oracle.index_bwd(g, want, idx)
    assert np.array_equal(dt.numpy(), want)


@pytest.mark.parametrize("rows,cols", [(1, 8), (37, 64), (1000, 1028), (513, 100), (64, 4096), (7, 13), (300, 3)])
def test_add_row_bias_matches_the_oracle_bitwise(hip, oracle, rows, cols):
    # vector path (cols % 4 == 0) and the scalar path (cols = 13, 3)
    rng = np.random.default_rng(rows * 131 + cols)
    A = rng.standard_normal((rows, cols)).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32)
    out = hip.add_row_bias(hip.from_numpy(A), hip.from_numpy(b)).numpy()
    assert np.array_equal(out, oracle.add_row_bias(A, b))


@pytest.mark.parametrize("rows,cols", [(1, 8), (3, 64), (5, 256), (9, 4096), (37, 64), (1000, 1028), (4097, 96),
                                       (7, 13), (300, 3)])
def test_sum_rows_against_the_left_fold(hip, oracle, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    # integer-valued cotangents: every summation order is exact, so bit-equal
    G = rng.integers(-512, 512, (rows, cols)).astype(np.float32)
    assert np.array_equal(hip.sum_rows(hip.from_numpy(G)).numpy(), oracle.sum_rows(G))
    # general values: within the sum tolerance, relative to sum |g| per column
    G = rng.standard_normal((rows, cols)).astype(np.float32)
    got = hip.sum_rows(hip.from_numpy(G)).numpy().astype(np.float64)
    want = oracle.sum_rows(G).astype(np.float64)
    scale = np.abs(G).astype(np.float64).sum(axis=0)
    assert np.all(np.abs(got - want) <= 1e-5 * scale + 1e-30)


def test_sum_rows_is_deterministic_and_at_full_size(hip):
    # the H-sized cotangent of config 4's hidden layer: sums of a constant are exact
    g = hip.empty((65536, 4096))
    hip.fill_uniform(g, seed=5, lo=0.25, hi=0.25)
    s1 = hip.sum_rows(g).numpy()
    assert np.all(s1 == np.float32(0.25 * 65536))
    x = hip.fill_normal(hip.empty((8192, 1024)), seed=6)
    a, b = hip.sum_rows(x).numpy(), hip.sum_rows(x).numpy()
    assert np.array_equal(a, b)
