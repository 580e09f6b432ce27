"""Pins the f64 forms of the CPU oracle (oracle/oracle.c, the Tensor<f64, ...>
section) before the device's f64 path is checked against them.

Each check is one a plausible slip would fail: the reference's known-answer
vectors in f64, witnesses of the operation order (an unfused mul/add, a left
fold from v[0]) that a contracted or reassociated loop gets wrong, brute force
in extended precision, closed forms and special values of exp/tanh, finite
differences of the backward rules, and numpy's own row-major indexing."""
from __future__ import annotations

import math

import numpy as np
import pytest

EPS = np.finfo(np.float64).eps


def test_matmul_golden_vectors(oracle, golden):
    for g in golden["matmul"]:
        A = np.array(g["a"], np.float64)
        B = np.array(g["b"], np.float64)
        assert np.array_equal(oracle.matmul_f64(A, B), np.array(g["c"], np.float64)), g["source"]


def test_matmul_rounds_the_product_before_the_add():
    # a0*b0 = -(1 + 2^-29) exactly; a1*b1 = 1 + 2^-29 + 2^-60 rounds to 1 + 2^-29.
    # mulf then addf gives 0; a fused multiply-add would give 2^-60.
    from oracle import oracle as o
    a = np.array([[-(1 + 2.0**-29), 1 + 2.0**-30]])
    b = np.array([[1.0], [1 + 2.0**-30]])
    assert o.matmul_f64(a, b)[0, 0] == 0.0


def test_matmul_accumulates_k_ascending_from_zero():
    # ((0 + 1e16) + 1) + -1e16 = 0 in k order; any other order can give 1 or 2
    from oracle import oracle as o
    a = np.array([[1e16, 1.0, -1e16, 1.0]])
    b = np.ones((4, 1))
    assert o.matmul_f64(a, b)[0, 0] == 1.0  # (((1e16 + 1) - 1e16) + 1) = 0 + 1
    a = np.array([[1.0, 1e16, -1e16]])
    assert o.matmul_f64(a, np.ones((3, 1)))[0, 0] == 0.0  # (1 + 1e16) - 1e16 = 0


def test_matmul_against_extended_precision(oracle):
    rng = np.random.default_rng(60)
    M, N, K = 17, 23, 301
    A = rng.standard_normal((M, K))
    B = rng.standard_normal((K, N))
    C = oracle.matmul_f64(A, B)
    exact = A.astype(np.longdouble) @ B.astype(np.longdouble)
    bound = K * EPS * (np.abs(A) @ np.abs(B))  # sequential summation bound
    assert np.all(np.abs(C - exact.astype(np.float64)) <= bound)
    # and it is not the exact value every time (it rounds in f64)
    assert np.any(C != exact.astype(np.float64))


def test_matmul_transposed_forms_and_threads_agree_bitwise(oracle):
    rng = np.random.default_rng(61)
    M, N, K = 19, 11, 37
    A = rng.standard_normal((M, K))
    B = rng.standard_normal((K, N))
    C = oracle.matmul_f64(A, B)
    assert np.array_equal(oracle.matmul_f64(A.T.copy(), B, trans_a=True), C)
    assert np.array_equal(oracle.matmul_f64(A, B.T.copy(), trans_b=True), C)
    assert np.array_equal(oracle.matmul_f64(A.T.copy(), B.T.copy(), trans_a=True, trans_b=True), C)
    assert np.array_equal(oracle.matmul_f64(A, B, threads=4), C)
    assert np.array_equal(oracle.matmul_f64_rows(A, B, M, N, K, 5, 9), C[5:9])


def test_matmul_identity_and_zero(oracle):
    rng = np.random.default_rng(62)
    A = rng.standard_normal((9, 9))
    assert np.array_equal(oracle.matmul_f64(A, np.eye(9)), A)
    z = oracle.matmul_f64(A, np.zeros((9, 4)))
    assert np.array_equal(z, np.zeros((9, 4))) and not np.any(np.signbit(z))


def test_elementwise_and_activation_golden(oracle, golden):
    for g in golden["elementwise_add"]:
        assert np.array_equal(oracle.add_f64(g["a"], g["b"]), np.array(g["out"], np.float64))
    a = golden["activations"]
    assert np.array_equal(oracle.relu_f64(a["relu_in"]), np.array(a["relu_out"], np.float64))
    assert np.array_equal(oracle.sigmoid_f64(a["sigmoid_in"]), np.array(a["sigmoid_out"], np.float64))
    assert np.array_equal(oracle.tanh_f64(a["tanh_in"]), np.array(a["tanh_out"], np.float64))


def test_ring_ops_are_ieee_f64(oracle):
    rng = np.random.default_rng(63)
    a = rng.standard_normal(10000) * 1e3
    b = rng.standard_normal(10000) * 1e-3 + 0.5
    assert np.array_equal(oracle.add_f64(a, b), a + b)
    assert np.array_equal(oracle.sub_f64(a, b), a - b)
    assert np.array_equal(oracle.mul_f64(a, b), a * b)
    assert np.array_equal(oracle.div_f64(a, b), a / b)
    n = oracle.neg_f64(np.array([0.0, -0.0, 1.5]))
    assert np.array_equal(np.signbit(n), [True, False, True])
    # the f64 ops differ from f32 ones on inputs f32 cannot hold
    x = np.array([1 + 2.0**-40])
    assert oracle.add_f64(x, x)[0] == 2 + 2.0**-39


def test_relu_is_ieee_maximum(oracle):
    r = oracle.relu_f64(np.array([np.nan, -0.0, 0.0, -3.0, 2.5, -np.inf, np.inf]))
    assert np.isnan(r[0])
    assert r[1] == 0.0 and not np.signbit(r[1]) and not np.signbit(r[2])
    assert list(r[3:]) == [0.0, 2.5, 0.0, np.inf]


def test_sigmoid_and_tanh_against_extended_precision(oracle):
    x = np.concatenate([np.linspace(-40, 40, 20001), [-700.0, -709.0, 36.7, 1e-300, -1e-300]])
    s = oracle.sigmoid_f64(x)
    xl = x.astype(np.longdouble)
    exact = 1 / (1 + np.exp(-xl))
    assert np.all(np.abs(s - exact) <= 4 * EPS * np.abs(exact.astype(np.float64)))
    assert oracle.sigmoid_f64([0.0])[0] == 0.5
    # exp(-x) overflows to inf below -709.78: 1 / (1 + inf) = 0; large x gives exactly 1
    assert list(oracle.sigmoid_f64([-710.0, -800.0, 40.0])) == [0.0, 0.0, 1.0]
    t = oracle.tanh_f64(x[:20001])
    texact = np.tanh(xl[:20001])
    assert np.all(np.abs(t - texact) <= 4 * EPS * np.abs(texact.astype(np.float64)) + 1e-300)
    assert list(oracle.tanh_f64([25.0, -25.0])) == [1.0, -1.0]
    # the f64 functions, not f32 ones rounded back: tanh(0.5) carries f64 digits
    assert oracle.tanh_f64([0.5])[0] == math.tanh(0.5) and oracle.tanh_f64([0.5])[0] != float(np.float32(math.tanh(0.5)))


def test_backward_rules_against_finite_differences(oracle):
    rng = np.random.default_rng(64)
    x = rng.uniform(-3, 3, 200)
    g = rng.uniform(-2, 2, 200)
    h = 1e-6

    def fd(f):
        return (f(x + h) - f(x - h)) / (2 * h)

    s = oracle.sigmoid_f64(x)
    assert np.allclose(oracle.sigmoid_bwd_f64(s, g), g * fd(oracle.sigmoid_f64), rtol=1e-7, atol=1e-9)
    t = oracle.tanh_f64(x)
    assert np.allclose(oracle.tanh_bwd_f64(t, g), g * fd(oracle.tanh_f64), rtol=1e-7, atol=1e-9)
    assert np.array_equal(oracle.relu_bwd_f64(x, g), np.where(x > 0, g, 0.0))
    b = rng.uniform(0.5, 2.0, 200)
    da, db = oracle.div_bwd_f64(x, b, g)
    assert np.allclose(da, g * (1 / b), rtol=1e-12)
    assert np.allclose(db, g * ((x / (b + h) - x / (b - h)) / (2 * h)), rtol=1e-6, atol=1e-9)


def test_bias_and_its_reverse_rule(oracle):
    rng = np.random.default_rng(65)
    a = rng.standard_normal((7, 5))
    bias = rng.standard_normal(5)
    assert np.array_equal(oracle.add_row_bias_f64(a, bias), a + bias[None, :])
    col = np.array([[1e16], [1.0], [-1e16], [1.0]])  # left fold down the column
    assert oracle.sum_rows_f64(col)[0] == 1.0
    s = oracle.sum_rows_f64(a)
    assert np.allclose(s, a.sum(axis=0), rtol=1e-14)


@pytest.mark.parametrize("shape", [(7,), (3, 5), (2, 3, 4)])
def test_index_is_row_major_extract(oracle, shape):
    t = np.arange(int(np.prod(shape)), dtype=np.float64).reshape(shape) * 0.25 - 1
    for idx in np.ndindex(shape):
        assert oracle.index_f64(t, idx) == t[idx]
    with pytest.raises(IndexError):
        oracle.index_f64(t, tuple(d for d in shape))
    dt = np.zeros(shape)
    last = tuple(d - 1 for d in shape)
    oracle.index_bwd_f64(1.5, dt, last)
    oracle.index_bwd_f64(2.0, dt, last)
    want = np.zeros(shape)
    want[last] = 3.5
    assert np.array_equal(dt, want)


def test_reductions_golden_and_fold_order(oracle, golden):
    r = golden["reductions"]
    assert oracle.sum_f64(r["v"]) == r["sum"] and oracle.mean_f64(r["v"]) == r["mean"]
    assert oracle.max_of_f64(r["v"]) == r["max_of"]
    assert oracle.sum_f64([1e16, 1.0, -1e16, 1.0]) == 1.0  # left fold from v[0]
    assert oracle.sum_f64([1.0, 1e16, -1e16]) == 0.0
    assert oracle.mean_f64([1.0, 2.0, 4.0]) == 7.0 / 3.0
    v = np.array([1.0, 5.0, 5.0, -0.0, 0.0, np.nan, 2.0])
    assert oracle.max_of_f64(v) == 5.0 and oracle.argmax_f64(v) == 1  # first of the ties, NaN later ignored
    assert np.isnan(oracle.max_of_f64([np.nan, 3.0])) and oracle.argmax_f64([np.nan, 3.0]) == 0
    z = np.array([-0.0, 0.0])
    assert np.signbit(oracle.max_of_f64(z)) and oracle.argmax_f64(z) == 0
