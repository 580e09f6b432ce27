"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each group uses checks that a plausible mistake would fail: the reference's
own known-answer vectors (tests/golden/reference_vectors.json), closed forms,
independent float64 computations, exact-arithmetic cases, invariants
(conjugate symmetry, transpose consistency) and brute force on tiny inputs.
"""
from __future__ import annotations

import math

import numpy as np
import pytest


# ---- generators ---------------------------------------------------------------

def test_splitmix64_known_answer(oracle):
    # Published first outputs of splitmix64 seeded with 0.
    expect = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    assert [oracle.splitmix64_at(0, i) for i in range(4)] == expect


def test_uniform_is_exact_grid_in_range(oracle):
    u = oracle.uniform(200_000, seed=0)
    assert u.dtype == np.float32
    assert u.min() >= -1.0 and u.max() < 1.0
    # lo + 2*u24*2^-24 -> multiples of 2^-23, exactly
    q = u.astype(np.float64) * 2.0**23
    assert np.array_equal(q, np.round(q))
    assert abs(u.mean()) < 0.01 and abs(u.var() - 1.0 / 3.0) < 0.01
    # the integer stream drives it: the first value follows from the first draw
    x0 = oracle.splitmix64_at(0, 0)
    assert u[0] == np.float32(-1.0 + 2.0 * ((x0 >> 40) * 2.0**-24))


def test_normal_moments_and_shape(oracle):
    from scipy import stats

    z = oracle.normal(200_000, seed=7)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert stats.kstest(z.astype(np.float64), "norm").pvalue > 1e-3
    w = oracle.normal(1000, seed=7, mean=0.0, std=0.02)
    assert np.allclose(w, z[:1000] * np.float32(0.02), rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("bits_in,bits_out", [
    (0x3F800000, 0x3F80),  # 1.0
    (0x3F808000, 0x3F80),  # halfway, even below -> down
    (0x3F818000, 0x3F82),  # halfway, odd below -> up
    (0x3F808001, 0x3F81),  # just above halfway -> up
    (0x3F807FFF, 0x3F80),  # just below halfway -> down
    (0x80000000, 0x8000),  # -0.0
    (0x7F800000, 0x7F80),  # +inf
    (0x7F7FFFFF, 0x7F80),  # max finite rounds to inf
    (0x00000001, 0x0000),  # smallest denormal -> +0
])
def test_bf16_round_nearest_even(oracle, bits_in, bits_out):
    x = np.array([bits_in], np.uint32).view(np.float32)
    assert int(oracle.to_bf16(x)[0]) == bits_out


def test_bf16_nan_stays_nan(oracle):
    x = np.array([0x7FC00001, 0xFF800001], np.uint32).view(np.float32)
    back = oracle.bf16_to_f32(oracle.to_bf16(x))
    assert np.isnan(back).all()


# ---- matmul -------------------------------------------------------------------

def test_matmul_golden_vectors(oracle, golden):
    for case in golden["matmul"]:
        got = oracle.matmul(np.array(case["a"]), np.array(case["b"]))
        assert np.array_equal(got, np.array(case["c"], np.float32)), case["source"]


def test_matmul_matches_float64_within_sequential_bound(oracle):
    rng = np.random.default_rng(1)
    for (M, N, K) in [(1, 1, 1), (3, 5, 7), (16, 9, 33), (8, 8, 257)]:
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = rng.standard_normal((K, N)).astype(np.float32)
        exact = A.astype(np.float64) @ B.astype(np.float64)
        bound = np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64)
        got = oracle.matmul(A, B).astype(np.float64)
        # sequential f32 summation error is at most about K * eps * sum|a||b|
        assert np.all(np.abs(got - exact) <= (K + 1) * 2.0**-24 * bound + 1e-30)


def test_matmul_transposed_forms_agree_bitwise(oracle):
    rng = np.random.default_rng(2)
    M, N, K = 7, 11, 13
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    ref = oracle.matmul(A, B)
    assert np.array_equal(oracle.matmul(np.ascontiguousarray(A.T), B, trans_a=True), ref)
    assert np.array_equal(oracle.matmul(A, np.ascontiguousarray(B.T), trans_b=True), ref)
    assert np.array_equal(oracle.matmul(np.ascontiguousarray(A.T), np.ascontiguousarray(B.T),
                                        trans_a=True, trans_b=True), ref)


def test_matmul_threaded_rows_and_entries_are_bitwise_the_same(oracle):
    rng = np.random.default_rng(3)
    M, N, K = 37, 29, 101
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    ref = oracle.matmul(A, B)
    assert np.array_equal(oracle.matmul(A, B, threads=4), ref)
    assert np.array_equal(oracle.matmul_rows(A, B, M, N, K, 5, 9), ref[5:9])
    ii = rng.integers(0, M, 50)
    jj = rng.integers(0, N, 50)
    vals, absv = oracle.matmul_entries(A, B, M, N, K, ii, jj)
    assert np.array_equal(vals, ref[ii, jj])
    assert np.allclose(absv, (np.abs(A) @ np.abs(B))[ii, jj], rtol=1e-5)


def test_matmul_identity_and_zero(oracle):
    rng = np.random.default_rng(4)
    A = rng.standard_normal((6, 6)).astype(np.float32)
    assert np.array_equal(oracle.matmul(A, np.eye(6, dtype=np.float32)), A)
    assert np.array_equal(oracle.matmul(A, np.zeros((6, 6), np.float32)), np.zeros((6, 6), np.float32))


def test_bf16_matmul_entries_use_upcast_values(oracle):
    rng = np.random.default_rng(5)
    M, N, K = 9, 10, 40
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    Ab, Bb = oracle.to_bf16(A), oracle.to_bf16(B)
    ref = oracle.matmul(oracle.bf16_to_f32(Ab).reshape(M, K), oracle.bf16_to_f32(Bb).reshape(K, N))
    ii, jj = np.repeat(np.arange(M), N), np.tile(np.arange(N), M)
    vals, _ = oracle.matmul_entries(Ab, Bb, M, N, K, ii, jj, bf16=True)
    assert np.array_equal(vals.reshape(M, N), ref)


def test_bf16_matmul_rows_equal_the_entries_form_bitwise(oracle):
    # or_matmul_bf16_rows (the bf16 CPU baseline's loop) computes what the
    # entries form computes, bit for bit, on every entry of a band of rows;
    # a swapped index or a dropped term would change values.
    rng = np.random.default_rng(6)
    M, N, K = 13, 21, 67
    Ab = oracle.to_bf16(rng.standard_normal((M, K)).astype(np.float32))
    Bb = oracle.to_bf16(rng.standard_normal((K, N)).astype(np.float32))
    rows = oracle.matmul_bf16_rows(Ab, Bb, M, N, K, 3, 11)
    ii, jj = np.repeat(np.arange(3, 11), N), np.tile(np.arange(N), 8)
    vals, _ = oracle.matmul_entries(Ab, Bb, M, N, K, ii, jj, bf16=True)
    assert np.array_equal(rows.ravel(), vals)
    # and both equal the f32 loop on the upcast values
    ref = oracle.matmul(oracle.bf16_to_f32(Ab).reshape(M, K), oracle.bf16_to_f32(Bb).reshape(K, N))
    assert np.array_equal(rows, ref[3:11])


# ---- elementwise --------------------------------------------------------------

def test_elementwise_golden(oracle, golden):
    for case in golden["elementwise_add"]:
        assert np.array_equal(oracle.add(case["a"], case["b"]), np.array(case["out"], np.float32))
    act = golden["activations"]
    assert np.array_equal(oracle.relu(act["relu_in"]), np.array(act["relu_out"], np.float32))
    assert np.array_equal(oracle.sigmoid(act["sigmoid_in"]), np.array(act["sigmoid_out"], np.float32))
    assert np.array_equal(oracle.tanh(act["tanh_in"]), np.array(act["tanh_out"], np.float32))


def test_ring_ops_are_ieee_f32(oracle):
    rng = np.random.default_rng(6)
    a = rng.standard_normal(4096).astype(np.float32)
    b = rng.standard_normal(4096).astype(np.float32)
    # numpy float32 ufuncs round each element once: an independent IEEE computation
    assert np.array_equal(oracle.add(a, b), a + b)
    assert np.array_equal(oracle.sub(a, b), a - b)
    assert np.array_equal(oracle.mul(a, b), a * b)
    assert np.array_equal(oracle.div(a, b), a / b)
    assert np.array_equal(oracle.neg(a).view(np.uint32), (-a).view(np.uint32))


def test_relu_is_ieee_maximum(oracle):
    x = np.array([-0.0, 0.0, -2.0, 3.0, -np.inf, np.inf, np.nan], np.float32)
    r = oracle.relu(x)
    assert r[0] == 0.0 and not np.signbit(r[0])  # max(-0, +0) = +0
    assert r[1] == 0.0 and not np.signbit(r[1])
    assert list(r[2:6]) == [0.0, 3.0, 0.0, np.inf]
    assert np.isnan(r[6])  # NaN propagates (maximumf, not maxnum)


def test_sigmoid_tanh_against_float64(oracle):
    x = np.linspace(-30, 30, 20001).astype(np.float32)
    s64 = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(oracle.sigmoid(x) - s64) / s64) < 1e-6
    t64 = np.tanh(x.astype(np.float64))
    nz = np.abs(t64) > 1e-30
    assert np.max(np.abs(oracle.tanh(x)[nz] - t64[nz]) / np.abs(t64[nz])) < 1e-6


def test_backward_rules_against_finite_differences(oracle):
    x = np.linspace(-4, 4, 81).astype(np.float32)
    g = np.linspace(0.5, 1.5, 81).astype(np.float32)
    h = 1e-4
    xd = x.astype(np.float64)
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    fd = (sig(xd + h) - sig(xd - h)) / (2 * h)
    assert np.allclose(oracle.sigmoid_bwd(oracle.sigmoid(x), g), g * fd, rtol=1e-4, atol=1e-6)
    fd = (np.tanh(xd + h) - np.tanh(xd - h)) / (2 * h)
    assert np.allclose(oracle.tanh_bwd(oracle.tanh(x), g), g * fd, rtol=1e-4, atol=1e-6)
    assert np.array_equal(oracle.relu_bwd(x, g), np.where(x > 0, g, 0).astype(np.float32))
    a = np.linspace(-2, 2, 9).astype(np.float32)
    b = np.linspace(0.5, 3, 9).astype(np.float32)
    gg = np.ones(9, np.float32)
    da, db = oracle.div_bwd(a, b, gg)
    assert np.allclose(da, 1.0 / b.astype(np.float64), rtol=1e-6)
    assert np.allclose(db, -a.astype(np.float64) / b.astype(np.float64) ** 2, rtol=1e-6)


def test_reference_derivative_known_answers(oracle, golden):
    d = {case["source"].split(":")[1]: case for case in golden["derivatives"]}
    one = np.ones(1, np.float32)
    # d(x*x)/dx at 3 via the mul rule de*e + e*de
    x = np.float32(3.0)
    assert float(x + x) == golden["derivatives"][0]["grad"][0]
    # d(x*y + x) at (3,5): (y + 1, x)
    assert [5.0 + 1.0, 3.0] == golden["derivatives"][1]["grad"]
    # tanh' = 1 - t*t, bitwise the reference test's own expression
    t = oracle.tanh(np.array([0.5], np.float32))
    assert oracle.tanh_bwd(t, one)[0] == np.float32(1.0) - t[0] * t[0]
    # (1/w)' at 2 through the quotient rule
    _, db = oracle.div_bwd(one, np.array([2.0], np.float32), one)
    assert db[0] == golden["derivatives"][4]["grad"][0]
    # (sigmoid(w)^2)' = 2 s s (1 - s): chain rule through the mul rule
    s = oracle.sigmoid(np.array([0.5], np.float32))
    got = oracle.sigmoid_bwd(s, s + s)[0]
    want = np.float32(2.0) * s[0] * s[0] * (np.float32(1.0) - s[0])
    assert abs(got - want) < 1e-7
    # sigmoid(w1)*sigmoid(w2) at (0.5, 1.5), reference tolerance 1e-4
    s1 = oracle.sigmoid(np.array([0.5], np.float32))
    s2 = oracle.sigmoid(np.array([1.5], np.float32))
    g1 = oracle.sigmoid_bwd(s1, s2)[0]
    g2 = oracle.sigmoid_bwd(s2, s1)[0]
    assert abs(g1 - s1[0] * (1 - s1[0]) * s2[0]) < 1e-4
    assert abs(g2 - s1[0] * s2[0] * (1 - s2[0])) < 1e-4
    # grad of trace(A I) w.r.t. A: dA = dC B^T with dC = I, B = I
    I2 = np.eye(2, dtype=np.float32)
    dA = oracle.matmul(I2, I2, trans_b=True)
    assert list(dA.ravel()) == golden["derivatives"][7]["grad"]
    # sum_i w * data[i]: the mul rule gives data[i] per term, the sum adds them
    loop = d["2540-2558"]
    terms = oracle.mul(np.ones(3, np.float32), np.array(loop["data"], np.float32))
    assert oracle.sum_f32(terms) == loop["grad"][0]
    # w[0] + w[1]*w[1] with w built from (w1, w2): Index's rule scatters each
    # read's cotangent back; the product rule gives w[1] + w[1] for the square
    built = d["2738-2757"]
    w = np.array(built["at"], np.float32)
    dw = np.zeros(2, np.float32)
    oracle.index_bwd(1.0, dw, (0,))
    w1 = oracle.index(w, (1,))
    oracle.index_bwd(float(np.float32(w1) + np.float32(w1)), dw, (1,))
    assert list(dw) == built["grad"]
    assert len(d) == len(golden["derivatives"])  # every source is distinct


# ---- row-broadcast bias ---------------------------------------------------------

def test_add_row_bias_is_broadcast_add(oracle):
    rng = np.random.default_rng(31)
    a = rng.standard_normal((37, 19)).astype(np.float32)
    b = rng.standard_normal(19).astype(np.float32)
    assert np.array_equal(oracle.add_row_bias(a, b), a + b[None, :])
    # one row is the reference's own same-shape bias add (xor_tensor, batch of 1)
    assert np.array_equal(oracle.add_row_bias(a[:1], b)[0], oracle.add(a[0], b))


def test_sum_rows_is_a_left_fold_down_each_column(oracle):
    rng = np.random.default_rng(32)
    ints = rng.integers(-1000, 1000, (300, 7)).astype(np.float32)
    assert np.array_equal(oracle.sum_rows(ints), ints.sum(axis=0, dtype=np.float64).astype(np.float32))
    # the fold order decides what cancels: ((1e8 + 1) - 1e8) = 0 in f32, 1 in exact arithmetic
    g = np.array([[1e8, 1.0], [1.0, 1e8], [-1e8, -1e8]], np.float32)
    assert list(oracle.sum_rows(g)) == [0.0, 0.0]
    g2 = np.array([[1.0, 1.0], [1e8, 1e8], [-1e8, -1e8]], np.float32)
    assert list(oracle.sum_rows(g2)) == [0.0, 0.0]
    h = np.array([[1e8, 1e8], [-1e8, -1e8], [1.0, 1.0]], np.float32)
    assert list(oracle.sum_rows(h)) == [1.0, 1.0]
    x = rng.standard_normal((500, 9)).astype(np.float32)
    exact = x.astype(np.float64).sum(axis=0)
    assert np.all(np.abs(oracle.sum_rows(x) - exact) <= 500 * 2**-24 * np.abs(x).astype(np.float64).sum(axis=0))


# ---- Index ----------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(7,), (3, 5), (2, 3, 4), (2, 1, 3, 5)])
def test_index_is_row_major_extract(oracle, shape):
    # tensor.extract over the row-major buffer: numpy's C-order indexing is the
    # same closed form, offset = sum_d idx[d] * prod_{e>d} shape[e]
    rng = np.random.default_rng(len(shape))
    T = rng.standard_normal(shape).astype(np.float32)
    for flat in range(T.size):
        idx = np.unravel_index(flat, shape)
        assert oracle.index(T, idx) == T[idx] == T.ravel()[flat]
    for bad in [tuple(s for s in shape), tuple([-1] + [0] * (len(shape) - 1))]:
        with pytest.raises(IndexError):
            oracle.index(T, bad)


def test_index_bwd_scatters_and_accumulates(oracle):
    dt = np.zeros((3, 4), np.float32)
    oracle.index_bwd(2.5, dt, (1, 2))
    oracle.index_bwd(0.5, dt, (1, 2))
    oracle.index_bwd(-1.0, dt, (2, 3))
    want = np.zeros((3, 4), np.float32)
    want[1, 2], want[2, 3] = 3.0, -1.0
    assert np.array_equal(dt, want)
    with pytest.raises(IndexError):
        oracle.index_bwd(1.0, dt, (3, 0))
    assert np.array_equal(dt, want)  # a rejected call leaves dt alone


# ---- reductions -----------------------------------------------------------------

def test_reduction_golden(oracle, golden):
    r = golden["reductions"]
    assert oracle.sum_f32(r["v"]) == r["sum"]
    assert oracle.mean_f32(r["v"]) == r["mean"]
    assert oracle.max_of(r["v"]) == r["max_of"]


def test_sum_is_left_fold(oracle):
    # 1e8 + 1 + 1 ... in f32: a left fold drops every +1 (1e8 ulp is 8)
    v = np.array([1e8] + [1.0] * 16, np.float32)
    assert oracle.sum_f32(v) == np.float32(1e8)
    # the reversed order accumulates the ones first (16), then adds 1e8 -> 100000016
    assert oracle.sum_f32(v[::-1].copy()) == np.float32(1e8 + 16)
    ints = np.arange(1, 1001, dtype=np.float32)
    assert oracle.sum_f32(ints) == 500500.0
    assert oracle.mean_f32(ints) == np.float32(500500.0) / np.float32(1000)


def test_max_semantics(oracle):
    assert np.isnan(oracle.max_of(np.array([np.nan, 1.0, 2.0], np.float32)))  # NaN at v[0] sticks
    assert oracle.max_of(np.array([1.0, np.nan, 2.0], np.float32)) == 2.0     # later NaN ignored
    z = oracle.max_of(np.array([-0.0, 0.0], np.float32))
    assert z == 0.0 and np.signbit(z)  # +0 > -0 is false: the first zero is kept
    assert oracle.argmax(np.array([3.0, 7.0, 7.0, 1.0], np.float32)) == 1
    assert oracle.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert oracle.sum_u64(np.array([0xFFFFFFFF] * 5, np.uint32)) == 5 * 0xFFFFFFFF


# ---- escape counts ---------------------------------------------------------------

def test_escape_count_special_points(oracle, golden):
    mb = golden["mandelbrot_example"]
    for cr, ci in mb["never_escapes"]:
        assert oracle.escape_count(cr, ci, 1000) == 1000
    for cr, ci in mb["escapes_at_0"]:
        assert oracle.escape_count(cr, ci, 1000) == 0
    assert oracle.escape_count(0.5, 0.5, 1000) == 4  # 0.5+0.5i escapes at the 5th step
    assert oracle.escape_count(1.0, 0.0, 100) == 2   # z = 1, 2, 5: |2|^2 = 4 is not > 4; 25 is


def test_escape_count_latch_form_is_equivalent(oracle):
    w, h = 96, 64
    x0, y0, dx, dy = -2.0, -1.5, 3.0 / w, 3.0 / h
    fast = oracle.mandelbrot(w, h, x0, y0, dx, dy, 200)
    latch = np.array([[oracle.escape_count(np.float32(x0 + np.float32(c) * np.float32(dx)),
                                           np.float32(y0 + np.float32(r) * np.float32(dy)), 200, latch=True)
                       for c in range(w)] for r in range(h)], np.uint32)
    assert np.array_equal(fast, latch)


def test_escape_count_conjugate_symmetry_and_float64_agreement(oracle):
    # negating ci is exact, and every later step mirrors, so counts are symmetric
    w, h = 128, 128
    dy = 3.0 / 128
    top = oracle.mandelbrot(w, h, -2.0, -1.5, 3.0 / w, dy, 300)
    # rows r and 128 - r have ci = -1.5 + r*dy and +1.5 - r*dy... mirror of row r is row 128-r
    assert np.array_equal(top[1:64], top[127:64:-1])
    # far from the boundary f32 and f64 agree: compare with a float64 escape loop
    pts = [(-0.1, 0.1), (0.3, 0.0), (-1.9, 0.0), (0.4, 0.4), (-0.75, 0.3)]
    for cr, ci in pts:
        z = 0j
        c = complex(cr, ci)
        n64 = 300
        for n in range(300):
            z = z * z + c
            if abs(z) ** 2 > 4:
                n64 = n
                break
        assert oracle.escape_count(cr, ci, 300) == n64


def test_mandelbrot_threaded_row_band_is_the_rows_form(oracle):
    w, h = 200, 120
    args = (w, h, -2.0, -1.5, 3.0 / w, 3.0 / h, 300)
    band = oracle.mandelbrot(*args, threads=4, rows=(17, 90))
    seq = oracle.mandelbrot(*args, rows=(17, 90))
    assert np.array_equal(band, seq)
    assert np.array_equal(band[17:90], oracle.mandelbrot(*args)[17:90])
    assert not band[:17].any() and not band[90:].any()


# ---- MLP + autograd ----------------------------------------------------------------

def test_mlp_gradients_against_finite_differences(oracle):
    rng = np.random.default_rng(8)
    B, D, Hd = 8, 5, 6
    X = rng.standard_normal((B, D)).astype(np.float32)
    y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = rng.uniform(-0.8, 0.8, (D, Hd)).astype(np.float32)
    W2 = rng.uniform(-0.8, 0.8, Hd).astype(np.float32)
    loss, dW1, dW2, _, _ = oracle.mlp_step(X, y, W1, W2, lr=0.0)
    assert abs(loss - oracle.mlp_loss_f64(X, y, W1, W2)) < 1e-6
    h = 1e-3
    for (k, n) in [(0, 0), (2, 3), (4, 5), (1, 1)]:
        Wp, Wm = W1.copy(), W1.copy()
        Wp[k, n] += h
        Wm[k, n] -= h
        fd = (oracle.mlp_loss_f64(X, y, Wp, W2) - oracle.mlp_loss_f64(X, y, Wm, W2)) / (
            float(Wp[k, n]) - float(Wm[k, n]))
        assert abs(dW1[k, n] - fd) < 1e-4 * max(1.0, abs(fd)), (k, n)
    for n in range(Hd):
        Wp, Wm = W2.copy(), W2.copy()
        Wp[n] += h
        Wm[n] -= h
        fd = (oracle.mlp_loss_f64(X, y, W1, Wp) - oracle.mlp_loss_f64(X, y, W1, Wm)) / (
            float(Wp[n]) - float(Wm[n]))
        assert abs(dW2[n] - fd) < 1e-4 * max(1.0, abs(fd)), n


def test_mlp_sgd_update_is_w_minus_lr_g(oracle):
    rng = np.random.default_rng(9)
    B, D, Hd = 16, 4, 8
    X = rng.standard_normal((B, D)).astype(np.float32)
    y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = rng.uniform(-0.5, 0.5, (D, Hd)).astype(np.float32)
    W2 = rng.uniform(-0.5, 0.5, Hd).astype(np.float32)
    lr = np.float32(0.01)
    _, dW1, dW2, W1n, W2n = oracle.mlp_step(X, y, W1, W2, lr=float(lr))
    assert np.array_equal(W1n, W1 - lr * dW1)
    assert np.array_equal(W2n, W2 - lr * dW2)
    _, dW1t, _, _, _ = oracle.mlp_step(X, y, W1, W2, lr=0.0, threads=4)
    assert np.array_equal(dW1t, dW1)  # threading does not change any bit


@pytest.mark.parametrize("B,D,Hd", [(64, 32, 48), (130, 20, 36), (256, 64, 128)])
def test_mlp_grad_entries_equal_the_full_step_bitwise(oracle, B, D, Hd):
    # The sampled-gradient oracle used at full size computes each entry exactly
    # as the whole step does: every entry of dW1 and dW2, and the loss.
    rng = np.random.default_rng(B + D + Hd)
    X = rng.standard_normal((B, D)).astype(np.float32)
    y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = rng.uniform(-0.3, 0.3, (D, Hd)).astype(np.float32)
    W2 = rng.uniform(-0.3, 0.3, Hd).astype(np.float32)
    L, dW1, dW2, _, _ = oracle.mlp_step(X, y, W1, W2, lr=0.01)
    kk, nn = np.meshgrid(np.arange(D), np.arange(Hd), indexing="ij")
    L2, g1, a1, g2, a2 = oracle.mlp_grad_entries(X, y, W1, W2, kk.ravel(), nn.ravel(), np.arange(Hd), threads=4)
    assert L2 == L
    assert np.array_equal(g1, dW1.ravel()) and np.array_equal(g2, dW2)
    assert np.all(a1 >= np.abs(g1)) and np.all(a2 >= np.abs(g2))


def test_xor_tensor_training_matches_reference_record(oracle, golden):
    g = golden["xor_tensor"]
    preds = oracle.xor_tensor_train(g["steps"], g["lr"])
    # The record is the reference's printed f32 output; its gradient expressions
    # come from e-graph extraction and its libm is MSVC's, so bits may differ.
    assert np.allclose(preds, g["predictions"], atol=1e-6, rtol=0)


# ---- broadcasting maps and their reverse rule (extension) ---------------------------

_BCAST_PAIRS = [
    ((3, 4), (4,)), ((3, 4), (3, 1)), ((3, 1), (1, 4)), ((2, 3, 4), (3, 1)), ((2, 1, 4), (1, 3, 1)),
    ((5,), ()), ((), (2, 3)), ((1,), (7,)), ((2, 3, 4, 5), (1, 3, 1, 5)), ((4, 1, 1), (4, 6, 2)),
    ((2, 0, 3), (3,)), ((6, 5), (6, 5)),
]


@pytest.mark.parametrize("ashape,bshape", _BCAST_PAIRS)
@pytest.mark.parametrize("f64", [False, True])
def test_bcast_is_numpy_broadcast_arithmetic(oracle, ashape, bshape, f64):
    # numpy applies the same rule and one IEEE operation per element in the
    # operands' dtype, so the restated loop must agree bit for bit
    rng = np.random.default_rng(len(ashape) * 31 + len(bshape))
    dt = np.float64 if f64 else np.float32
    a = rng.standard_normal(ashape).astype(dt)
    b = (rng.standard_normal(bshape) + 3.0).astype(dt)
    for op, f in (("add", np.add), ("sub", np.subtract), ("mul", np.multiply), ("div", np.divide)):
        got = oracle.bcast(op, a, b, f64=f64)
        want = f(a, b)
        assert got.shape == want.shape
        assert np.array_equal(got.view(np.uint64 if f64 else np.uint32), want.view(np.uint64 if f64 else np.uint32))


def test_bcast_equal_shapes_is_the_same_shape_map(oracle):
    rng = np.random.default_rng(5)
    a, b = rng.standard_normal((7, 9)).astype(np.float32), rng.standard_normal((7, 9)).astype(np.float32)
    assert np.array_equal(oracle.bcast("add", a, b).ravel(), oracle.add(a.ravel(), b.ravel()))
    assert np.array_equal(oracle.bcast("div", a, b).ravel(), oracle.div(a.ravel(), b.ravel()))


@pytest.mark.parametrize("ashape,bshape", [((3, 4), (3,)), ((2, 3), (3, 2)), ((4, 1, 5), (2, 5, 1, 1, 3))])
def test_bcast_rejects_shapes_that_do_not_broadcast(oracle, ashape, bshape):
    with pytest.raises(ValueError):
        oracle.bcast("add", np.zeros(ashape), np.zeros(bshape))


_SUM_CASES = [((6, 5), (5,)), ((6, 5), (6, 1)), ((6, 5), (1, 1)), ((6, 5), ()), ((2, 3, 4), (3, 1)),
              ((2, 3, 4), (1, 3, 4)), ((2, 3, 4), (2, 1, 4)), ((3, 1, 4), (1, 1, 4)), ((4, 5), (4, 5))]


@pytest.mark.parametrize("gshape,oshape", _SUM_CASES)
def test_sum_to_shape_against_numpy(oracle, gshape, oshape):
    rng = np.random.default_rng(len(gshape) + 7 * len(oshape))
    g = rng.standard_normal(gshape).astype(np.float32)
    got = oracle.sum_to_shape(g, oshape)
    R = len(gshape)
    full = (1,) * (R - len(oshape)) + tuple(oshape)
    axes = tuple(i for i in range(R) if full[i] == 1 and gshape[i] != 1)
    want = g.astype(np.float64).sum(axis=axes, keepdims=True).reshape(oshape)
    den = np.abs(g.astype(np.float64)).sum(axis=axes, keepdims=True).reshape(oshape)
    n = max(1, int(np.prod([gshape[i] for i in axes])))
    assert got.shape == tuple(oshape)
    assert np.all(np.abs(got - want) <= 1e-6 * n * den + 1e-30)
    # integer values: every partial sum is exact, so any order gives the sum
    gi = rng.integers(-50, 50, gshape).astype(np.float32)
    assert np.array_equal(oracle.sum_to_shape(gi, oshape),
                          gi.astype(np.float64).sum(axis=axes, keepdims=True).reshape(oshape).astype(np.float32))
    # f64 form
    got64 = oracle.sum_to_shape(g.astype(np.float64), oshape, f64=True)
    assert np.all(np.abs(got64 - want) <= 1e-14 * n * den + 1e-300)


@pytest.mark.parametrize("gshape,oshape,axes", [((0, 5), (1, 5), (0,)), ((3, 0, 4), (3, 1, 4), (1,)), ((0,), (), (0,))])
def test_sum_to_shape_over_an_empty_dimension_is_zero(oracle, gshape, oshape, axes):
    # numpy's sum over nothing: zeros of the kept shape
    g = np.zeros(gshape, np.float32)
    want = g.sum(axis=axes, keepdims=len(oshape) == len(gshape)).reshape(oshape)
    assert np.array_equal(want, np.zeros(oshape, np.float32))
    assert np.array_equal(oracle.sum_to_shape(g, oshape), want)
    assert np.array_equal(oracle.sum_to_shape(g.astype(np.float64), oshape, f64=True), want)


def test_sum_to_shape_leading_rows_is_the_column_sum(oracle):
    # [rows, cols] -> [cols] is the row bias's reverse rule: the same left fold
    # down each column (0 + g[0][j] = g[0][j] for nonzero data)
    g = np.random.default_rng(3).standard_normal((37, 11)).astype(np.float32)
    assert np.array_equal(oracle.sum_to_shape(g, (11,)), oracle.sum_rows(g))


def test_sum_to_shape_adds_in_row_major_order(oracle):
    # 1e8 + 1 rounds back to 1e8 in f32, so the row-major order over the
    # stretched dimension gives 0 where the exact sum is 1; a different order
    # (1 last, or pairwise) would not
    g = np.array([[1e8], [1.0], [-1e8]], np.float32)
    assert oracle.sum_to_shape(g, (1,))[0] == 0.0
    g2 = np.array([[[1e8, 2.0], [1.0, 0.0]], [[-1e8, 0.0], [0.0, 0.0]]], np.float32)  # (2, 2, 2) -> (1, 2)
    got = oracle.sum_to_shape(g2, (1, 2))
    assert got[0, 0] == 0.0 and got[0, 1] == 2.0
    with pytest.raises(ValueError):
        oracle.sum_to_shape(np.zeros((3, 4), np.float32), (2, 4))
