"""Tensor<f64, ...> on the GPU, through the C ABI, against the f64 oracle.

Tolerances (f64 counterparts of the f32 bar, scaled by the unit roundoff):
  GEMM  |C - C_ref| <= 2e-14 * sqrt(K) * sum_k |A_ik||B_kj|   per entry
  sums  |s - s_ref| <= 2e-14 * sqrt(n) * sum_i |x_i|
  exp / tanh maps: rel <= 1e-14 (device and host libm differ in the last bits)
  IEEE maps (add, sub, mul, div, neg, relu, the backward rules, the bias add,
  the SGD update), max_of, argmax, Index: bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import gemm_normalised_error, rel_close

pytestmark = pytest.mark.gpu

GEMM_TOL = 2e-14
SUM_TOL = 2e-14


def _assert_gemm64(got, ref, den, K, what):
    err = gemm_normalised_error(got, ref, den)
    tol = GEMM_TOL * np.sqrt(max(K, 1))
    assert err <= tol, f"{what}: normalised error {err:.3e} > {tol:.3e}"
    return err


def _check(hip, oracle, A, B, ta, tb, what):
    c = hip.matmul(hip.from_numpy(A), hip.from_numpy(B), trans_a=bool(ta), trans_b=bool(tb))
    assert c.dtype == "f64"
    Ak = np.ascontiguousarray(A.T) if ta else A  # M x K
    Bk = B if tb else np.ascontiguousarray(B.T)  # N x K
    ref = oracle.matmul_f64(Ak, Bk, trans_b=True, threads=16)
    den = np.abs(Ak) @ np.abs(Bk).T
    return _assert_gemm64(c.numpy(), ref, den, Ak.shape[1], what)


def test_golden_vectors_exact(hip, golden):
    for case in golden["matmul"]:
        A = np.array(case["a"], np.float64)
        B = np.array(case["b"], np.float64)
        got = hip.matmul(hip.from_numpy(A), hip.from_numpy(B)).numpy()
        assert np.array_equal(got, np.array(case["c"], np.float64)), case["source"]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (2, 3, 2), (127, 129, 33), (300, 200, 17), (128, 128, 16),
                                   (256, 384, 48), (130, 257, 1000), (513, 64, 7), (64, 1, 300)])
def test_shapes_and_layouts(hip, oracle, M, N, K, ta, tb):
    rng = np.random.default_rng(M * 7 + N * 3 + K + 11 * ta + tb)
    A = rng.standard_normal((K, M) if ta else (M, K))
    B = rng.standard_normal((N, K) if tb else (K, N))
    _check(hip, oracle, A, B, ta, tb, f"f64 {M}x{N}x{K} ta={ta} tb={tb}")


def test_k_zero_gives_zeros_and_overwrites_c(hip):
    # matrix.cleave:59 zero-fills the accumulator: K = 0 is an all-zero C
    a = hip.empty((5, 0), "f64")
    b = hip.empty((0, 7), "f64")
    c = hip.from_numpy(np.full((5, 7), np.nan))
    hip.matmul(a, b, out=c)
    assert np.array_equal(c.numpy(), np.zeros((5, 7)))


def test_matmul_against_zero_is_exactly_zero(hip):
    rng = np.random.default_rng(1)
    A = rng.standard_normal((200, 200))
    c = hip.from_numpy(np.full((200, 200), np.nan))
    hip.matmul(hip.from_numpy(A), hip.from_numpy(np.zeros((200, 200))), out=c)
    assert np.array_equal(c.numpy(), np.zeros((200, 200)))


def test_misaligned_operands_take_the_single_double_loads(hip, oracle):
    # a view one double into its buffer is 8-byte aligned only
    rng = np.random.default_rng(2)
    M, N, K = 130, 66, 34
    A = rng.standard_normal(M * K + 1)
    B = rng.standard_normal(K * N + 1)
    a = hip.from_numpy(A).sub(1, (M, K))
    b = hip.from_numpy(B).sub(1, (K, N))
    got = hip.matmul(a, b).numpy()
    Am, Bm = A[1:].reshape(M, K), B[1:].reshape(K, N)
    ref = oracle.matmul_f64(Am, Bm, threads=16)
    _assert_gemm64(got, ref, np.abs(Am) @ np.abs(Bm), K, "misaligned f64")


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_config2_shape_in_f64_every_entry(hip, oracle, ta, tb):
    # BASELINE config 2's 4096^3 product on Tensor<f64>: every entry
    n = 4096
    rng = np.random.default_rng(40 + ta)
    A = rng.standard_normal((n, n))
    B = rng.standard_normal((n, n))
    _check(hip, oracle, A, B, ta, tb, f"f64 4096^3 ta={ta} tb={tb}")


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
def test_batched(hip, oracle, ta, tb):
    rng = np.random.default_rng(50 + 2 * ta + tb)
    bsz, M, N, K = 6, 96, 130, 40
    A = rng.standard_normal((bsz, K, M) if ta else (bsz, M, K))
    B = rng.standard_normal((bsz, N, K) if tb else (bsz, K, N))
    c = hip.matmul_batched(hip.from_numpy(A), hip.from_numpy(B), trans_a=bool(ta), trans_b=bool(tb)).numpy()
    for i in range(bsz):
        Ak = np.ascontiguousarray(A[i].T) if ta else A[i]
        Bk = B[i] if tb else np.ascontiguousarray(B[i].T)
        ref = oracle.matmul_f64(Ak, Bk, trans_b=True)
        _assert_gemm64(c[i], ref, np.abs(Ak) @ np.abs(Bk).T, K, f"batched f64 #{i}")


def _special():
    return np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-310, -1e-310, 709.0, -709.0, 710.0, -710.0, 745.0,
                     -745.0, 20.0, -20.0, 1e-8, -1e-8])


def test_ieee_maps_bit_exact(hip, oracle):
    rng = np.random.default_rng(60)
    n = 100003
    a = np.concatenate([rng.standard_normal(n - 17) * 10, _special()])
    b = np.concatenate([rng.standard_normal(n - 17) + 0.25, _special()[::-1]])
    da, db = hip.from_numpy(a), hip.from_numpy(b)
    for name in ("add", "sub", "mul", "div"):
        got = getattr(hip, name)(da, db).numpy()
        ref = getattr(oracle, f"{name}_f64")(a, b)
        assert np.array_equal(got, ref, equal_nan=True), name
    for name in ("neg", "relu"):
        got = getattr(hip, name)(da).numpy()
        assert np.array_equal(got, getattr(oracle, f"{name}_f64")(a), equal_nan=True), name
        assert np.array_equal(np.signbit(got), np.signbit(getattr(oracle, f"{name}_f64")(a))), name
    s = oracle.sigmoid_f64(a)
    t = oracle.tanh_f64(a)
    for name, x in (("sigmoid_bwd", s), ("tanh_bwd", t), ("relu_bwd", a)):
        got = getattr(hip, name)(hip.from_numpy(x), db).numpy()
        assert np.array_equal(got, getattr(oracle, f"{name}_f64")(x, b), equal_nan=True), name
    gda, gdb = hip.div_bwd(da, db, hip.from_numpy(s))
    rda, rdb = oracle.div_bwd_f64(a, b, s)
    assert np.array_equal(gda.numpy(), rda, equal_nan=True) and np.array_equal(gdb.numpy(), rdb, equal_nan=True)
    z = hip.from_numpy(np.full(1001, 3.0))
    hip.zero(z)
    assert np.array_equal(z.numpy(), np.zeros(1001))


def test_exp_and_tanh_maps(hip, oracle):
    rng = np.random.default_rng(61)
    x = np.concatenate([rng.uniform(-40, 40, 200000), np.linspace(-1e-3, 1e-3, 2001), _special()])
    d = hip.from_numpy(x)
    assert rel_close(hip.sigmoid(d).numpy(), oracle.sigmoid_f64(x), rtol=1e-14)
    assert rel_close(hip.tanh(d).numpy(), oracle.tanh_f64(x), rtol=1e-14)
    assert hip.sigmoid(hip.from_numpy(np.zeros(3))).numpy().tolist() == [0.5, 0.5, 0.5]


def test_sgd_bias_and_column_sums(hip, oracle):
    rng = np.random.default_rng(62)
    w = rng.standard_normal(4099)
    g = rng.standard_normal(4099)
    dw = hip.from_numpy(w)
    hip.sgd_update(dw, hip.from_numpy(g), 0.01)
    assert np.array_equal(dw.numpy(), w - 0.01 * g)
    for rows, cols in ((37, 64), (1000, 130), (3, 5), (4096, 1024)):
        m = rng.standard_normal((rows, cols))
        bias = rng.standard_normal(cols)
        got = hip.add_row_bias(hip.from_numpy(m), hip.from_numpy(bias)).numpy()
        assert np.array_equal(got, oracle.add_row_bias_f64(m, bias))
        s = hip.sum_rows(hip.from_numpy(m)).numpy()
        ref = oracle.sum_rows_f64(m)
        assert np.all(np.abs(s - ref) <= SUM_TOL * np.sqrt(rows) * np.abs(m).sum(axis=0)), (rows, cols)


@pytest.mark.parametrize("n", [1, 2, 3, 7, 1024, 100003, (1 << 24) + 3])
def test_reductions(hip, oracle, n):
    rng = np.random.default_rng(63 + n % 97)
    v = rng.standard_normal(n) * 3 + 0.5
    d = hip.from_numpy(v)
    scale = SUM_TOL * np.sqrt(n) * np.abs(v).sum()
    assert abs(hip.sum(d) - oracle.sum_f64(v)) <= scale
    assert abs(hip.mean(d) - oracle.mean_f64(v)) <= scale / n
    assert hip.max_of(d) == oracle.max_of_f64(v)
    assert hip.argmax(d) == oracle.argmax_f64(v)
    if n > 3:  # a view starting one double in: 8-byte aligned only
        w = d.sub(1, (n - 1,))
        assert abs(hip.sum(w) - oracle.sum_f64(v[1:])) <= scale
        assert hip.argmax(w) == oracle.argmax_f64(v[1:])


def test_reduction_golden_and_max_semantics(hip, oracle, golden):
    r = golden["reductions"]
    d = hip.from_numpy(np.array(r["v"], np.float64))
    assert (hip.sum(d), hip.mean(d), hip.max_of(d)) == (r["sum"], r["mean"], r["max_of"])
    v = np.array([1.0, 5.0, 5.0, -0.0, 0.0, np.nan, 2.0] * 1000)
    dv = hip.from_numpy(v)
    assert hip.max_of(dv) == 5.0 and hip.argmax(dv) == 1
    nanfirst = hip.from_numpy(np.array([np.nan, 3.0, 4.0]))
    assert np.isnan(hip.max_of(nanfirst)) and hip.argmax(nanfirst) == 0
    z = hip.from_numpy(np.array([-0.0, 0.0] * 5000))
    assert np.signbit(hip.max_of(z)) and hip.argmax(z) == 0


def test_index_and_its_reverse_rule(hip, oracle):
    t = np.arange(3 * 5 * 7, dtype=np.float64).reshape(3, 5, 7) * 0.125 - 2.0
    d = hip.from_numpy(t)
    for idx in [(0, 0, 0), (2, 4, 6), (1, 3, 2)]:
        assert hip.index(d, idx) == oracle.index_f64(t, idx)
    dt = hip.from_numpy(np.zeros((3, 5, 7)))
    hip.index_bwd(2.5, dt, (1, 2, 3))
    hip.index_bwd(0.25, dt, (1, 2, 3))
    ref = np.zeros((3, 5, 7))
    oracle.index_bwd_f64(2.5, ref, (1, 2, 3))
    oracle.index_bwd_f64(0.25, ref, (1, 2, 3))
    assert np.array_equal(dt.numpy(), ref)


def test_host_forms(hip, oracle):
    from cleave_amd import host

    rng = np.random.default_rng(64)
    A = rng.standard_normal((70, 45))
    B = rng.standard_normal((45, 33))
    got = host.matmul(A, B)
    assert got.dtype == np.float64
    _assert_gemm64(got, oracle.matmul_f64(A, B), np.abs(A) @ np.abs(B), 45, "host f64")
    a = rng.standard_normal(5001)
    b = rng.standard_normal(5001) + 3
    assert np.array_equal(host.add(a, b), oracle.add_f64(a, b))
    assert np.array_equal(host.div(a, b), oracle.div_f64(a, b))
    assert rel_close(host.sigmoid(a), oracle.sigmoid_f64(a), rtol=1e-14)
    assert abs(host.sum(a) - oracle.sum_f64(a)) <= SUM_TOL * np.sqrt(a.size) * np.abs(a).sum()
    assert host.max_of(a) == oracle.max_of_f64(a) and host.argmax(a) == oracle.argmax_f64(a)
    t = rng.standard_normal((4, 6))
    assert host.index(t, (3, 5)) == t[3, 5]
    Ab = rng.standard_normal((3, 20, 10))
    Bb = rng.standard_normal((3, 10, 15))
    gb = host.matmul_batched(Ab, Bb)
    for i in range(3):
        _assert_gemm64(gb[i], oracle.matmul_f64(Ab[i], Bb[i]), np.abs(Ab[i]) @ np.abs(Bb[i]), 10, "host batched f64")


@pytest.mark.parametrize("ta,tb", [(False, False), (True, True)])
def test_memref_forms(hip, oracle, ta, tb):
    # memref<... x f64> descriptors: strides select the transposed products,
    # rank 3 the batched one; maps, reductions and Index as in f32
    from cleave_amd import memref as mr

    rng = np.random.default_rng(65 + ta)
    M, N, K = 70, 50, 30
    A = rng.standard_normal((K, M) if ta else (M, K))
    B = rng.standard_normal((N, K) if tb else (K, N))
    a, b, c = hip.from_numpy(A), hip.from_numpy(B), hip.empty((M, N), "f64")
    mr.call("cleave_hip_matmul_f64", mr.transposed(a) if ta else mr.of(a), mr.transposed(b) if tb else mr.of(b),
            mr.of(c))
    ref = oracle.matmul_f64(A, B, trans_a=ta, trans_b=tb)
    _assert_gemm64(c.numpy(), ref, np.abs(A.T if ta else A) @ np.abs(B.T if tb else B), K, "memref f64")
    A3, B3 = rng.standard_normal((2, M, K)), rng.standard_normal((2, K, N))
    c3 = hip.empty((2, M, N), "f64")
    mr.call("cleave_hip_matmul_f64", mr.of(hip.from_numpy(A3)), mr.of(hip.from_numpy(B3)), mr.of(c3))
    for i in range(2):
        _assert_gemm64(c3.numpy()[i], oracle.matmul_f64(A3[i], B3[i]), np.abs(A3[i]) @ np.abs(B3[i]), K, "rank 3")
    x = rng.standard_normal((17, 9))
    y = rng.standard_normal((17, 9)) + 4
    dx, dy, out = hip.from_numpy(x), hip.from_numpy(y), hip.empty((17, 9), "f64")
    for name in ("add", "sub", "mul", "div"):
        mr.call(f"cleave_hip_{name}_f64", mr.of(dx), mr.of(dy), mr.of(out))
        assert np.array_equal(out.numpy(), getattr(oracle, f"{name}_f64")(x, y)), name
    mr.call("cleave_hip_tanh_f64", mr.of(dx), mr.of(out))
    assert rel_close(out.numpy(), oracle.tanh_f64(x), rtol=1e-14)
    mr.call("cleave_hip_relu_bwd_f64", mr.of(dx), mr.of(dy), mr.of(out))
    assert np.array_equal(out.numpy(), oracle.relu_bwd_f64(x, y))
    assert abs(mr.call("cleave_hip_sum_f64", mr.of(dx)) - oracle.sum_f64(x)) <= SUM_TOL * np.sqrt(x.size) * np.abs(x).sum()
    assert mr.call("cleave_hip_max_of_f64", mr.of(dx)) == oracle.max_of_f64(x)
    assert mr.call("cleave_hip_argmax_f64", mr.of(dx)) == oracle.argmax_f64(x)
    idx = np.array([16, 8], np.int32)
    assert mr.call("cleave_hip_index_f64", mr.of(dx), mr.host(idx)) == x[16, 8]
    g = hip.from_numpy(np.zeros((17, 9)))
    mr.call("cleave_hip_index_bwd_f64", 1.25, mr.of(g), mr.host(idx))
    want = np.zeros((17, 9))
    want[16, 8] = 1.25
    assert np.array_equal(g.numpy(), want)
