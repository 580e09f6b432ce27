"""Every `extern(symbol) fn` that the integration guide declares on the cleave side,
called on the GPU exactly as the reference's lowering would call it
(tests/cleave_decls.py: each array argument as (pointer, i64 length), an array
result as the first array argument handed back, the C result an i64), and its
cleave-level result checked against the oracle."""
from __future__ import annotations

import numpy as np
import pytest

import cleave_decls as cd
from helpers import assert_gemm_close, rel_close

pytestmark = pytest.mark.gpu

NP = {"f32": np.float32, "f64": np.float64, "i32": np.int32, "i64": np.int64}


def call_lowered(e: cd.Extern, values):
    """Lowers one call of `e` on `values` (one per cleave parameter) and runs it."""
    from cleave_amd._lib import last_error, load

    lib = load()
    args, arrays = [], []
    for (_, t), v in zip(e.params, values):
        if cd.is_array(t):
            assert isinstance(v, np.ndarray) and v.dtype == NP[cd.array_elem(t)] and v.flags["C_CONTIGUOUS"]
            arrays.append(v)
            args += [v.ctypes.data, v.size]
        else:
            args.append(v)
    r = getattr(lib, e.symbol)(*args)
    code, msg = last_error()
    if cd.is_array(e.ret):
        assert r == arrays[0].size, f"{e.symbol} returned {r} ({msg})"
        return arrays[0]  # the array-return identity
    assert code == 0, f"{e.symbol}: {msg}"
    return r


@pytest.fixture(scope="module")
def externs(hip):
    _, ex = cd.parse()
    return {e.symbol: e for e in ex}


def _vals(rng, n, lo=-3.0, hi=3.0):
    return rng.uniform(lo, hi, n).astype(np.float32)


def test_reductions(externs, oracle):
    rng = np.random.default_rng(90)
    for n in (1, 7, 4099, 1 << 20):
        x = rng.standard_normal(n).astype(np.float32)
        s = call_lowered(externs["cleave_hip_sum_f32_host"], [x])
        assert abs(s - oracle.sum_f32(x)) <= 1e-5 * float(np.sum(np.abs(x), dtype=np.float64))
        m = call_lowered(externs["cleave_hip_mean_f32_host"], [x])
        assert abs(m - oracle.mean_f32(x)) <= 1e-5 * float(np.sum(np.abs(x), dtype=np.float64)) / n
        assert call_lowered(externs["cleave_hip_max_of_f32_host"], [x]) == oracle.max_of(x)
        assert call_lowered(externs["cleave_hip_argmax_f32_host"], [x]) == oracle.argmax(x)
    # i32 counts summed exactly in i64, negative values included
    for n in (1, 5, 1000003):
        c = rng.integers(-2**31, 2**31, n, dtype=np.int64).astype(np.int32)
        assert call_lowered(externs["cleave_hip_sum_i32_i64_host"], [c]) == int(np.sum(c, dtype=np.int64))
    big = np.full(1 << 22, 2**31 - 1, np.int32)  # the total needs all 64 bits of the sum's range
    assert call_lowered(externs["cleave_hip_sum_i32_i64_host"], [big]) == (2**31 - 1) << 22


def test_index_at(externs, oracle):
    t = np.arange(3 * 5 * 7, dtype=np.float32) * 0.5 - 3.0
    dims = np.array([3, 5, 7], np.int32)
    for idx in ([0, 0, 0], [2, 4, 6], [1, 3, 2]):
        got = call_lowered(externs["cleave_hip_index_f32_host"], [t, dims, np.array(idx, np.int32)])
        assert got == oracle.index(t.reshape(3, 5, 7), tuple(idx))


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_matmul_into(externs, oracle, ta, tb):
    rng = np.random.default_rng(91 + 2 * ta + tb)
    M, N, K = 67, 130, 45
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    c0 = np.zeros(M * N, np.float32)  # the `[0.0; MN]` a caller passes
    c = call_lowered(externs["cleave_hip_matmul_f32_into"], [c0, A.ravel(), B.ravel(), M, N, K, ta, tb])
    assert c is c0
    ref = oracle.matmul(A, B, trans_a=bool(ta), trans_b=bool(tb))
    den = np.abs(A.T if ta else A).astype(np.float64) @ np.abs(B.T if tb else B).astype(np.float64)
    assert_gemm_close(c.reshape(M, N), ref, den, K, f"matmul_into ta={ta} tb={tb}")


def test_maps_into(externs, oracle):
    rng = np.random.default_rng(92)
    n = 10007
    a, b = _vals(rng, n), _vals(rng, n, 0.5, 2.0)
    s = oracle.sigmoid(a)
    g = _vals(rng, n)
    exact2 = {"add": (a, b, oracle.add), "sub": (a, b, oracle.sub), "mul": (a, b, oracle.mul),
              "div": (a, b, oracle.div), "sigmoid_bwd": (s, g, oracle.sigmoid_bwd),
              "tanh_bwd": (oracle.tanh(a), g, oracle.tanh_bwd), "relu_bwd": (a, g, oracle.relu_bwd)}
    for op, (x, y, f) in exact2.items():
        out = call_lowered(externs[f"cleave_hip_{op}_f32_into"], [np.zeros(n, np.float32), x, y])
        assert np.array_equal(out, f(x, y)), op
    for op, f in {"neg": oracle.neg, "relu": oracle.relu}.items():
        out = call_lowered(externs[f"cleave_hip_{op}_f32_into"], [np.zeros(n, np.float32), a])
        assert np.array_equal(out, f(a)), op
    for op, f in {"sigmoid": oracle.sigmoid, "tanh": oracle.tanh}.items():
        out = call_lowered(externs[f"cleave_hip_{op}_f32_into"], [np.zeros(n, np.float32), a])
        assert rel_close(out, f(a), rtol=1e-5), op


def test_an_into_call_that_fails_returns_its_status_and_leaves_out_alone(externs):
    from cleave_amd._lib import ERR_ARG, load

    lib = load()
    out = np.full(8, 7.0, np.float32)
    x = np.ones(9, np.float32)  # length mismatch
    r = lib.cleave_hip_sigmoid_f32_into(out.ctypes.data, out.size, x.ctypes.data, x.size)
    assert r == ERR_ARG and np.all(out == 7.0)


def test_escape_grid(externs, oracle):
    # the reference example's own window (examples/mandelbrot.cleave:30-35) in f32,
    # then a larger grid
    for (w, h, x0, y0, dx, dy, it) in [(70, 25, -2.5, -1.25, 0.05, 0.1, 50),
                                      (640, 480, -2.0, -1.5, 3.0 / 640, 3.0 / 480, 300)]:
        out0 = np.zeros(w * h, np.int32)
        out = call_lowered(externs["cleave_hip_escape_grid_i32"],
                           [out0, w, h, float(x0), float(y0), float(dx), float(dy), it])
        ref = oracle.mandelbrot(w, h, x0, y0, np.float32(dx), np.float32(dy), it)
        assert out is out0 and np.array_equal(out.reshape(h, w), ref.astype(np.int32))
        total = call_lowered(externs["cleave_hip_sum_i32_i64_host"], [out])
        assert total == int(ref.sum(dtype=np.int64))


def test_f64_declarations(externs, oracle):
    # the Tensor<f64> impls of the same blocks: reductions, IndexAt, MatMulInto, MapInto
    rng = np.random.default_rng(93)
    x = rng.standard_normal(20011) * 2 + 0.1
    tol = 2e-14 * np.sqrt(x.size) * np.abs(x).sum()
    assert abs(call_lowered(externs["cleave_hip_sum_f64_host"], [x]) - oracle.sum_f64(x)) <= tol
    assert abs(call_lowered(externs["cleave_hip_mean_f64_host"], [x]) - oracle.mean_f64(x)) <= tol / x.size
    assert call_lowered(externs["cleave_hip_max_of_f64_host"], [x]) == oracle.max_of_f64(x)
    assert call_lowered(externs["cleave_hip_argmax_f64_host"], [x]) == oracle.argmax_f64(x)
    t = rng.standard_normal((4, 3, 5))
    got = call_lowered(externs["cleave_hip_index_f64_host"], [t.ravel(), np.array([4, 3, 5], np.int32),
                                                              np.array([3, 1, 4], np.int32)])
    assert got == t[3, 1, 4]
    M, N, K = 45, 70, 33
    A, B = rng.standard_normal((M, K)), rng.standard_normal((K, N))
    c0 = np.zeros(M * N)
    c = call_lowered(externs["cleave_hip_matmul_f64_into"], [c0, A.ravel(), B.ravel(), M, N, K, 0, 0])
    assert c is c0
    ref = oracle.matmul_f64(A, B)
    err = np.max(np.abs(c.reshape(M, N) - ref) / (np.abs(A) @ np.abs(B)))
    assert err <= 2e-14 * np.sqrt(K)
    a, b = rng.standard_normal(999), rng.standard_normal(999) + 3
    for op, f in {"add": oracle.add_f64, "sub": oracle.sub_f64, "mul": oracle.mul_f64, "div": oracle.div_f64,
                  "relu_bwd": oracle.relu_bwd_f64}.items():
        out = call_lowered(externs[f"cleave_hip_{op}_f64_into"], [np.zeros(999), a, b])
        assert np.array_equal(out, f(a, b)), op
    out = call_lowered(externs["cleave_hip_sigmoid_f64_into"], [np.zeros(999), a])
    assert rel_close(out, oracle.sigmoid_f64(a), rtol=1e-14)
