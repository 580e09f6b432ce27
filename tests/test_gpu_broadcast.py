"""Broadcasting maps and their reverse rule on the GPU (an extension: the
reference's Ring<Tensor> maps need equal shapes, stdlib/linalg/tensor.cleave:66-71,
and Activation<Tensor> is rank 1, stdlib/nn/nn.cleave:82).

The maps are one IEEE operation per output element, so they must equal the
oracle's restated loop (oracle/oracle.c or_bcast_*) bit for bit; the oracle is
pinned to numpy's broadcast arithmetic in tests/test_oracle.py.  The reverse
rule (cleave_hip_sum_to_shape_*) sums in an order fixed by the shapes, checked
against the oracle under the sum bound |got - ref| <= 1e-6 n sum|g| (f32) and
exactly on integer-valued data; each of its dispatch paths has a case.
"""
from __future__ import annotations


import numpy as np
import pytest

pytestmark = pytest.mark.gpu

_U = {np.float32: np.uint32, np.float64: np.uint64}

# Shapes chosen for the kernel's paths: a last dimension that is a multiple of
# the 16-byte chunk (vector loads) or not (element loads), an operand
# broadcast along the last dimension (stride 0 there), rank 0, stretched
# dimensions in the middle, both operands stretched, and more than 2^31
# elements of output (64-bit indexing).
_PAIRS = [
    ((65536, 4096), (4096,)), ((65536, 4096), (65536, 1)), ((4096, 1), (1, 4096)),
    ((8, 1, 512, 1), (1, 64, 1, 300)), ((3, 5, 7), ()), ((), (1000, 3)), ((129, 33), (33,)),
    ((2, 3, 4, 5, 6), (3, 1, 5, 1)), ((1,), (12345,)), ((16, 1, 1, 1, 1, 1, 1, 8), (1, 2, 3, 1, 1, 1, 2, 1)),
    ((0, 7), (7,)), ((1000, 1000), (1000, 1000)),
]


def _rand(rng, shape, dt, shift=0.0):
    return (rng.standard_normal(shape) + shift).astype(dt)


@pytest.mark.parametrize("ashape,bshape", _PAIRS)
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_bcast_maps_bit_exact(hip, oracle, ashape, bshape, dt):
    rng = np.random.default_rng(len(ashape) * 17 + len(bshape) + (dt == np.float64))
    A, B = _rand(rng, ashape, dt), _rand(rng, bshape, dt, 3.0)
    a, b = hip.from_numpy(A), hip.from_numpy(B)
    for op in ("add", "sub", "mul", "div"):
        got = getattr(hip, op)(a, b).numpy()
        ref = oracle.bcast(op, A, B, f64=dt == np.float64)
        assert got.shape == ref.shape
        assert np.array_equal(got.view(_U[dt]), ref.view(_U[dt])), f"{op} {ashape} {bshape}"


def test_bcast_past_2pow31_elements(hip, oracle):
    # 2^31 + 2^20 outputs: the 64-bit index path; checked at sampled rows
    rows, cols = (1 << 19) + 256, 4096
    rng = np.random.default_rng(8)
    B = rng.standard_normal((rows, 1)).astype(np.float32)
    A = rng.standard_normal((cols,)).astype(np.float32)
    a, b = hip.from_numpy(A), hip.from_numpy(B)
    out = hip.mul(b, a)  # (rows, 1) * (cols,) -> rows x cols
    assert out.shape == (rows, cols)
    for r in (0, 1, rows // 2, rows - 1):
        row = out.sub(r * cols, (cols,)).numpy()
        assert np.array_equal(row, B[r, 0] * A), r
    del out


def test_bcast_row_bias_equals_add_row_bias(hip):
    rng = np.random.default_rng(4)
    A, bias = rng.standard_normal((777, 1024)).astype(np.float32), rng.standard_normal(1024).astype(np.float32)
    a, b = hip.from_numpy(A), hip.from_numpy(bias)
    assert np.array_equal(hip.add(a, b).numpy(), hip.add_row_bias(a, b).numpy())


def test_bcast_unaligned_views(hip, oracle):
    # operands starting one element into their buffers: element loads
    rng = np.random.default_rng(6)
    A, B = rng.standard_normal((300, 64)).astype(np.float32), rng.standard_normal((64,)).astype(np.float32)
    abuf = hip.from_numpy(np.concatenate([np.zeros(1, np.float32), A.ravel()]))
    bbuf = hip.from_numpy(np.concatenate([np.zeros(3, np.float32), B]))
    got = hip.sub(abuf.sub(1, (300, 64)), bbuf.sub(3, (64,))).numpy()
    assert np.array_equal(got, oracle.bcast("sub", A, B))


def test_bcast_errors(hip):
    # the Python binding runs with abort-on-error off: statuses come back
    from cleave_amd._lib import ERR_ARG, last_error, load

    a, b = hip.from_numpy(np.ones((3, 4), np.float32)), hip.from_numpy(np.ones((3,), np.float32))
    with pytest.raises(ValueError):
        hip.add(a, b)  # the mirror checks first
    lib = load()
    out = hip.empty((3, 4))
    sa, sb = np.array([3, 4], np.int32), np.array([3], np.int32)
    r = lib.cleave_hip_add_bcast_f32(a.ptr, 12, sa.ctypes.data, 2, b.ptr, 3, sb.ctypes.data, 1, out.ptr, 12)
    assert r == ERR_ARG and "do not broadcast" in last_error()[1]
    sb2 = np.array([4], np.int32)
    r = lib.cleave_hip_add_bcast_f32(a.ptr, 12, sa.ctypes.data, 2, b.ptr, 3, sb2.ctypes.data, 1, out.ptr, 12)
    assert r == ERR_ARG  # b's length does not match its shape
    r = lib.cleave_hip_add_bcast_f32(a.ptr, 12, sa.ctypes.data, 9, b.ptr, 3, sb.ctypes.data, 1, out.ptr, 12)
    assert r == ERR_ARG  # rank above 8
    g = hip.from_numpy(np.ones((3, 4), np.float32))
    so = np.array([2, 4], np.int32)
    r = lib.cleave_hip_sum_to_shape_f32(g.ptr, 12, sa.ctypes.data, 2, out.ptr, 8, so.ctypes.data, 2)
    assert r == ERR_ARG  # (2, 4) does not broadcast to (3, 4)


# sum_to_shape paths: copy (nothing stretched), Sum (everything), column sums
# ([R, K]: vector and element forms), block per row ([K, R], R >= 256), and
# one thread per output (every other pattern)
_SUMS = [
    ((64, 512), (64, 512)), ((3, 1, 5), (1, 1, 5)), ((1 << 20,), ()), ((4096, 100), (1, 1)),
    ((65536, 4096), (4096,)), ((1000, 37), (37,)), ((4096, 4096), (4096, 1)), ((256, 300), (256, 1)),
    ((4096, 100), (4096, 1)), ((64, 512, 512), (1, 512, 1)), ((128, 64, 300), (128, 1, 300)),
    ((2, 3, 4, 5), (3, 1, 1)),
]


@pytest.mark.parametrize("gshape,oshape", _SUMS)
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_sum_to_shape_against_oracle(hip, oracle, gshape, oshape, dt):
    rng = np.random.default_rng(len(gshape) + 3 * len(oshape) + (dt == np.float64))
    G = rng.standard_normal(gshape).astype(dt)
    g = hip.from_numpy(G)
    got = hip.sum_to_shape(g, oshape).numpy()
    again = hip.sum_to_shape(g, oshape).numpy()
    assert np.array_equal(got.view(_U[dt]), again.view(_U[dt])), "repeat"
    ref = oracle.sum_to_shape(G, oshape, f64=dt == np.float64)
    R = len(gshape)
    full = (1,) * (R - len(oshape)) + tuple(oshape)
    axes = tuple(i for i in range(R) if full[i] == 1 and gshape[i] != 1)
    den = np.abs(G.astype(np.float64)).sum(axis=axes, keepdims=True).reshape(oshape)
    n = max(1, int(np.prod([gshape[i] for i in axes])))
    eps = 1e-6 if dt == np.float32 else 1e-15
    assert got.shape == tuple(oshape)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= eps * n * den + 1e-30)
    # integer values: exact in every order
    Gi = rng.integers(-20, 20, gshape).astype(dt)
    assert np.array_equal(hip.sum_to_shape(hip.from_numpy(Gi), oshape).numpy(),
                          oracle.sum_to_shape(Gi, oshape, f64=dt == np.float64))


@pytest.mark.parametrize("gshape,oshape", [((0, 5), (1, 5)), ((0, 5), (5,)), ((3, 0, 4), (3, 1, 4)), ((0,), ()),
                                           ((2, 0), (2, 1))])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_sum_to_shape_over_an_empty_dimension_is_zero(hip, oracle, gshape, oshape, dt):
    # a reduced dimension of 0 sums over nothing: zeros, as numpy and the
    # oracle give, over whatever out held before
    G = np.zeros(gshape, dt)
    out = hip.from_numpy(np.full(oshape, np.nan, dt))
    got = hip.sum_to_shape(hip.from_numpy(G), oshape, out=out).numpy()
    assert got.shape == tuple(oshape)
    assert np.array_equal(got, oracle.sum_to_shape(G, oshape, f64=dt == np.float64))
    assert np.array_equal(got, np.zeros(oshape, dt))


def test_sum_to_shape_general_path_is_the_oracle_order(hip, oracle):
    # the one-thread-per-output path adds each output's terms in row-major
    # order from zero, as the oracle does: bit for bit
    rng = np.random.default_rng(12)
    G = rng.standard_normal((64, 512, 40)).astype(np.float32)
    got = hip.sum_to_shape(hip.from_numpy(G), (1, 512, 1)).numpy()
    assert np.array_equal(got, oracle.sum_to_shape(G, (1, 512, 1)))


def test_host_forms(hip, oracle):
    from cleave_amd._lib import load

    lib = load()
    rng = np.random.default_rng(14)
    A, B = rng.standard_normal((50, 30)).astype(np.float32), rng.standard_normal((50, 1)).astype(np.float32)
    out = np.zeros((50, 30), np.float32)
    sa, sb = np.array([50, 30], np.int32), np.array([50, 1], np.int32)
    assert lib.cleave_hip_div_bcast_f32_host(A.ctypes.data, A.size, sa.ctypes.data, 2, B.ctypes.data, B.size,
                                             sb.ctypes.data, 2, out.ctypes.data, out.size) == 0
    assert np.array_equal(out, oracle.bcast("div", A, B))
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    out64 = np.zeros((50, 30))
    assert lib.cleave_hip_mul_bcast_f64_host(A64.ctypes.data, A64.size, sa.ctypes.data, 2, B64.ctypes.data,
                                             B64.size, sb.ctypes.data, 2, out64.ctypes.data, out64.size) == 0
    assert np.array_equal(out64, oracle.bcast("mul", A64, B64, f64=True))
    s = np.zeros(30, np.float32)
    so = np.array([30], np.int32)
    assert lib.cleave_hip_sum_to_shape_f32_host(A.ctypes.data, A.size, sa.ctypes.data, 2, s.ctypes.data, 30,
                                                so.ctypes.data, 1) == 0
    assert np.allclose(s, A.astype(np.float64).sum(axis=0), rtol=0, atol=1e-5 * np.abs(A).sum(axis=0).max())


def test_tape_broadcast_gradients(hip):
    # loss = sum(((X W + b) * s - c) / d): b (H,), s (1, H), c (B, 1), d a
    # scalar shape (); every gradient against float64 numpy
    from cleave_amd import autograd as ag

    rng = np.random.default_rng(21)
    Bn, D, H = 300, 40, 130
    X = rng.standard_normal((Bn, D)).astype(np.float32)
    W = (rng.standard_normal((D, H)) * 0.1).astype(np.float32)
    b = rng.standard_normal(H).astype(np.float32)
    s = rng.standard_normal((1, H)).astype(np.float32)
    c = rng.standard_normal((Bn, 1)).astype(np.float32)
    d = np.array(1.5, np.float32)
    vX = ag.const(X)
    vW, vb, vs, vc, vd = (ag.param(v) for v in (W, b, s, c, d))
    z = ag.div(ag.sub(ag.mul(ag.add(ag.matmul(vX, vW), vb), vs), vc), vd)
    loss = ag.sum(z)
    ag.backward(loss)
    X64, W64, b64, s64, c64, d64 = (v.astype(np.float64) for v in (X, W, b, s, c, d))
    Z = X64 @ W64 + b64
    ones = np.ones((Bn, H))
    g_pre = ones * s64 / d64                      # d loss / d (XW + b)
    want = {
        "W": X64.T @ g_pre, "b": g_pre.sum(axis=0), "s": (Z / d64).sum(axis=0, keepdims=True),
        "c": -(ones / d64).sum(axis=1, keepdims=True),
        "d": -(((Z * s64 - c64)) / (d64 * d64)).sum(),
    }
    for name, v in (("W", vW), ("b", vb), ("s", vs), ("c", vc), ("d", vd)):
        got = v.grad.numpy().astype(np.float64).reshape(np.shape(want[name]))
        scale = np.abs(want[name]).max() + 1e-30
        assert np.max(np.abs(got - want[name])) <= 1e-4 * scale, name
