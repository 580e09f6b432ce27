"""ctypes wrapper of liboracle.so -- the CPU restatement (TEST INFRASTRUCTURE).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module.  It is the checker: the product (cleave_amd / libcleave_hip.so)
never imports or calls it.  Function-level citations of the reference live in
oracle/oracle.c.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_f = C.c_float
_i32 = C.c_int32
_i64 = C.c_int64
_u64 = C.c_uint64
_p = C.c_void_p

_SIGS = {
    "or_splitmix64_at": (_u64, [_u64, _u64]),
    "or_fill_uniform_f32": (None, [_p, _i64, _u64, _f, _f]),
    "or_fill_normal_f32": (None, [_p, _i64, _u64, _f, _f]),
    "or_f32_to_bf16": (C.c_uint16, [_f]),
    "or_bf16_to_f32": (_f, [C.c_uint16]),
    "or_f32_to_bf16_array": (None, [_p, _p, _i64]),
    "or_matmul_f32_rows": (None, [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "or_matmul_f32": (None, [_p, _p, _p, _i32, _i32, _i32, _i32, _i32]),
    "or_matmul_f32_mt": (None, [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32]),
    "or_matmul_f32_entries": (None, [_p, _p, _i32, _i32, _i32, _i32, _i32, _p, _p, _i64, _p, _p]),
    "or_matmul_bf16_entries": (None, [_p, _p, _i32, _i32, _i32, _i32, _i32, _p, _p, _i64, _p, _p]),
    "or_matmul_bf16_rows": (None, [_p, _p, _p, _i32, _i32, _i32, _i32, _i32]),
    "or_add_f32": (None, [_p, _p, _p, _i64]),
    "or_sub_f32": (None, [_p, _p, _p, _i64]),
    "or_mul_f32": (None, [_p, _p, _p, _i64]),
    "or_div_f32": (None, [_p, _p, _p, _i64]),
    "or_neg_f32": (None, [_p, _p, _i64]),
    "or_relu_f32": (None, [_p, _p, _i64]),
    "or_sigmoid_f32": (None, [_p, _p, _i64]),
    "or_tanh_f32": (None, [_p, _p, _i64]),
    "or_sigmoid_scalar": (_f, [_f]),
    "or_sigmoid_bwd_f32": (None, [_p, _p, _p, _i64]),
    "or_tanh_bwd_f32": (None, [_p, _p, _p, _i64]),
    "or_relu_bwd_f32": (None, [_p, _p, _p, _i64]),
    "or_div_bwd_f32": (None, [_p, _p, _p, _p, _p, _i64]),
    "or_sum_f32": (_f, [_p, _i64]),
    "or_mean_f32": (_f, [_p, _i64]),
    "or_max_of_f32": (_f, [_p, _i64]),
    "or_argmax_f32": (_i64, [_p, _i64]),
    "or_index_f32": (_i32, [_p, _p, _i32, _p, _p]),
    "or_add_row_bias_f32": (None, [_p, _p, _p, _i32, _i32]),
    "or_sum_rows_f32": (None, [_p, _p, _i32, _i32]),
    "or_bcast_f32": (_i32, [_i32, _p, _p, _i32, _p, _p, _i32, _p]),
    "or_bcast_f64": (_i32, [_i32, _p, _p, _i32, _p, _p, _i32, _p]),
    "or_sum_to_shape_f32": (_i32, [_p, _p, _i32, _p, _p, _i32]),
    "or_sum_to_shape_f64": (_i32, [_p, _p, _i32, _p, _p, _i32]),
    "or_index_bwd_f32": (_i32, [_f, _p, _p, _i32, _p]),
    "or_sum_u32_u64": (_u64, [_p, _i64]),
    "or_escape_count_f32": (C.c_uint32, [_f, _f, _i32]),
    "or_escape_count_latch_f32": (C.c_uint32, [_f, _f, _i32]),
    "or_mandelbrot_rows": (None, [_p, _i32, _i32, _f, _f, _f, _f, _i32, _i32, _i32]),
    "or_mandelbrot_mt": (None, [_p, _i32, _i32, _f, _f, _f, _f, _i32, _i32]),
    "or_mlp_step_f32": (_f, [_p, _p, _p, _p, _i32, _i32, _i32, _f, _p, _p, _i32]),
    "or_mlp_loss_f64": (C.c_double, [_p, _p, _p, _p, _i32, _i32, _i32]),
    "or_mlp_grad_entries": (_f, [_p, _p, _p, _p, _i32, _i32, _i32, _p, _p, _i64, _p, _p, _p, _i64, _p, _p,
                                 _i32]),
    "or_mandelbrot_rows_mt": (None, [_p, _i32, _i32, _f, _f, _f, _f, _i32, _i32, _i32, _i32]),
    "or_xor_tensor_train": (None, [_i32, _f, _p]),
    # f64 forms
    "or_matmul_f64_rows": (None, [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "or_matmul_f64_mt": (None, [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32]),
    "or_add_f64": (None, [_p, _p, _p, _i64]),
    "or_sub_f64": (None, [_p, _p, _p, _i64]),
    "or_mul_f64": (None, [_p, _p, _p, _i64]),
    "or_div_f64": (None, [_p, _p, _p, _i64]),
    "or_neg_f64": (None, [_p, _p, _i64]),
    "or_relu_f64": (None, [_p, _p, _i64]),
    "or_sigmoid_f64": (None, [_p, _p, _i64]),
    "or_sigmoid_f64_scalar": (C.c_double, [C.c_double]),
    "or_tanh_f64": (None, [_p, _p, _i64]),
    "or_sigmoid_bwd_f64": (None, [_p, _p, _p, _i64]),
    "or_tanh_bwd_f64": (None, [_p, _p, _p, _i64]),
    "or_relu_bwd_f64": (None, [_p, _p, _p, _i64]),
    "or_div_bwd_f64": (None, [_p, _p, _p, _p, _p, _i64]),
    "or_add_row_bias_f64": (None, [_p, _p, _p, _i32, _i32]),
    "or_sum_rows_f64": (None, [_p, _p, _i32, _i32]),
    "or_index_f64": (_i32, [_p, _p, _i32, _p, _p]),
    "or_index_bwd_f64": (_i32, [C.c_double, _p, _p, _i32, _p]),
    "or_sum_f64": (C.c_double, [_p, _i64]),
    "or_mean_f64": (C.c_double, [_p, _i64]),
    "or_max_of_f64": (C.c_double, [_p, _i64]),
    "or_argmax_f64": (_i64, [_p, _i64]),
}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- generators --------------------------------------------------------------

def splitmix64_at(seed: int, i: int) -> int:
    return int(lib().or_splitmix64_at(seed, i))


def uniform(n: int, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_fill_uniform_f32(_ptr(out), n, seed, lo, hi)
    return out


def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_fill_normal_f32(_ptr(out), n, seed, mean, std)
    return out


def to_bf16(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16_array(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


# ---- matmul -------------------------------------------------------------------

def matmul(A, B, trans_a=False, trans_b=False, threads: int = 0) -> np.ndarray:
    A, B = _f32(A), _f32(B)
    M, K = (A.shape[1], A.shape[0]) if trans_a else A.shape
    N = B.shape[0] if trans_b else B.shape[1]
    C_ = np.empty((M, N), np.float32)
    if threads > 0:
        lib().or_matmul_f32_mt(_ptr(A), _ptr(B), _ptr(C_), M, N, K, int(trans_a), int(trans_b), threads)
    else:
        lib().or_matmul_f32(_ptr(A), _ptr(B), _ptr(C_), M, N, K, int(trans_a), int(trans_b))
    return C_


def matmul_rows(A, B, M, N, K, row0, row1, trans_a=False, trans_b=False) -> np.ndarray:
    """Rows [row0,row1) of C; the rest of the returned buffer is unspecified."""
    A, B = _f32(A), _f32(B)
    C_ = np.empty((M, N), np.float32)
    lib().or_matmul_f32_rows(_ptr(A), _ptr(B), _ptr(C_), M, N, K, int(trans_a), int(trans_b), row0, row1)
    return C_[row0:row1]


def matmul_bf16_rows(A, B, M, N, K, row0, row1) -> np.ndarray:
    """Rows [row0,row1) of the A*B product of bf16 bit arrays (NN), upcast to f32."""
    A = np.ascontiguousarray(A, np.uint16)
    B = np.ascontiguousarray(B, np.uint16)
    C_ = np.empty((M, N), np.float32)
    lib().or_matmul_bf16_rows(_ptr(A), _ptr(B), _ptr(C_), M, N, K, row0, row1)
    return C_[row0:row1]


def matmul_entries(A, B, M, N, K, ii, jj, trans_a=False, trans_b=False, bf16=False):
    """C[ii[e], jj[e]] and sum_k |a||b| for each entry."""
    ii = np.ascontiguousarray(ii, np.int32)
    jj = np.ascontiguousarray(jj, np.int32)
    out = np.empty(ii.size, np.float32)
    absout = np.empty(ii.size, np.float32)
    if bf16:
        A = np.ascontiguousarray(A, np.uint16)
        B = np.ascontiguousarray(B, np.uint16)
        fn = lib().or_matmul_bf16_entries
    else:
        A, B = _f32(A), _f32(B)
        fn = lib().or_matmul_f32_entries
    fn(_ptr(A), _ptr(B), M, N, K, int(trans_a), int(trans_b), _ptr(ii), _ptr(jj), ii.size,
       _ptr(out), _ptr(absout))
    return out, absout


# ---- maps -----------------------------------------------------------------------

def _map1(name, a):
    a = _f32(a)
    out = np.empty_like(a)
    getattr(lib(), name)(_ptr(a), _ptr(out), a.size)
    return out


def _map2(name, a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    getattr(lib(), name)(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out


def add(a, b): return _map2("or_add_f32", a, b)
def sub(a, b): return _map2("or_sub_f32", a, b)
def mul(a, b): return _map2("or_mul_f32", a, b)
def div(a, b): return _map2("or_div_f32", a, b)
def neg(a): return _map1("or_neg_f32", a)
def relu(a): return _map1("or_relu_f32", a)
def sigmoid(a): return _map1("or_sigmoid_f32", a)
def tanh(a): return _map1("or_tanh_f32", a)
def sigmoid_bwd(s, g): return _map2("or_sigmoid_bwd_f32", s, g)
def tanh_bwd(t, g): return _map2("or_tanh_bwd_f32", t, g)
def relu_bwd(x, g): return _map2("or_relu_bwd_f32", x, g)


def div_bwd(a, b, g):
    a, b, g = _f32(a), _f32(b), _f32(g)
    da, db = np.empty_like(a), np.empty_like(a)
    lib().or_div_bwd_f32(_ptr(a), _ptr(b), _ptr(g), _ptr(da), _ptr(db), a.size)
    return da, db


# ---- row-broadcast bias ----------------------------------------------------------------

def add_row_bias(a, bias) -> np.ndarray:
    a, bias = _f32(a), _f32(bias)
    rows, cols = a.shape
    assert bias.shape == (cols,)
    out = np.empty_like(a)
    lib().or_add_row_bias_f32(_ptr(a), _ptr(bias), _ptr(out), rows, cols)
    return out


def sum_rows(g) -> np.ndarray:
    g = _f32(g)
    rows, cols = g.shape
    out = np.empty(cols, np.float32)
    lib().or_sum_rows_f32(_ptr(g), _ptr(out), rows, cols)
    return out


# ---- broadcasting maps and their reverse rule (extension) -------------------------------

_BCAST_OPS = {"add": 0, "sub": 1, "mul": 2, "div": 3}


def _shape_arg(shape):
    arr = np.ascontiguousarray(np.array(shape, dtype=np.int32).reshape(-1))
    return arr, (_ptr(arr) if arr.size else None)


def _bcast_out_shape(ashape, bshape):
    """The broadcast shape, by the rule itself (aligned at the last dimension,
    missing leading dimensions 1, a 1 stretches); None when it fails."""
    R = max(len(ashape), len(bshape), 1)
    da = (1,) * (R - len(ashape)) + tuple(ashape)
    db = (1,) * (R - len(bshape)) + tuple(bshape)
    out = []
    for x, y in zip(da, db):
        if x != y and x != 1 and y != 1:
            return None
        out.append(y if x == 1 else x)
    return tuple(out) if (len(ashape) or len(bshape)) else ()


def bcast(op: str, a, b, f64: bool = False) -> np.ndarray:
    """a op b under broadcasting (or_bcast_f32 / _f64); ValueError when the
    shapes do not broadcast."""
    conv = _f64 if f64 else _f32
    a, b = conv(a), conv(b)
    shape = _bcast_out_shape(a.shape, b.shape)
    if shape is None:
        raise ValueError(f"shapes {a.shape} and {b.shape} do not broadcast")
    out = np.empty(shape, np.float64 if f64 else np.float32)
    sa, pa = _shape_arg(a.shape)
    sb, pb = _shape_arg(b.shape)
    fn = lib().or_bcast_f64 if f64 else lib().or_bcast_f32
    rc = fn(_BCAST_OPS[op], _ptr(a), pa, a.ndim, _ptr(b), pb, b.ndim, _ptr(out))
    assert rc == 0
    return out


def sum_to_shape(g, shape, f64: bool = False) -> np.ndarray:
    """g summed down to `shape` over the dimensions it stretches
    (or_sum_to_shape_f32 / _f64)."""
    g = (_f64 if f64 else _f32)(g)
    out = np.empty(tuple(shape), np.float64 if f64 else np.float32)
    sg, pg = _shape_arg(g.shape)
    so, po = _shape_arg(tuple(shape))
    fn = lib().or_sum_to_shape_f64 if f64 else lib().or_sum_to_shape_f32
    rc = fn(_ptr(g), pg, g.ndim, _ptr(out), po, len(shape))
    if rc != 0:
        raise ValueError(f"shape {tuple(shape)} does not broadcast to {g.shape}")
    return out


# ---- Index ---------------------------------------------------------------------------

def _dims_idx(shape, idx):
    dims = np.ascontiguousarray(shape, np.int32)
    ix = np.ascontiguousarray(idx, np.int32)
    if dims.size != ix.size:
        raise ValueError("index rank differs from the tensor's")
    return dims, ix


def index(t, idx) -> float:
    """Element of t at idx (row-major); IndexError outside the shape."""
    t = _f32(t)
    dims, ix = _dims_idx(t.shape, idx)
    out = np.zeros(1, np.float32)
    if lib().or_index_f32(_ptr(t), _ptr(dims), dims.size, _ptr(ix), _ptr(out)) != 0:
        raise IndexError(f"index {tuple(idx)} outside shape {t.shape}")
    return float(out[0])


def index_bwd(g: float, dt: np.ndarray, idx) -> None:
    """dt[idx] += g in place (dt float32, C-contiguous); IndexError outside."""
    assert dt.dtype == np.float32 and dt.flags["C_CONTIGUOUS"]
    dims, ix = _dims_idx(dt.shape, idx)
    if lib().or_index_bwd_f32(g, _ptr(dt), _ptr(dims), dims.size, _ptr(ix)) != 0:
        raise IndexError(f"index {tuple(idx)} outside shape {dt.shape}")


# ---- reductions ---------------------------------------------------------------------

def sum_f32(v) -> float:
    v = _f32(v)
    return float(lib().or_sum_f32(_ptr(v), v.size))


def mean_f32(v) -> float:
    v = _f32(v)
    return float(lib().or_mean_f32(_ptr(v), v.size))


def max_of(v) -> float:
    v = _f32(v)
    return float(lib().or_max_of_f32(_ptr(v), v.size))


def argmax(v) -> int:
    v = _f32(v)
    return int(lib().or_argmax_f32(_ptr(v), v.size))


def sum_u64(v) -> int:
    v = np.ascontiguousarray(v, np.uint32)
    return int(lib().or_sum_u32_u64(_ptr(v), v.size))


# ---- escape counts ---------------------------------------------------------------

def escape_count(cr: float, ci: float, max_iter: int, latch: bool = False) -> int:
    fn = lib().or_escape_count_latch_f32 if latch else lib().or_escape_count_f32
    return int(fn(cr, ci, max_iter))


def mandelbrot(width, height, x0, y0, dx, dy, max_iter, threads: int = 0, rows=None):
    """Escape counts of the grid; with `rows` = (r0, r1) only those rows are
    computed (the rest of the returned array stays zero), on `threads`
    threads when threads > 0."""
    out = np.zeros((height, width), np.uint32)
    if rows is not None and threads > 0:
        lib().or_mandelbrot_rows_mt(_ptr(out), width, height, x0, y0, dx, dy, max_iter, rows[0], rows[1],
                                    threads)
    elif rows is not None:
        lib().or_mandelbrot_rows(_ptr(out), width, height, x0, y0, dx, dy, max_iter, rows[0], rows[1])
    elif threads > 0:
        lib().or_mandelbrot_mt(_ptr(out), width, height, x0, y0, dx, dy, max_iter, threads)
    else:
        lib().or_mandelbrot_rows(_ptr(out), width, height, x0, y0, dx, dy, max_iter, 0, height)
    return out


# ---- MLP ---------------------------------------------------------------------------

def mlp_step(X, y, W1, W2, lr: float, threads: int = 1):
    """Returns (loss, dW1, dW2, W1_new, W2_new); inputs are not modified."""
    X, y = _f32(X), _f32(y)
    W1n, W2n = _f32(W1).copy(), _f32(W2).copy()
    B, D = X.shape
    Hd = W1n.shape[1]
    dW1 = np.empty((D, Hd), np.float32)
    dW2 = np.empty(Hd, np.float32)
    loss = lib().or_mlp_step_f32(_ptr(X), _ptr(y), _ptr(W1n), _ptr(W2n), B, D, Hd, lr, _ptr(dW1),
                                 _ptr(dW2), threads)
    return float(loss), dW1, dW2, W1n, W2n


def mlp_grad_entries(X, y, W1, W2, k1, n1, n2, threads: int = 16):
    """Selected entries of one step's gradients, computed as mlp_step computes
    them: returns (loss, dW1[k1, n1], sum|x||d1|, dW2[n2], sum|h||d2|)."""
    X, y, W1, W2 = _f32(X), _f32(y), _f32(W1), _f32(W2)
    k1 = np.ascontiguousarray(k1, np.int32)
    n1 = np.ascontiguousarray(n1, np.int32)
    n2 = np.ascontiguousarray(n2, np.int32)
    B, D = X.shape
    Hd = W1.shape[1]
    dw1, abs1 = np.empty(k1.size, np.float32), np.empty(k1.size, np.float32)
    dw2, abs2 = np.empty(n2.size, np.float32), np.empty(n2.size, np.float32)
    loss = lib().or_mlp_grad_entries(_ptr(X), _ptr(y), _ptr(W1), _ptr(W2), B, D, Hd, _ptr(k1), _ptr(n1),
                                     k1.size, _ptr(dw1), _ptr(abs1), _ptr(n2), n2.size, _ptr(dw2),
                                     _ptr(abs2), threads)
    return float(loss), dw1, abs1, dw2, abs2


def mlp_loss_f64(X, y, W1, W2) -> float:
    X, y, W1, W2 = _f32(X), _f32(y), _f32(W1), _f32(W2)
    B, D = X.shape
    return float(lib().or_mlp_loss_f64(_ptr(X), _ptr(y), _ptr(W1), _ptr(W2), B, D, W1.shape[1]))


def xor_tensor_train(steps: int = 4000, lr: float = 1.0) -> np.ndarray:
    out = np.empty(4, np.float32)
    lib().or_xor_tensor_train(steps, lr, _ptr(out))
    return out


# ---- f64 forms (Tensor<f64, ...>) --------------------------------------------------

def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float64)


def matmul_f64(A, B, trans_a=False, trans_b=False, threads: int = 1) -> np.ndarray:
    A, B = _f64(A), _f64(B)
    M, K = (A.shape[1], A.shape[0]) if trans_a else A.shape
    N = B.shape[0] if trans_b else B.shape[1]
    C_ = np.empty((M, N), np.float64)
    lib().or_matmul_f64_mt(_ptr(A), _ptr(B), _ptr(C_), M, N, K, int(trans_a), int(trans_b), max(1, threads))
    return C_


def matmul_f64_rows(A, B, M, N, K, row0, row1, trans_a=False, trans_b=False) -> np.ndarray:
    """Rows [row0,row1) of the f64 product."""
    A, B = _f64(A), _f64(B)
    C_ = np.empty((M, N), np.float64)
    lib().or_matmul_f64_rows(_ptr(A), _ptr(B), _ptr(C_), M, N, K, int(trans_a), int(trans_b), row0, row1)
    return C_[row0:row1]


def _map1_64(name, a):
    a = _f64(a)
    out = np.empty_like(a)
    getattr(lib(), name)(_ptr(a), _ptr(out), a.size)
    return out


def _map2_64(name, a, b):
    a, b = _f64(a), _f64(b)
    out = np.empty_like(a)
    getattr(lib(), name)(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out


def add_f64(a, b): return _map2_64("or_add_f64", a, b)
def sub_f64(a, b): return _map2_64("or_sub_f64", a, b)
def mul_f64(a, b): return _map2_64("or_mul_f64", a, b)
def div_f64(a, b): return _map2_64("or_div_f64", a, b)
def neg_f64(a): return _map1_64("or_neg_f64", a)
def relu_f64(a): return _map1_64("or_relu_f64", a)
def sigmoid_f64(a): return _map1_64("or_sigmoid_f64", a)
def tanh_f64(a): return _map1_64("or_tanh_f64", a)
def sigmoid_bwd_f64(s, g): return _map2_64("or_sigmoid_bwd_f64", s, g)
def tanh_bwd_f64(t, g): return _map2_64("or_tanh_bwd_f64", t, g)
def relu_bwd_f64(x, g): return _map2_64("or_relu_bwd_f64", x, g)


def div_bwd_f64(a, b, g):
    a, b, g = _f64(a), _f64(b), _f64(g)
    da, db = np.empty_like(a), np.empty_like(a)
    lib().or_div_bwd_f64(_ptr(a), _ptr(b), _ptr(g), _ptr(da), _ptr(db), a.size)
    return da, db


def add_row_bias_f64(a, bias) -> np.ndarray:
    a, bias = _f64(a), _f64(bias)
    out = np.empty_like(a)
    lib().or_add_row_bias_f64(_ptr(a), _ptr(bias), _ptr(out), a.shape[0], a.shape[1])
    return out


def sum_rows_f64(g) -> np.ndarray:
    g = _f64(g)
    out = np.empty(g.shape[1], np.float64)
    lib().or_sum_rows_f64(_ptr(g), _ptr(out), g.shape[0], g.shape[1])
    return out


def index_f64(t, idx) -> float:
    t = _f64(t)
    dims, ix = _dims_idx(t.shape, idx)
    out = np.zeros(1, np.float64)
    if lib().or_index_f64(_ptr(t), _ptr(dims), dims.size, _ptr(ix), _ptr(out)) != 0:
        raise IndexError(f"index {tuple(idx)} outside shape {t.shape}")
    return float(out[0])


def index_bwd_f64(g: float, dt: np.ndarray, idx) -> None:
    assert dt.dtype == np.float64 and dt.flags["C_CONTIGUOUS"]
    dims, ix = _dims_idx(dt.shape, idx)
    if lib().or_index_bwd_f64(g, _ptr(dt), _ptr(dims), dims.size, _ptr(ix)) != 0:
        raise IndexError(f"index {tuple(idx)} outside shape {dt.shape}")


def sum_f64(v) -> float:
    v = _f64(v)
    return float(lib().or_sum_f64(_ptr(v), v.size))


def mean_f64(v) -> float:
    v = _f64(v)
    return float(lib().or_mean_f64(_ptr(v), v.size))


def max_of_f64(v) -> float:
    v = _f64(v)
    return float(lib().or_max_of_f64(_ptr(v), v.size))


def argmax_f64(v) -> int:
    v = _f64(v)
    return int(lib().or_argmax_f64(_ptr(v), v.size))
