"""Host-array mirror of the stdlib operators: numpy arrays in, numpy arrays out.

Every function here calls a `cleave_hip_*_host` entry point of
libcleave_hip.so, the form a `.cleave` program's `extern` call reaches: its
arrays are host memory passed as (aligned pointer, i64 length) pairs
(/root/reference/cleave/src/mlir_lower.rs:1720-1751).  The library stages them
through HBM, runs the HIP kernels and copies the results back before it
returns.  Names follow the stdlib (/root/reference/stdlib/linalg/matrix.cleave,
tensor.cleave, /root/reference/stdlib/nn/nn.cleave); device-resident work uses
the functions of the package itself instead.  float64 arrays take the f64
entry points (Tensor<f64, ...>); other float arrays are converted to f32.
"""
from __future__ import annotations

import numpy as np

from . import _lib
from ._lib import CleaveHipError, call, load


def _arr(x, dtype) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=dtype)


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _scalar(fn: str, *args):
    out = getattr(load(), fn)(*args)
    code, msg = _lib.last_error()
    if code < 0:
        raise CleaveHipError(code, msg)
    return out


# ---- MatMul (stdlib/linalg/matrix.cleave:22-61) --------------------------------------

def _kind(a) -> str:
    """Operand element type: bf16 bit patterns (uint16), f64 (float64), else f32."""
    dt = np.asarray(a).dtype
    return "bf16" if dt == np.uint16 else ("f64" if dt == np.float64 else "f32")


_NP = {"f32": np.float32, "f64": np.float64, "bf16": np.uint16}


def matmul(a: np.ndarray, b: np.ndarray, trans_a: bool = False, trans_b: bool = False) -> np.ndarray:
    """C = op(A) op(B).  float32 operands run the f32 product, uint16 operands
    (bf16 bit patterns) the bf16 one, both with an f32 result; float64
    operands run the f64 product."""
    kind = _kind(a)
    a, b = _arr(a, _NP[kind]), _arr(b, _NP[kind])
    M, K = (a.shape[1], a.shape[0]) if trans_a else a.shape
    Kb, N = (b.shape[1], b.shape[0]) if trans_b else b.shape
    if K != Kb:
        raise ValueError(f"matmul: inner dimensions differ ({K} vs {Kb})")
    c = np.empty((M, N), np.float64 if kind == "f64" else np.float32)
    call(f"cleave_hip_matmul_{kind}_host", _p(a), a.size, _p(b), b.size, _p(c), c.size, M, N, K, int(trans_a),
         int(trans_b))
    return c


def matmul_batched(a: np.ndarray, b: np.ndarray, trans_a: bool = False, trans_b: bool = False) -> np.ndarray:
    kind = _kind(a)
    a, b = _arr(a, _NP[kind]), _arr(b, _NP[kind])
    batch, M, K = a.shape
    _, Kb, N = b.shape
    if trans_a:
        M, K = K, M
    if trans_b:
        Kb, N = N, Kb
    c = np.empty((batch, M, N), np.float64 if kind == "f64" else np.float32)
    call(f"cleave_hip_matmul_batched_{kind}_host", _p(a), a.size, _p(b), b.size, _p(c), c.size, batch, M, N, K,
         int(trans_a), int(trans_b))
    return c


# ---- Ring<Tensor>, Activation<Tensor>, backward maps -------------------------------------

def _fkind(a) -> str:
    """f64 for float64 arrays, f32 for everything else (converted)."""
    return "f64" if np.asarray(a).dtype == np.float64 else "f32"


def _map1(op: str, x) -> np.ndarray:
    kind = _fkind(x)
    x = _arr(x, _NP[kind])
    out = np.empty_like(x)
    call(f"cleave_hip_{op}_{kind}_host", _p(x), x.size, _p(out), out.size)
    return out


def _map2(op: str, a, b) -> np.ndarray:
    kind = _fkind(a)
    a, b = _arr(a, _NP[kind]), _arr(b, _NP[kind])
    out = np.empty_like(a)
    call(f"cleave_hip_{op}_{kind}_host", _p(a), a.size, _p(b), b.size, _p(out), out.size)
    return out


def add(a, b): return _map2("add", a, b)
def sub(a, b): return _map2("sub", a, b)
def mul(a, b): return _map2("mul", a, b)
def div(a, b): return _map2("div", a, b)
def neg(a): return _map1("neg", a)
def relu(x): return _map1("relu", x)
def sigmoid(x): return _map1("sigmoid", x)
def tanh(x): return _map1("tanh", x)
def sigmoid_bwd(s, g): return _map2("sigmoid_bwd", s, g)
def tanh_bwd(t, g): return _map2("tanh_bwd", t, g)
def relu_bwd(x, g): return _map2("relu_bwd", x, g)


def zero(shape) -> np.ndarray:
    out = np.empty(shape, np.float32)
    call("cleave_hip_zero_f32_host", _p(out), out.size)
    return out


def div_bwd(a, b, g) -> tuple[np.ndarray, np.ndarray]:
    a, b, g = (_arr(v, np.float32) for v in (a, b, g))
    da, db = np.empty_like(a), np.empty_like(a)
    call("cleave_hip_div_bwd_f32_host", _p(a), a.size, _p(b), b.size, _p(g), g.size, _p(da), da.size,
         _p(db), db.size)
    return da, db


def sgd_update(w: np.ndarray, g, lr: float) -> np.ndarray:
    """w -= lr * g, in place (w must be a C-contiguous float32 array)."""
    if w.dtype != np.float32 or not w.flags["C_CONTIGUOUS"]:
        raise TypeError("sgd_update: w must be a C-contiguous float32 array (updated in place)")
    g = _arr(g, np.float32)
    call("cleave_hip_sgd_update_f32_host", _p(w), w.size, _p(g), g.size, float(lr))
    return w


def add_row_bias(a, bias) -> np.ndarray:
    a, bias = _arr(a, np.float32), _arr(bias, np.float32)
    rows, cols = a.shape
    out = np.empty_like(a)
    call("cleave_hip_add_row_bias_f32_host", _p(a), a.size, _p(bias), bias.size, _p(out), out.size, rows, cols)
    return out


def sum_rows(g) -> np.ndarray:
    g = _arr(g, np.float32)
    rows, cols = g.shape
    out = np.empty(cols, np.float32)
    call("cleave_hip_sum_rows_f32_host", _p(g), g.size, _p(out), out.size, rows, cols)
    return out


# ---- Sum / Mean / Max (stdlib/nn/nn.cleave:111-149) -------------------------------------

def _reduce(op: str, x):
    kind = _fkind(x)
    x = _arr(x, _NP[kind])
    return _scalar(f"cleave_hip_{op}_{kind}_host", _p(x), x.size)


def sum(x) -> float:  # noqa: A001 - mirrors the stdlib name
    return float(_reduce("sum", x))


def mean(x) -> float:
    return float(_reduce("mean", x))


def max_of(x) -> float:
    return float(_reduce("max_of", x))


def argmax(x) -> int:
    return int(_reduce("argmax", x))


def sum_u64(x) -> int:
    x = _arr(x, np.uint32)
    return int(_scalar("cleave_hip_sum_u32_u64_host", _p(x), x.size))


def sum_i64(x) -> int:
    """Exact i64 sum of an i32 array (cleave's Sum<[i32; N], i64> binding)."""
    x = _arr(x, np.int32)
    return int(_scalar("cleave_hip_sum_i32_i64_host", _p(x), x.size))


# ---- Index<Tensor> (stdlib/linalg/tensor.cleave:113-133) ----------------------------------

def index(t: np.ndarray, idx) -> float:
    kind = _fkind(t)
    t = _arr(t, _NP[kind])
    dims = _arr(t.shape, np.int32)
    ix = _arr(np.atleast_1d(idx), np.int32)
    return float(_scalar(f"cleave_hip_index_{kind}_host", _p(t), t.size, _p(dims), dims.size, _p(ix), ix.size))


def index_bwd(g: float, dt: np.ndarray, idx) -> np.ndarray:
    """dt[idx] += g, in place (dt must be a C-contiguous float32 array)."""
    if dt.dtype != np.float32 or not dt.flags["C_CONTIGUOUS"]:
        raise TypeError("index_bwd: dt must be a C-contiguous float32 array (updated in place)")
    dims = _arr(dt.shape, np.int32)
    ix = _arr(np.atleast_1d(idx), np.int32)
    call("cleave_hip_index_bwd_f32_host", float(g), _p(dt), dt.size, _p(dims), dims.size, _p(ix), ix.size)
    return dt


# ---- escape_count map (examples/mandelbrot.cleave:14-26) ----------------------------------

def escape_counts(width: int, height: int, x0: float, y0: float, dx: float, dy: float,
                  max_iter: int) -> np.ndarray:
    out = np.empty((height, width), np.uint32)
    call("cleave_hip_mandelbrot_u32_host", _p(out), out.size, width, height, float(x0), float(y0),
         float(dx), float(dy), max_iter)
    return out


# ---- MLP step (examples/xor_tensor.cleave:38-92 style) ------------------------------------

def mlp_step(x, y, w1: np.ndarray, w2: np.ndarray, lr: float, want_grads: bool = True):
    """One SGD step on host arrays; w1 and w2 (C-contiguous float32) are updated
    in place.  Returns (loss, dW1, dW2), the gradients None unless want_grads."""
    for w in (w1, w2):
        if w.dtype != np.float32 or not w.flags["C_CONTIGUOUS"]:
            raise TypeError("mlp_step: w1 and w2 must be C-contiguous float32 arrays (updated in place)")
    x, y = _arr(x, np.float32), _arr(y, np.float32)
    B, D = x.shape
    Hd = w1.shape[1]
    dw1 = np.empty((D, Hd), np.float32) if want_grads else None
    dw2 = np.empty(Hd, np.float32) if want_grads else None
    loss = np.empty(1, np.float32)
    call("cleave_hip_mlp_step_f32_host", _p(x), x.size, _p(y), y.size, _p(w1), w1.size, _p(w2), w2.size,
         _p(dw1) if want_grads else None, dw1.size if want_grads else 0,
         _p(dw2) if want_grads else None, dw2.size if want_grads else 0, _p(loss), B, D, Hd, float(lr))
    return float(loss[0]), dw1, dw2


# ---- output-first forms (cleave's array-return identity) -----------------------------------

def into(fn: str, out: np.ndarray, *args) -> np.ndarray:
    """Calls a `cleave_hip_*_into` entry point the way cleave's extern lowering
    does (/root/reference/cleave/src/mlir_lower.rs:1062-1130): every array
    argument, `out` first, becomes (pointer, length); the C result is an i64
    (the output length, or a negative status); the value handed back is `out`
    itself, filled in place."""
    if not out.flags["C_CONTIGUOUS"]:
        raise TypeError(f"{fn}: out must be C-contiguous (written in place)")
    flat = [_p(out), out.size]
    for a in args:
        if isinstance(a, np.ndarray):
            flat += [_p(a), a.size]
        else:
            flat.append(a)
    n = getattr(load(), fn)(*flat)
    if n < 0:
        code, msg = _lib.last_error()
        raise CleaveHipError(int(n), msg)
    if n != out.size:
        raise CleaveHipError(_lib.ERR_RUNTIME, f"{fn} returned {n}, expected the output length {out.size}")
    return out
