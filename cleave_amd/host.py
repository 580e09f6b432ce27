"""Host-array mirror of the stdlib operators: numpy arrays in, numpy arrays out.

Every function here calls a `cleave_hip_*_host` entry point of
libcleave_hip.so, the form a `.cleave` program's `extern` call reaches: its
arrays are host memory passed as (aligned pointer, i64 length) pairs
(/root/reference/cleave/src/mlir_lower.rs:1720-1751).  The library stages them
through HBM, runs the HIP kernels and copies the results back before it
returns.  Names follow the stdlib (/root/reference/stdlib/linalg/matrix.cleave,
tensor.cleave, /root/reference/stdlib/nn/nn.cleave); device-resident work uses
the functions of the package itself instead.
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

def matmul(a: np.ndarray, b: np.ndarray, trans_a: bool = False, trans_b: bool = False) -> np.ndarray:
    """C = op(A) op(B), f32 accumulate and output.  float32 operands run the f32
    product; uint16 operands are bf16 bit patterns and run the bf16 product."""
    bf16 = np.asarray(a).dtype == np.uint16
    dt = np.uint16 if bf16 else np.float32
    a, b = _arr(a, dt), _arr(b, dt)
    M, K = (a.shape[1], a.shape[0]) if trans_a else a.shape
    Kb, N = (b.shape[1], b.shape[0]) if trans_b else b.shape
    if K != Kb:
        raise ValueError(f"matmul: inner dimensions differ ({K} vs {Kb})")
    c = np.empty((M, N), np.float32)
    fn = "cleave_hip_matmul_bf16_host" if bf16 else "cleave_hip_matmul_f32_host"
    call(fn, _p(a), a.size, _p(b), b.size, _p(c), c.size, M, N, K, int(trans_a), int(trans_b))
    return c


def matmul_batched(a: np.ndarray, b: np.ndarray, trans_a: bool = False, trans_b: bool = False) -> np.ndarray:
    bf16 = np.asarray(a).dtype == np.uint16
    dt = np.uint16 if bf16 else np.float32
    a, b = _arr(a, dt), _arr(b, dt)
    batch, M, K = a.shape
    _, Kb, N = b.shape
    if trans_a:
        M, K = K, M
    if trans_b:
        Kb, N = N, Kb
    c = np.empty((batch, M, N), np.float32)
    fn = "cleave_hip_matmul_batched_bf16_host" if bf16 else "cleave_hip_matmul_batched_f32_host"
    call(fn, _p(a), a.size, _p(b), b.size, _p(c), c.size, batch, M, N, K, int(trans_a), int(trans_b))
    return c


# ---- Ring<Tensor>, Activation<Tensor>, backward maps -------------------------------------

def _map1(fn: str, x) -> np.ndarray:
    x = _arr(x, np.float32)
    out = np.empty_like(x)
    call(fn, _p(x), x.size, _p(out), out.size)
    return out


def _map2(fn: str, a, b) -> np.ndarray:
    a, b = _arr(a, np.float32), _arr(b, np.float32)
    out = np.empty_like(a)
    call(fn, _p(a), a.size, _p(b), b.size, _p(out), out.size)
    return out


def add(a, b): return _map2("cleave_hip_add_f32_host", a, b)
def sub(a, b): return _map2("cleave_hip_sub_f32_host", a, b)
def mul(a, b): return _map2("cleave_hip_mul_f32_host", a, b)
def div(a, b): return _map2("cleave_hip_div_f32_host", a, b)
def neg(a): return _map1("cleave_hip_neg_f32_host", a)
def relu(x): return _map1("cleave_hip_relu_f32_host", x)
def sigmoid(x): return _map1("cleave_hip_sigmoid_f32_host", x)
def tanh(x): return _map1("cleave_hip_tanh_f32_host", x)
def sigmoid_bwd(s, g): return _map2("cleave_hip_sigmoid_bwd_f32_host", s, g)
def tanh_bwd(t, g): return _map2("cleave_hip_tanh_bwd_f32_host", t, g)
def relu_bwd(x, g): return _map2("cleave_hip_relu_bwd_f32_host", x, g)


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

def sum(x) -> float:  # noqa: A001 - mirrors the stdlib name
    x = _arr(x, np.float32)
    return float(_scalar("cleave_hip_sum_f32_host", _p(x), x.size))


def mean(x) -> float:
    x = _arr(x, np.float32)
    return float(_scalar("cleave_hip_mean_f32_host", _p(x), x.size))


def max_of(x) -> float:
    x = _arr(x, np.float32)
    return float(_scalar("cleave_hip_max_of_f32_host", _p(x), x.size))


def argmax(x) -> int:
    x = _arr(x, np.float32)
    return int(_scalar("cleave_hip_argmax_f32_host", _p(x), x.size))


def sum_u64(x) -> int:
    x = _arr(x, np.uint32)
    return int(_scalar("cleave_hip_sum_u32_u64_host", _p(x), x.size))


def sum_i64(x) -> int:
    """Exact i64 sum of an i32 array (cleave's Sum<[i32; N], i64> binding)."""
    x = _arr(x, np.int32)
    return int(_scalar("cleave_hip_sum_i32_i64_host", _p(x), x.size))


# ---- Index<Tensor> (stdlib/linalg/tensor.cleave:113-133) ----------------------------------

def index(t: np.ndarray, idx) -> float:
    t = _arr(t, np.float32)
    dims = _arr(t.shape, np.int32)
    ix = _arr(np.atleast_1d(idx), np.int32)
    return float(_scalar("cleave_hip_index_f32_host", _p(t), t.size, _p(dims), dims.size, _p(ix), ix.size))


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
