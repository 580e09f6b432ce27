"""cleave_amd -- MI355X (gfx950) backend for cleave's tensor operator surface.

The product is libcleave_hip.so and its C ABI (include/cleave_hip.h).  This
module is a thin host-side mirror of the stdlib operator names a .cleave
program calls (/root/reference/stdlib/linalg/{tensor,matrix}.cleave,
/root/reference/stdlib/nn/nn.cleave), over device-resident tensors:

    matmul(a, b)                     MatMul::matmul          matrix.cleave:27-61
    (every Float operator takes f32 tensors, or f64 ones for Tensor<f64, ...>)
    add/sub/mul/div/neg, zero        Ring<Tensor>            tensor.cleave:66-80
    relu/sigmoid/tanh                Activation<Tensor>      nn.cleave:82-95
    sum/mean/max_of                  Sum/Mean/Max            nn.cleave:111-149
    index, index_bwd                 Index + its derivative  tensor.cleave:113-133
    escape_counts                    escape_count over a grid, examples/mandelbrot.cleave:14-26
    mlp_step                         SGD step, examples/xor_tensor.cleave:38-92 style
    sigmoid_hidden_fwd / _bwd        that step's hidden layer, z = sigmoid(X W1) w2, and its rule

Errors raise CleaveHipError (the ABI returns a negative status instead of
aborting once the binding switches abort-on-error off).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import CleaveHipError, call, load

__all__ = [
    "CleaveHipError", "Tensor", "device_available", "init", "sync", "empty", "from_numpy",
    "matmul", "matmul_batched", "add", "sub", "mul", "div", "neg", "zero", "relu", "sigmoid",
    "tanh", "sigmoid_bwd", "tanh_bwd", "relu_bwd", "div_bwd", "sgd_update", "sum", "mean",
    "max_of", "argmax", "sum_u64", "index", "index_bwd", "reduce_sum", "reduce_max", "reduce_sum_u64", "escape_counts", "mlp_step", "fill_uniform", "fill_normal",
    "fill_bernoulli", "to_bf16", "Timer", "symbol_table", "sigmoid_hidden_fwd", "sigmoid_hidden_bwd",
]

_DTYPES = {"f32": (np.float32, 4), "f64": (np.float64, 8), "bf16": (np.uint16, 2), "u32": (np.uint32, 4),
           "u64": (np.uint64, 8), "i64": (np.int64, 8)}


def device_available() -> bool:
    return bool(load().cleave_hip_device_available())


def init() -> None:
    call("cleave_hip_init")


def sync() -> None:
    call("cleave_hip_sync")


def symbol_table() -> dict[str, int]:
    return _lib.symbol_table()


@dataclass
class Tensor:
    """A device buffer (opaque handle from cleave_hip_buf_alloc) with a shape."""

    ptr: int
    shape: tuple
    dtype: str
    owned: bool = True
    base: "Tensor | None" = field(default=None, repr=False, compare=False)  # keeps a view's buffer alive

    @property
    def size(self) -> int:
        n = 1
        for d in self.shape:
            n *= int(d)
        return n

    @property
    def nbytes(self) -> int:
        return self.size * _DTYPES[self.dtype][1]

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=_DTYPES[self.dtype][0])
        if out.nbytes:
            n = call("cleave_hip_download", out.ctypes.data, self.ptr, out.nbytes)
            if n != out.nbytes:
                raise CleaveHipError(n, _lib.last_error()[1])
        return out

    def upload(self, arr: np.ndarray) -> "Tensor":
        arr = np.ascontiguousarray(arr, dtype=_DTYPES[self.dtype][0])
        if arr.size != self.size:
            raise ValueError(f"upload of {arr.size} elements into a tensor of {self.size}")
        if arr.nbytes:
            n = call("cleave_hip_upload", self.ptr, arr.ctypes.data, arr.nbytes)
            if n != arr.nbytes:
                raise CleaveHipError(n, _lib.last_error()[1])
        return self

    def view(self, shape) -> "Tensor":
        """The same buffer under another shape with the same element count (no copy)."""
        shape = tuple(int(d) for d in shape)
        t = Tensor(self.ptr, shape, self.dtype, owned=False, base=self)
        if t.size != self.size:
            raise ValueError(f"view {shape} does not cover {self.size} elements")
        return t

    def sub(self, offset: int, shape) -> "Tensor":
        """The elements [offset, offset + prod(shape)) of the buffer, as a tensor of
        that shape (no copy)."""
        shape = tuple(int(d) for d in shape)
        t = Tensor(self.ptr + int(offset) * _DTYPES[self.dtype][1], shape, self.dtype, owned=False,
                   base=self)
        if offset < 0 or offset + t.size > self.size:
            raise ValueError(f"sub-tensor [{offset}, {offset + t.size}) outside {self.size} elements")
        return t

    def free(self) -> None:
        if self.owned and self.ptr:
            load().cleave_hip_buf_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def empty(shape, dtype: str = "f32") -> Tensor:
    shape = tuple(int(d) for d in (shape if isinstance(shape, (tuple, list)) else (shape,)))
    nbytes = max(1, int(np.prod(shape, dtype=np.int64)) * _DTYPES[dtype][1])
    ptr = load().cleave_hip_buf_alloc(nbytes)
    if not ptr:
        code, msg = _lib.last_error()
        raise CleaveHipError(code, msg)
    return Tensor(ptr, shape, dtype)


def from_numpy(arr: np.ndarray, dtype: str | None = None) -> Tensor:
    if dtype is None:
        dtype = {np.dtype(np.float32): "f32", np.dtype(np.float64): "f64", np.dtype(np.uint16): "bf16",
                 np.dtype(np.uint32): "u32"}[np.dtype(arr.dtype)]
    t = empty(arr.shape, dtype)
    return t.upload(arr)


def _need(t: Tensor, dtype: str, what: str) -> None:
    if t.dtype != dtype:
        raise TypeError(f"{what}: expected {dtype} tensor, got {t.dtype}")


def _float_sfx(t: Tensor, what: str) -> str:
    """The entry-point suffix of a Float tensor: f32, or f64 for Tensor<f64, ...>."""
    if t.dtype not in ("f32", "f64"):
        raise TypeError(f"{what}: expected an f32 or f64 tensor, got {t.dtype}")
    return t.dtype


# ---- MatMul (stdlib/linalg/matrix.cleave:22-61) ------------------------------

def matmul(a: Tensor, b: Tensor, trans_a: bool = False, trans_b: bool = False,
           out: Tensor | None = None) -> Tensor:
    """C = op(A) op(B): f32 or bf16 operands give an f32 product (f32
    accumulation), f64 operands an f64 one."""
    if len(a.shape) != 2 or len(b.shape) != 2:
        raise ValueError("matmul: rank-2 operands required")
    M, K = (a.shape[1], a.shape[0]) if trans_a else a.shape
    Kb, N = (b.shape[1], b.shape[0]) if trans_b else b.shape
    if K != Kb:
        raise ValueError(f"matmul: inner dimensions differ ({K} vs {Kb})")
    if a.dtype != b.dtype:
        raise TypeError("matmul: operands must share a dtype")
    out = out if out is not None else empty((M, N), "f64" if a.dtype == "f64" else "f32")
    fn = {"f32": "cleave_hip_matmul_f32", "bf16": "cleave_hip_matmul_bf16", "f64": "cleave_hip_matmul_f64"}[a.dtype]
    call(fn, a.ptr, a.size, b.ptr, b.size, out.ptr, out.size, M, N, K, int(trans_a), int(trans_b))
    return out


def matmul_batched(a: Tensor, b: Tensor, out: Tensor | None = None, trans_a: bool = False,
                   trans_b: bool = False) -> Tensor:
    """batch x op(M x K) . batch x op(K x N), with the single product's trans flags."""
    batch, M, K = a.shape
    _, Kb, N = b.shape
    if trans_a:
        M, K = K, M
    if trans_b:
        Kb, N = N, Kb
    out = out if out is not None else empty((batch, M, N), "f64" if a.dtype == "f64" else "f32")
    call(f"cleave_hip_matmul_batched_{a.dtype}", a.ptr, a.size, b.ptr, b.size, out.ptr, out.size,
         batch, M, N, K, int(trans_a), int(trans_b))
    return out


# ---- Ring<Tensor> / Activation<Tensor> ------------------------------------------

def _binary(op: str, a: Tensor, b: Tensor, out: Tensor | None) -> Tensor:
    sfx = _float_sfx(a, op)
    out = out if out is not None else empty(a.shape, sfx)
    call(f"cleave_hip_{op}_{sfx}", a.ptr, a.size, b.ptr, b.size, out.ptr, out.size)
    return out


def _unary(op: str, a: Tensor, out: Tensor | None) -> Tensor:
    sfx = _float_sfx(a, op)
    out = out if out is not None else empty(a.shape, sfx)
    call(f"cleave_hip_{op}_{sfx}", a.ptr, a.size, out.ptr, out.size)
    return out


def broadcast_shape(ashape, bshape) -> tuple:
    """numpy's broadcast of two shapes: aligned at the last dimension, missing
    leading dimensions 1, a 1 stretching to the other's; ValueError otherwise."""
    R = max(len(ashape), len(bshape))
    da = (1,) * (R - len(ashape)) + tuple(ashape)
    db = (1,) * (R - len(bshape)) + tuple(bshape)
    out = []
    for i, (x, y) in enumerate(zip(da, db)):
        if x != y and x != 1 and y != 1:
            raise ValueError(f"shapes {tuple(ashape)} and {tuple(bshape)} do not broadcast (dimension {i})")
        out.append(y if x == 1 else x)
    return tuple(out)


def _shape_i32(shape):
    arr = np.ascontiguousarray(np.array(shape, dtype=np.int32).reshape(-1))
    return arr, (arr.ctypes.data if arr.size else None)


def _ring(op: str, a: Tensor, b: Tensor, out: Tensor | None) -> Tensor:
    """Ring<Tensor> op: equal shapes take the same-shape map; broadcastable
    shapes the broadcasting map (extension: the reference needs equal shapes)."""
    if tuple(a.shape) == tuple(b.shape):
        return _binary(op, a, b, out)
    sfx = _float_sfx(a, op)
    if b.dtype != a.dtype:
        raise TypeError(f"{op}: operands must share a dtype")
    shape = broadcast_shape(a.shape, b.shape)
    out = out if out is not None else empty(shape, sfx)
    sa, pa = _shape_i32(a.shape)
    sb, pb = _shape_i32(b.shape)
    call(f"cleave_hip_{op}_bcast_{sfx}", a.ptr, a.size, pa, len(a.shape), b.ptr, b.size, pb, len(b.shape),
         out.ptr, out.size)
    return out


def add(a, b, out=None): return _ring("add", a, b, out)
def sub(a, b, out=None): return _ring("sub", a, b, out)
def mul(a, b, out=None): return _ring("mul", a, b, out)
def div(a, b, out=None): return _ring("div", a, b, out)


def sum_to_shape(g: Tensor, shape, out: Tensor | None = None) -> Tensor:
    """g summed over the dimensions that broadcasting stretched to reach g's
    shape from `shape`: the reverse rule of the broadcasting maps."""
    sfx = _float_sfx(g, "sum_to_shape")
    shape = tuple(shape)
    out = out if out is not None else empty(shape, sfx)
    sg, pg = _shape_i32(g.shape)
    so, po = _shape_i32(shape)
    call(f"cleave_hip_sum_to_shape_{sfx}", g.ptr, g.size, pg, len(g.shape), out.ptr, out.size, po, len(shape))
    return out
def neg(a, out=None): return _unary("neg", a, out)
def relu(x, out=None): return _unary("relu", x, out)
def sigmoid(x, out=None): return _unary("sigmoid", x, out)
def tanh(x, out=None): return _unary("tanh", x, out)
def sigmoid_bwd(s, g, out=None): return _binary("sigmoid_bwd", s, g, out)
def tanh_bwd(t, g, out=None): return _binary("tanh_bwd", t, g, out)
def relu_bwd(x, g, out=None): return _binary("relu_bwd", x, g, out)


def add_row_bias(a: Tensor, bias: Tensor, out: Tensor | None = None) -> Tensor:
    """out[i, j] = a[i, j] + bias[j]: a bias shared by every row of a batch."""
    rows, cols = a.shape
    sfx = _float_sfx(a, "add_row_bias")
    out = out if out is not None else empty(a.shape, sfx)
    call(f"cleave_hip_add_row_bias_{sfx}", a.ptr, a.size, bias.ptr, bias.size, out.ptr, out.size, rows, cols)
    return out


def sum_rows(g: Tensor, out: Tensor | None = None) -> Tensor:
    """out[j] = sum_i g[i, j]: the reverse rule of add_row_bias."""
    rows, cols = g.shape
    sfx = _float_sfx(g, "sum_rows")
    out = out if out is not None else empty((cols,), sfx)
    call(f"cleave_hip_sum_rows_{sfx}", g.ptr, g.size, out.ptr, out.size, rows, cols)
    return out


def zero(shape_or_tensor) -> Tensor:
    """Ring::zero (stdlib/linalg/tensor.cleave:79)."""
    t = shape_or_tensor if isinstance(shape_or_tensor, Tensor) else empty(shape_or_tensor, "f32")
    call(f"cleave_hip_zero_{_float_sfx(t, 'zero')}", t.ptr, t.size)
    return t


def div_bwd(a: Tensor, b: Tensor, g: Tensor) -> tuple[Tensor, Tensor]:
    sfx = _float_sfx(a, "div_bwd")
    da, db = empty(a.shape, sfx), empty(a.shape, sfx)
    call(f"cleave_hip_div_bwd_{sfx}", a.ptr, a.size, b.ptr, b.size, g.ptr, g.size, da.ptr, da.size,
         db.ptr, db.size)
    return da, db


def sgd_update(w: Tensor, g: Tensor, lr: float) -> Tensor:
    call(f"cleave_hip_sgd_update_{_float_sfx(w, 'sgd_update')}", w.ptr, w.size, g.ptr, g.size, float(lr))
    return w


# ---- Sum / Mean / Max ----------------------------------------------------------

def sum(t: Tensor) -> float:  # noqa: A001 - mirrors the stdlib name
    return _checked_scalar(f"cleave_hip_sum_{_float_sfx(t, 'sum')}", t)


def mean(t: Tensor) -> float:
    return _checked_scalar(f"cleave_hip_mean_{_float_sfx(t, 'mean')}", t)


def max_of(t: Tensor) -> float:
    return _checked_scalar(f"cleave_hip_max_of_{_float_sfx(t, 'max_of')}", t)


def argmax(t: Tensor) -> int:
    return int(_checked_scalar(f"cleave_hip_argmax_{_float_sfx(t, 'argmax')}", t))


def sum_u64(t: Tensor) -> int:
    _need(t, "u32", "sum_u64")
    return int(_checked_scalar("cleave_hip_sum_u32_u64", t))


def reduce_sum(t: Tensor, out: Tensor) -> Tensor:
    """Queued sum into a device scalar (no synchronisation)."""
    call(f"cleave_hip_reduce_sum_{_float_sfx(t, 'reduce_sum')}", t.ptr, t.size, out.ptr)
    return out


def reduce_max(t: Tensor, out_max: Tensor | None, out_argmax: Tensor | None) -> None:
    """Queued max_of / argmax into device scalars (no synchronisation)."""
    call(f"cleave_hip_reduce_max_{_float_sfx(t, 'reduce_max')}", t.ptr, t.size, out_max.ptr if out_max else None,
         out_argmax.ptr if out_argmax else None)


def reduce_sum_u64(t: Tensor, out: Tensor) -> Tensor:
    """Queued exact u64 sum of u32 values into a device scalar (no synchronisation)."""
    _need(t, "u32", "reduce_sum_u64")
    call("cleave_hip_reduce_sum_u32_u64", t.ptr, t.size, out.ptr)
    return out


def _checked_scalar(fn: str, t: Tensor):
    # The host-returning reductions clear the error state on entry and return
    # a NaN / sentinel on failure, so the error state tells the two apart.
    out = getattr(load(), fn)(t.ptr, t.size)
    code, msg = _lib.last_error()
    if code < 0:
        raise CleaveHipError(code, msg)
    return out


# ---- Index<Tensor> (stdlib/linalg/tensor.cleave:113-133) -------------------------

def _dims_idx(t: Tensor, idx):
    dims = np.ascontiguousarray(t.shape, dtype=np.int32)
    ix = np.ascontiguousarray(np.atleast_1d(np.asarray(idx)), dtype=np.int32)
    return dims, ix


def index(t: Tensor, idx) -> float:
    """t[idx]: one index per dimension of t, row-major (Index::index)."""
    sfx = _float_sfx(t, "index")
    dims, ix = _dims_idx(t, idx)
    v = getattr(load(), f"cleave_hip_index_{sfx}")(t.ptr, t.size, dims.ctypes.data, dims.size, ix.ctypes.data,
                                                     ix.size)
    code, msg = _lib.last_error()
    if code < 0:
        raise CleaveHipError(code, msg)
    return float(v)


def index_bwd(g: float, dt: Tensor, idx) -> Tensor:
    """Reverse mode of `derivative index(c, idx): index(d(c), idx)`: dt[idx] += g."""
    sfx = _float_sfx(dt, "index_bwd")
    dims, ix = _dims_idx(dt, idx)
    call(f"cleave_hip_index_bwd_{sfx}", float(g), dt.ptr, dt.size, dims.ctypes.data, dims.size,
         ix.ctypes.data, ix.size)
    return dt


# ---- escape_count map ----------------------------------------------------------

def escape_counts(width: int, height: int, x0: float, y0: float, dx: float, dy: float,
                  max_iter: int, out: Tensor | None = None) -> Tensor:
    out = out if out is not None else empty((height, width), "u32")
    call("cleave_hip_mandelbrot_u32", out.ptr, out.size, width, height, float(x0), float(y0),
         float(dx), float(dy), max_iter)
    return out


# ---- MLP step --------------------------------------------------------------------

def mlp_step(x: Tensor, y: Tensor, w1: Tensor, w2: Tensor, lr: float,
             dw1: Tensor | None = None, dw2: Tensor | None = None,
             loss: Tensor | None = None) -> None:
    B, D = x.shape
    Hd = w1.shape[1]
    call("cleave_hip_mlp_step_f32", x.ptr, x.size, y.ptr, y.size, w1.ptr, w1.size, w2.ptr,
         w2.size, dw1.ptr if dw1 else None, dw1.size if dw1 else 0,
         dw2.ptr if dw2 else None, dw2.size if dw2 else 0, loss.ptr if loss else None,
         B, D, Hd, float(lr))


def sigmoid_hidden_fwd(x: Tensor, w1: Tensor, w2: Tensor, h: Tensor | None = None,
                       z: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """H = sigmoid(X W1) and z = H w2 (w2 a column of Hd): the MLP step's fused
    forward kernels as one layer.  Returns (H, z)."""
    B, D = x.shape
    Hd = w1.shape[1]
    h = h if h is not None else empty((B, Hd))
    z = z if z is not None else empty((B, 1))
    call("cleave_hip_sigmoid_hidden_fwd_f32", x.ptr, x.size, w1.ptr, w1.size, w2.ptr, w2.size, h.ptr, h.size,
         z.ptr, z.size, B, D, Hd)
    return h, z


def sigmoid_hidden_bwd(x: Tensor, h: Tensor, w2: Tensor, g: Tensor, dw1: Tensor | None = None,
                       dw2: Tensor | None = None) -> None:
    """Reverse rule of z = sigmoid(X W1) w2 given H and g = dL/dz: dW1 = X^T d1 and
    dW2 = H^T g, d1 = (g w2^T) H(1 - H).  Either output may be None."""
    B, D = x.shape
    Hd = h.shape[1]
    call("cleave_hip_sigmoid_hidden_bwd_f32", x.ptr, x.size, h.ptr, h.size, w2.ptr, w2.size, g.ptr, g.size,
         dw1.ptr if dw1 else None, dw1.size if dw1 else 0, dw2.ptr if dw2 else None, dw2.size if dw2 else 0,
         B, D, Hd)


# ---- synthetic inputs ------------------------------------------------------------

def fill_uniform(t: Tensor, seed: int, lo: float = -1.0, hi: float = 1.0) -> Tensor:
    call("cleave_hip_fill_uniform_f32", t.ptr, t.size, seed, lo, hi)
    return t


def fill_normal(t: Tensor, seed: int, mean: float = 0.0, std: float = 1.0) -> Tensor:
    call("cleave_hip_fill_normal_f32", t.ptr, t.size, seed, mean, std)
    return t


def fill_bernoulli(t: Tensor, seed: int, p: float = 0.5) -> Tensor:
    call("cleave_hip_fill_bernoulli_f32", t.ptr, t.size, seed, p)
    return t


def to_bf16(t: Tensor, out: Tensor | None = None) -> Tensor:
    out = out if out is not None else empty(t.shape, "bf16")
    call("cleave_hip_cast_f32_bf16", t.ptr, t.size, out.ptr, out.size)
    return out


class Timer:
    """HIP events recorded on the library stream (the stream every kernel uses)."""

    def __init__(self):
        lib = load()
        self.e0 = lib.cleave_hip_event_create()
        self.e1 = lib.cleave_hip_event_create()
        if not self.e0 or not self.e1:
            raise CleaveHipError(*_lib.last_error())

    def start(self):
        call("cleave_hip_event_record", self.e0)

    def stop(self) -> float:
        call("cleave_hip_event_record", self.e1)
        ms = load().cleave_hip_event_elapsed_ms(self.e0, self.e1)
        if ms < 0:
            raise CleaveHipError(*_lib.last_error())
        return ms

    def __del__(self):
        try:
            lib = load()
            lib.cleave_hip_event_destroy(self.e0)
            lib.cleave_hip_event_destroy(self.e1)
        except Exception:
            pass
