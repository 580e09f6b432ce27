"""Reverse-mode differentiation of tensor programs built from the library's operators.

The reference differentiates forward-mode, once per scalar parameter, at compile time
(`derive`, /root/reference/cleave/src/egraph.rs:2298-2299).  That cannot scale to the
millions of parameters of a tensor MLP.  This module records the operators a program
applies (a tape) and walks it backwards, applying each operator's derivative rule in
reverse form with the library's backward kernels:

  matmul            add(matmul(d(a), b), matmul(a, d(b)))  (stdlib/linalg/matrix.cleave:24)
                    -> dA = G B^T, dB = A^T G
  add / sub / neg   linearity (stdlib/num/num.cleave:123-136)
  mul               product rule d(a*b) = da*b + a*db      -> dA = G*b, dB = a*G
  div               quotient rule (num.cleave:132-134)       -> cleave_hip_div_bwd_f32
  sigmoid / tanh    s(1 - s) (= e^-x/(1+e^-x)^2) and 1 - t^2 (num.cleave:222-223)
  relu              x > 0 ? g : 0
  sum               every element receives the cotangent
  index             `derivative index(c, idx): index(d(c), idx)` (tensor.cleave:126)
                    -> scatter-add at idx
  add_row_bias      the bias cotangent is the column sum over the broadcast rows

A cotangent reaching a value along several paths is summed in the order the uses
were recorded.  Every computation is a libcleave_hip.so kernel; the tape itself is
host bookkeeping.
"""
from __future__ import annotations

import numpy as np

import cleave_amd as ca
from cleave_amd import Tensor


class Var:
    """A device tensor on the tape, with the cotangent backward() accumulates."""

    __slots__ = ("tensor", "grad", "parents", "rule", "requires_grad", "order")
    _counter = 0

    def __init__(self, tensor: Tensor, parents=(), rule=None, requires_grad: bool = False):
        self.tensor = tensor
        self.grad: Tensor | None = None
        self.parents = tuple(parents)
        self.rule = rule  # g -> tuple of cotangents, one per parent (None to skip)
        self.requires_grad = requires_grad or any(p.requires_grad for p in self.parents)
        Var._counter += 1
        self.order = Var._counter

    @property
    def shape(self):
        return self.tensor.shape

    def numpy(self) -> np.ndarray:
        return self.tensor.numpy()

    def __add__(self, o): return add(self, o)
    def __sub__(self, o): return sub(self, o)
    def __mul__(self, o): return mul(self, o)
    def __truediv__(self, o): return div(self, o)
    def __neg__(self): return neg(self)
    def __matmul__(self, o): return matmul(self, o)


def param(t: Tensor | np.ndarray) -> Var:
    """A value the loss is differentiated with respect to."""
    return Var(ca.from_numpy(t) if isinstance(t, np.ndarray) else t, requires_grad=True)


def const(t: Tensor | np.ndarray) -> Var:
    """A value the loss is not differentiated with respect to (data, targets)."""
    return Var(ca.from_numpy(t) if isinstance(t, np.ndarray) else t)


def _scale(t: Tensor, c: float) -> Tensor:
    """c * t, as 0 - (-c) * t through the SGD kernel (both steps exact but the product)."""
    out = ca.zero(t.shape)
    return ca.sgd_update(out, t, -c)


def _broadcast_scalar(g: Tensor, shape) -> Tensor:
    """A tensor of `shape` filled with the one element of g (the rule of Sum)."""
    n = int(np.prod(shape, dtype=np.int64))
    out = ca.add_row_bias(ca.zero((n, 1)), g.view((1,)))
    return out.view(shape)


# ---- operators -----------------------------------------------------------------------

def matmul(a: Var, b: Var) -> Var:
    out = ca.matmul(a.tensor, b.tensor)

    def rule(g):
        ga = ca.matmul(g, b.tensor, trans_b=True) if a.requires_grad else None  # G B^T
        gb = ca.matmul(a.tensor, g, trans_a=True) if b.requires_grad else None  # A^T G
        return ga, gb

    return Var(out, (a, b), rule)


def _same_shape(a: Var, b: Var, what: str) -> None:
    if a.shape != b.shape:
        raise ValueError(f"{what}: shapes {a.shape} and {b.shape} differ (no broadcasting; see add_row_bias)")


def add(a: Var, b: Var) -> Var:
    _same_shape(a, b, "add")
    return Var(ca.add(a.tensor, b.tensor), (a, b), lambda g: (g, g))


def sub(a: Var, b: Var) -> Var:
    _same_shape(a, b, "sub")
    return Var(ca.sub(a.tensor, b.tensor), (a, b),
               lambda g: (g, ca.neg(g) if b.requires_grad else None))


def neg(a: Var) -> Var:
    return Var(ca.neg(a.tensor), (a,), lambda g: (ca.neg(g),))


def mul(a: Var, b: Var) -> Var:
    _same_shape(a, b, "mul")

    def rule(g):
        ga = ca.mul(g, b.tensor) if a.requires_grad else None
        gb = ca.mul(a.tensor, g) if b.requires_grad else None
        return ga, gb

    return Var(ca.mul(a.tensor, b.tensor), (a, b), rule)


def div(a: Var, b: Var) -> Var:
    _same_shape(a, b, "div")
    return Var(ca.div(a.tensor, b.tensor), (a, b), lambda g: ca.div_bwd(a.tensor, b.tensor, g))


def sigmoid(a: Var) -> Var:
    s = ca.sigmoid(a.tensor)
    return Var(s, (a,), lambda g: (ca.sigmoid_bwd(s, g),))


def tanh(a: Var) -> Var:
    t = ca.tanh(a.tensor)
    return Var(t, (a,), lambda g: (ca.tanh_bwd(t, g),))


def relu(a: Var) -> Var:
    return Var(ca.relu(a.tensor), (a,), lambda g: (ca.relu_bwd(a.tensor, g),))


def add_row_bias(a: Var, bias: Var) -> Var:
    if len(a.shape) != 2 or bias.tensor.size != a.shape[1]:
        raise ValueError(f"add_row_bias: a {a.shape}, bias {bias.shape}")
    return Var(ca.add_row_bias(a.tensor, bias.tensor.view((a.shape[1],))), (a, bias),
               lambda g: (g, ca.sum_rows(g).view(bias.shape) if bias.requires_grad else None))


def sum(a: Var) -> Var:  # noqa: A001 - mirrors the stdlib name
    """Sum (stdlib/nn/nn.cleave:111-117) as a one-element device tensor."""
    out = ca.empty((1,))
    ca.reduce_sum(a.tensor, out)
    return Var(out, (a,), lambda g: (_broadcast_scalar(g, a.shape),))


def mean(a: Var) -> Var:
    """Mean (stdlib/nn/nn.cleave:135-138): sum / N, differentiated through the
    quotient rule with a constant denominator."""
    n = const(np.array([float(a.tensor.size)], np.float32))
    return div(sum(a), n)


def index(a: Var, idx) -> Var:
    """a[idx] (tensor.extract) as a one-element device tensor."""
    idx = tuple(int(i) for i in idx)
    val = ca.index(a.tensor, idx)
    out = ca.from_numpy(np.array([val], np.float32))

    def rule(g):
        ga = ca.zero(a.shape)
        ca.index_bwd(float(g.numpy()[0]), ga, idx)
        return (ga,)

    return Var(out, (a,), rule)


# ---- the backward pass -----------------------------------------------------------------

def backward(loss: Var) -> None:
    """Accumulate d(loss)/d(v) into v.grad for every Var with requires_grad that the
    loss depends on.  loss must hold one element."""
    if loss.tensor.size != 1:
        raise ValueError(f"backward: the loss must hold one element, not {loss.shape}")
    order: list[Var] = []
    seen: set[int] = set()
    stack = [(loss, False)]
    while stack:  # iterative post-order over the tape
        v, done = stack.pop()
        if done:
            order.append(v)
            continue
        if id(v) in seen or not v.requires_grad:
            continue
        seen.add(id(v))
        stack.append((v, True))
        for p in v.parents:
            stack.append((p, False))
    loss.grad = ca.from_numpy(np.ones(loss.shape, np.float32))
    for v in reversed(order):
        if v.rule is None or v.grad is None:
            continue
        for p, gp in zip(v.parents, v.rule(v.grad)):
            if gp is None or not p.requires_grad:
                continue
            if gp.shape != p.shape:
                gp = gp.view(p.shape)
            p.grad = gp if p.grad is None else ca.add(p.grad, gp)
