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
                    add/sub/mul/div also take operands whose shapes broadcast
                    (an extension: the reference needs equal shapes); an
                    operand's cotangent is then summed back over the stretched
                    dimensions (cleave_hip_sum_to_shape_f32)
  sigmoid / tanh    s(1 - s) (= e^-x/(1+e^-x)^2) and 1 - t^2 (num.cleave:222-223)
  relu              x > 0 ? g : 0
  sum               every element receives the cotangent
  index             `derivative index(c, idx): index(d(c), idx)` (tensor.cleave:126)
                    -> scatter-add at idx
  add_row_bias      the bias cotangent is the column sum over the broadcast rows

A cotangent reaching a value along several paths is summed in the order the uses
were recorded.  Every computation is a libcleave_hip.so kernel; the tape itself is
host bookkeeping.

Fused where the graph allows.  A product and a sigmoid of a product are recorded
without being computed; a value is computed when something reads it.  The
subgraph z = sigmoid(X W1) w2 with w2 a column -- the hidden layer of the MLP
step -- then runs as that step's fused kernels (cleave_hip_sigmoid_hidden_fwd_f32:
the sigmoid and the partial products with w2 in the GEMM's epilogue, X W1 never
written).  In backward(), the same subgraph, when X takes no gradient and the
sigmoid and the inner product have no other use, takes one rule
(cleave_hip_sigmoid_hidden_bwd_f32: dW1 and dW2 in one pass over H, d1 formed as
the dW1 GEMM reads H) in place of the chain outer product -> sigmoid_bwd ->
product rule.  Values inside a fused subgraph receive no .grad.
"""
from __future__ import annotations

import numpy as np

import cleave_amd as ca
from cleave_amd import Tensor


class Var:
    """A device tensor on the tape, with the cotangent backward() accumulates.
    A recorded product (or sigmoid of one) holds a thunk until its tensor is
    read."""

    __slots__ = ("_tensor", "_thunk", "_shape", "grad", "parents", "rule", "requires_grad", "order", "kind")
    _counter = 0

    def __init__(self, tensor: Tensor | None, parents=(), rule=None, requires_grad: bool = False,
                 kind: str = "", thunk=None, shape=None):
        self._tensor = tensor
        self._thunk = thunk
        self._shape = tuple(tensor.shape) if tensor is not None else tuple(shape)
        self.grad: Tensor | None = None
        self.parents = tuple(parents)
        self.rule = rule  # g -> tuple of cotangents, one per parent (None to skip)
        self.requires_grad = requires_grad or any(p.requires_grad for p in self.parents)
        self.kind = kind
        Var._counter += 1
        self.order = Var._counter

    @property
    def tensor(self) -> Tensor:
        if self._tensor is None:
            self._tensor = self._thunk()
            self._thunk = None
        return self._tensor

    @property
    def pending(self) -> bool:
        return self._tensor is None

    @property
    def shape(self):
        return self._shape

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


_NP = {"f32": np.float32, "f64": np.float64}


def _broadcast_scalar(g: Tensor, shape) -> Tensor:
    """A tensor of `shape` filled with the one element of g (the rule of Sum)."""
    n = int(np.prod(shape, dtype=np.int64))
    out = ca.add_row_bias(ca.zero(ca.empty((n, 1), g.dtype)), g.view((1,)))
    return out.view(shape)


# ---- operators -----------------------------------------------------------------------

def _product_rule(a: Var, b: Var):
    def rule(g):
        ga = ca.matmul(g, b.tensor, trans_b=True) if a.requires_grad else None  # G B^T
        gb = ca.matmul(a.tensor, g, trans_a=True) if b.requires_grad else None  # A^T G
        return ga, gb

    return rule


def _aligned(t: Tensor) -> bool:
    return t.ptr % 16 == 0


def _hidden_forward(s: Var, w2: Var):
    """(X, W1) when s = sigmoid(X W1) is still unevaluated and s w2 can run as the
    fused hidden layer (f32, w2 a column of Hd), else None."""
    z = s.parents[0] if s.kind == "sigmoid" and s.pending else None
    if z is None or z.kind != "matmul" or not z.pending:
        return None
    x, w1 = z.parents
    if w2.shape != (s.shape[1], 1) or w2.tensor.dtype != "f32" or x.tensor.dtype != "f32" or \
            w1.tensor.dtype != "f32" or not _aligned(w2.tensor):
        return None
    return x, w1


def matmul(a: Var, b: Var) -> Var:
    """a @ b (MatMul::matmul), recorded; computed when read."""
    if len(a.shape) != 2 or len(b.shape) != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"matmul: shapes {a.shape} and {b.shape} do not chain")
    hidden = _hidden_forward(a, b)
    if hidden is not None:  # z = sigmoid(X W1) w2 in the fused kernels; X W1 is never written
        x, w1 = hidden
        h, z = ca.sigmoid_hidden_fwd(x.tensor, w1.tensor, b.tensor)
        a._tensor, a._thunk = h, None
        return Var(z, (a, b), _product_rule(a, b), kind="matmul")
    out_shape = (a.shape[0], b.shape[1])
    return Var(None, (a, b), _product_rule(a, b), kind="matmul",
               thunk=lambda: ca.matmul(a.tensor, b.tensor), shape=out_shape)


def _to_shape(g, shape):
    """The cotangent of a broadcast result, summed back over the dimensions
    that broadcasting stretched to reach an operand's shape."""
    return g if tuple(g.shape) == tuple(shape) else ca.sum_to_shape(g, shape)


def add(a: Var, b: Var) -> Var:
    return Var(ca.add(a.tensor, b.tensor), (a, b),
               lambda g: (_to_shape(g, a.shape) if a.requires_grad else None,
                          _to_shape(g, b.shape) if b.requires_grad else None))


def sub(a: Var, b: Var) -> Var:
    return Var(ca.sub(a.tensor, b.tensor), (a, b),
               lambda g: (_to_shape(g, a.shape) if a.requires_grad else None,
                          _to_shape(ca.neg(g), b.shape) if b.requires_grad else None))


def neg(a: Var) -> Var:
    return Var(ca.neg(a.tensor), (a,), lambda g: (ca.neg(g),))


def mul(a: Var, b: Var) -> Var:
    def rule(g):
        ga = _to_shape(ca.mul(g, b.tensor), a.shape) if a.requires_grad else None
        gb = _to_shape(ca.mul(a.tensor, g), b.shape) if b.requires_grad else None
        return ga, gb

    return Var(ca.mul(a.tensor, b.tensor), (a, b), rule)


def div(a: Var, b: Var) -> Var:
    if a.shape == b.shape:
        return Var(ca.div(a.tensor, b.tensor), (a, b), lambda g: ca.div_bwd(a.tensor, b.tensor, g))

    def rule(g):  # the quotient rule's two terms, broadcast, then summed back
        ga = _to_shape(ca.div(g, b.tensor), a.shape) if a.requires_grad else None
        gb = None
        if b.requires_grad:
            gb = _to_shape(ca.neg(ca.div(ca.mul(g, a.tensor), ca.mul(b.tensor, b.tensor))), b.shape)
        return ga, gb

    return Var(ca.div(a.tensor, b.tensor), (a, b), rule)


def sigmoid(a: Var) -> Var:
    if a.kind == "matmul" and a.pending:  # recorded; may become the fused hidden layer
        out = Var(None, (a,), None, kind="sigmoid", thunk=lambda: ca.sigmoid(a.tensor), shape=a.shape)
    else:
        out = Var(ca.sigmoid(a.tensor), (a,), None, kind="sigmoid")
    out.rule = lambda g: (ca.sigmoid_bwd(out.tensor, g),)
    return out


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
    out = ca.empty((1,), a.tensor.dtype)
    ca.reduce_sum(a.tensor, out)
    return Var(out, (a,), lambda g: (_broadcast_scalar(g, a.shape),))


def mean(a: Var) -> Var:
    """Mean (stdlib/nn/nn.cleave:135-138): sum / N, differentiated through the
    quotient rule with a constant denominator."""
    n = const(np.array([float(a.tensor.size)], _NP[a.tensor.dtype]))
    return div(sum(a), n)


def index(a: Var, idx) -> Var:
    """a[idx] (tensor.extract) as a one-element device tensor."""
    idx = tuple(int(i) for i in idx)
    val = ca.index(a.tensor, idx)
    out = ca.from_numpy(np.array([val], _NP[a.tensor.dtype]))

    def rule(g):
        ga = ca.zero(ca.empty(a.shape, a.tensor.dtype))
        ca.index_bwd(float(g.numpy()[0]), ga, idx)
        return (ga,)

    return Var(out, (a,), rule)


# ---- the backward pass -----------------------------------------------------------------

def _uses(loss: Var) -> dict[int, int]:
    """How many times each value reachable from the loss is an operand."""
    count: dict[int, int] = {}
    seen: set[int] = set()
    stack = [loss]
    while stack:
        v = stack.pop()
        if id(v) in seen:
            continue
        seen.add(id(v))
        for p in v.parents:
            count[id(p)] = count.get(id(p), 0) + 1
            stack.append(p)
    return count


def _hidden_backward(m: Var, uses: dict[int, int]):
    """For m = sigmoid(X W1) w2 whose sigmoid and inner product have no other use
    and whose X takes no gradient: (W1, w2) and the fused rule g -> (dW1, dW2)."""
    if m.kind != "matmul" or len(m.parents) != 2:
        return None
    s, w2 = m.parents
    if s.kind != "sigmoid" or uses.get(id(s)) != 1:
        return None
    z = s.parents[0]
    if z.kind != "matmul" or uses.get(id(z)) != 1:
        return None
    x, w1 = z.parents
    if x.requires_grad or w2.shape != (s.shape[1], 1):
        return None
    h = s.tensor
    if not all(t.dtype == "f32" for t in (x.tensor, w1.tensor, w2.tensor, h)) or not _aligned(w2.tensor) \
            or not _aligned(h):
        return None

    def rule(g):
        dw1 = ca.empty(w1.shape) if w1.requires_grad else None
        dw2 = ca.empty(w2.shape) if w2.requires_grad else None
        ca.sigmoid_hidden_bwd(x.tensor, h, w2.tensor, g, dw1, dw2)
        return dw1, dw2

    return (w1, w2), rule


def backward(loss: Var) -> None:
    """Accumulate d(loss)/d(v) into v.grad for every Var with requires_grad that the
    loss depends on.  loss must hold one element."""
    if loss.tensor.size != 1:
        raise ValueError(f"backward: the loss must hold one element, not {loss.shape}")
    uses = _uses(loss)
    fused: dict[int, tuple] = {}

    def edges(v: Var):
        if id(v) not in fused:
            fused[id(v)] = _hidden_backward(v, uses) or (v.parents, v.rule)
        return fused[id(v)]

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
        for p in edges(v)[0]:
            stack.append((p, False))
    loss.grad = ca.from_numpy(np.ones(loss.shape, _NP[loss.tensor.dtype]))
    for v in reversed(order):
        parents, rule = edges(v)
        if rule is None or v.grad is None:
            continue
        for p, gp in zip(parents, rule(v.grad)):
            if gp is None or not p.requires_grad:
                continue
            if gp.shape != p.shape:
                gp = gp.view(p.shape)
            p.grad = gp if p.grad is None else ca.add(p.grad, gp)
