"""Reverse-mode tape over the library's operators (cleave_amd/autograd.py), on the GPU.

Pinned three ways: every operator's rule against central differences of a float64
restatement of the same program; the tape's MLP gradients, entry by entry,
against the oracle's sequential step; and the reference's own xor_tensor training record
(doc/backlog.md:142), now reached by differentiating the forward pass instead of
hand-written backward code."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_mlp_grads_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ad(hip):
    from cleave_amd import autograd
    return autograd


def _sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def test_every_rule_against_float64_finite_differences(hip, ad):
    rng = np.random.default_rng(40)
    X = rng.standard_normal((8, 5)).astype(np.float32)
    Y = rng.uniform(0.1, 0.9, (8, 3)).astype(np.float32)
    D = rng.uniform(1.0, 2.0, (8, 3)).astype(np.float32)
    P = {"W1": rng.standard_normal((5, 6)).astype(np.float32) * 0.5,
         "b1": rng.standard_normal(6).astype(np.float32) * 0.1,
         "W2": rng.standard_normal((6, 3)).astype(np.float32) * 0.5}

    def f64(p):
        h = np.tanh(X.astype(np.float64) @ p["W1"] + p["b1"])
        r = np.maximum(h + 2.0, 0.0)                # relu on a strictly positive input
        z = _sig(r @ p["W2"])
        e = z - Y
        q = (e * e) / D - (-e) * 0.5 * e            # div, neg and mul rules
        return q.mean() + q.sum() * 0.01 + (h + 2.0)[1, 2]

    v = {k: ad.param(a) for k, a in P.items()}
    x, y, d = ad.const(X), ad.const(Y), ad.const(D)
    half = ad.const(np.full((8, 3), 0.5, np.float32))
    two = ad.const(np.full((8, 6), 2.0, np.float32))
    cent = ad.const(np.full((1,), 0.01, np.float32))
    h = ad.tanh(ad.add_row_bias(x @ v["W1"], v["b1"]))
    hp = h + two
    r = ad.relu(hp)
    z = ad.sigmoid(r @ v["W2"])
    e = z - y
    q = (e * e) / d - (-e) * half * e
    loss = ad.mean(q) + ad.sum(q) * cent + ad.index(hp, (1, 2))
    ad.backward(loss)
    assert abs(float(loss.numpy()[0]) - f64({k: a.astype(np.float64) for k, a in P.items()})) < 1e-4
    eps = 1e-3
    for k, a in P.items():
        base = {n: b.astype(np.float64) for n, b in P.items()}
        num = np.zeros(a.shape)
        for i in np.ndindex(a.shape):
            up, dn = {n: b.copy() for n, b in base.items()}, {n: b.copy() for n, b in base.items()}
            up[k][i] += eps
            dn[k][i] -= eps
            num[i] = (f64(up) - f64(dn)) / (2 * eps)
        got = v[k].grad.numpy().reshape(a.shape)
        assert np.allclose(got, num, rtol=2e-3, atol=2e-4), (k, np.abs(got - num).max())


def test_tape_gradients_against_the_oracle(hip, ad, oracle):
    # The MLP of BASELINE config 4 at 4096 x 256 x 512, differentiated by the
    # tape, against the oracle's sequential step (or_mlp_step_f32): every dW1 /
    # dW2 entry within the GEMM bound of its K = 4096 contraction.
    B, D, Hd = 4096, 256, 512
    rng = np.random.default_rng(41)
    X = rng.standard_normal((B, D)).astype(np.float32)
    Y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = rng.uniform(-0.05, 0.05, (D, Hd)).astype(np.float32)
    W2 = rng.uniform(-0.05, 0.05, Hd).astype(np.float32)
    L, dW1_r, dW2_r, _, _ = oracle.mlp_step(X, Y, W1, W2, lr=0.0, threads=16)
    w1, w2 = ad.param(W1), ad.param(W2.reshape(Hd, 1))
    yhat = ad.sigmoid(ad.sigmoid(ad.const(X) @ w1) @ w2)
    e = yhat - ad.const(Y.reshape(B, 1))
    loss = ad.mean(e * e)
    ad.backward(loss)
    assert abs(float(loss.numpy()[0]) - L) <= 1e-5 * L
    assert_mlp_grads_close(w1.grad.numpy(), w2.grad.numpy().ravel(), dW1_r, dW2_r, X, Y, W1, W2, "tape")


def test_xor_tensor_record_through_the_tape(hip, ad, golden):
    """examples/xor_tensor.cleave:38-92: forward as the reference writes it,
    `grad = derive(loss)` as a backward pass over the tape, SGD with lr 1.0."""
    g = golden["xor_tensor"]
    xs = np.array([[0, 0], [0, 1], [1, 0], [1, 1]], np.float32)
    ys = np.array([0, 1, 1, 0], np.float32)
    W = ad.param(np.array([[0.5, 0.5], [0.5, -0.5]], np.float32))
    b1 = ad.param(np.array([[-0.2, -0.2]], np.float32))
    W2 = ad.param(np.array([[1.0], [-1.0]], np.float32))
    b2 = ad.param(np.array([[0.0]], np.float32))
    X = [ad.const(xs[i:i + 1].copy()) for i in range(4)]
    Y = [ad.const(ys[i:i + 1].copy()) for i in range(4)]

    def forward(i):
        h = ad.sigmoid(X[i] @ W + b1)
        return ad.sigmoid(ad.index(h @ W2 + b2, (0, 0)))

    for step in range(g["steps"]):
        i = step % 4
        err = forward(i) - Y[i]
        for p in (W, b1, W2, b2):
            p.grad = None
        ad.backward(err * err)
        for p in (W, b1, W2, b2):
            hip.sgd_update(p.tensor, p.grad, g["lr"])
    preds = [float(forward(i).numpy()[0]) for i in range(4)]
    assert np.allclose(preds, g["predictions"], atol=2e-6, rtol=0), preds


def test_shape_errors_are_raised_before_any_kernel(hip, ad):
    # (2, 3) and (3, 2) do not broadcast (aligned at the last dimension, 3
    # against 2); the host mirror says so before launching anything
    a, b = ad.param(np.zeros((2, 3), np.float32)), ad.param(np.zeros((3, 2), np.float32))
    with pytest.raises(ValueError, match="do not broadcast"):
        ad.add(a, b)
    with pytest.raises(ValueError, match="one element"):
        ad.backward(a)


@pytest.mark.parametrize("B,D,Hd", [(1024, 256, 768), (300, 70, 130)])  # fused kernels, separate kernels
def test_tape_hidden_layer_takes_the_fused_rule(hip, ad, oracle, B, D, Hd):
    # sigmoid(X W1) w2 on the tape: X W1 is never written, the sigmoid's value is
    # the layer's H, and backward leaves the fused subgraph's inner values without
    # .grad; the gradients still meet the oracle's, entry by entry
    rng = np.random.default_rng(B + Hd)
    X = rng.standard_normal((B, D)).astype(np.float32)
    Y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = rng.uniform(-0.1, 0.1, (D, Hd)).astype(np.float32)
    W2 = rng.uniform(-0.1, 0.1, Hd).astype(np.float32)
    w1, w2 = ad.param(W1), ad.param(W2.reshape(Hd, 1))
    z1 = ad.const(X) @ w1
    s = ad.sigmoid(z1)
    z2 = s @ w2
    assert z1.pending and not s.pending and not z2.pending
    e = ad.sigmoid(z2) - ad.const(Y.reshape(B, 1))
    loss = ad.mean(e * e)
    ad.backward(loss)
    assert z1.pending and s.grad is None and z1.grad is None
    L, dW1_r, dW2_r, _, _ = oracle.mlp_step(X, Y, W1, W2, lr=0.0, threads=16)
    assert abs(float(loss.numpy()[0]) - L) <= 1e-5 * L
    assert_mlp_grads_close(w1.grad.numpy(), w2.grad.numpy().ravel(), dW1_r, dW2_r, X, Y, W1, W2, "fused tape")


def test_tape_without_the_pattern_uses_the_general_rules(hip, ad):
    # X takes a gradient here, so the hidden layer is not fused: every rule runs
    # on its own, and the inner product is computed when the backward reads it
    rng = np.random.default_rng(77)
    X = rng.standard_normal((6, 4))
    W1 = rng.standard_normal((4, 5)) * 0.5
    W2 = rng.standard_normal((5, 1)) * 0.5
    x, w1, w2 = ad.param(X.astype(np.float32)), ad.param(W1.astype(np.float32)), ad.param(W2.astype(np.float32))
    loss = ad.sum(ad.sigmoid(x @ w1) @ w2)
    ad.backward(loss)

    def f(Xv, W1v, W2v):
        return float(np.sum((1 / (1 + np.exp(-(Xv @ W1v)))) @ W2v))

    eps = 1e-3
    for P, v in ((X, x), (W1, w1), (W2, w2)):
        num = np.zeros_like(P)
        for i in np.ndindex(P.shape):
            up, dn = P.copy(), P.copy()
            up[i] += eps
            dn[i] -= eps
            args = [up if Q is P else Q for Q in (X, W1, W2)], [dn if Q is P else Q for Q in (X, W1, W2)]
            num[i] = (f(*args[0]) - f(*args[1])) / (2 * eps)
        assert np.allclose(v.grad.numpy().reshape(P.shape), num, rtol=2e-3, atol=2e-4)
