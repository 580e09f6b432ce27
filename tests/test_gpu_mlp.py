"""MLP training step (examples/xor_tensor.cleave:38-92 style) on the GPU.

* small shapes, on both the unfused kernel sequence and the fused GEMMs: the
  loss within rel 1e-5, every dW1 / dW2 entry within the GEMM bound of the
  oracle's, and the updated weights exactly w - lr * g;
* the reference's own end-to-end record: xor_tensor trained through the GPU
  primitives (matmul, add, sigmoid, sigmoid_bwd, A B^T / A^T B matmuls,
  sgd_update) reaches the printed predictions of doc/backlog.md:142;
* BASELINE config 4 at full size (X 65536 x 1024, W1 1024 x 4096): loss and
  gradients against an independent float64-accumulated numpy computation.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_mlp_grads_close

pytestmark = pytest.mark.gpu


def _xavier(rng, fan_in, fan_out, shape):
    lim = np.sqrt(6.0 / (fan_in + fan_out))
    return rng.uniform(-lim, lim, shape).astype(np.float32)


@pytest.mark.parametrize("B,D,Hd", [
    (64, 32, 48), (256, 64, 128), (100, 33, 70), (512, 128, 256),  # unfused kernel sequence
    (512, 256, 512), (1024, 256, 768), (2048, 512, 256),           # fused GEMM path (256-tile shapes)
])
def test_small_step_against_oracle(hip, oracle, B, D, Hd):
    rng = np.random.default_rng(B + D + Hd)
    X = rng.standard_normal((B, D)).astype(np.float32)
    y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = _xavier(rng, D, Hd, (D, Hd))
    W2 = _xavier(rng, Hd, 1, Hd)
    lr = 0.01
    loss_r, dW1_r, dW2_r, W1_r, W2_r = oracle.mlp_step(X, y, W1, W2, lr=lr, threads=16)
    x, yd, w1, w2 = (hip.from_numpy(v) for v in (X, y, W1, W2))
    dw1, dw2, loss = hip.empty((D, Hd)), hip.empty(Hd), hip.empty(1)
    hip.mlp_step(x, yd, w1, w2, lr, dw1=dw1, dw2=dw2, loss=loss)
    assert abs(loss.numpy()[0] - loss_r) <= 1e-5 * abs(loss_r)
    g1, g2 = dw1.numpy(), dw2.numpy()
    # every gradient entry within the GEMM bound of its K = B contraction
    assert_mlp_grads_close(g1, g2, dW1_r, dW2_r, X, y, W1, W2, f"B={B} D={D} Hd={Hd}")
    # the update is w - lr * g in f32 on exactly those gradients
    assert np.array_equal(w1.numpy(), W1 - np.float32(lr) * g1)
    assert np.array_equal(w2.numpy(), W2 - np.float32(lr) * g2)


def test_fused_step_zero_lr_keeps_weights_and_reports_gradients(hip, oracle):
    # the fused path reads W2 while forming d1, so W2 may only change after
    # the dW1 product; with lr = 0 both weights stay bit-identical
    rng = np.random.default_rng(11)
    B, D, Hd = 512, 256, 512
    X = rng.standard_normal((B, D)).astype(np.float32)
    y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = _xavier(rng, D, Hd, (D, Hd))
    W2 = _xavier(rng, Hd, 1, Hd)
    x, yd, w1, w2 = (hip.from_numpy(v) for v in (X, y, W1, W2))
    dw1, dw2 = hip.empty((D, Hd)), hip.empty(Hd)
    hip.mlp_step(x, yd, w1, w2, 0.0, dw1=dw1, dw2=dw2)
    assert np.array_equal(w1.numpy(), W1) and np.array_equal(w2.numpy(), W2)
    _, dW1_r, dW2_r, _, _ = oracle.mlp_step(X, y, W1, W2, lr=0.0, threads=16)
    assert_mlp_grads_close(dw1.numpy(), dw2.numpy(), dW1_r, dW2_r, X, y, W1, W2, "fused, lr 0")


def test_step_without_gradient_outputs_and_zero_lr(hip, oracle):
    rng = np.random.default_rng(3)
    B, D, Hd = 128, 16, 32
    X = rng.standard_normal((B, D)).astype(np.float32)
    y = (rng.random(B) < 0.5).astype(np.float32)
    W1 = _xavier(rng, D, Hd, (D, Hd))
    W2 = _xavier(rng, Hd, 1, Hd)
    x, yd, w1, w2 = (hip.from_numpy(v) for v in (X, y, W1, W2))
    hip.mlp_step(x, yd, w1, w2, 0.0)
    assert np.array_equal(w1.numpy(), W1) and np.array_equal(w2.numpy(), W2)


def test_xor_tensor_record_through_gpu_primitives(hip, golden):
    """examples/xor_tensor.cleave's loop (lr 1.0, 4000 per-example SGD steps,
    init :69-74), each forward/backward op a libcleave_hip.so kernel."""
    g = golden["xor_tensor"]
    xs = np.array([[0, 0], [0, 1], [1, 0], [1, 1]], np.float32)
    ys = np.array([0, 1, 1, 0], np.float32)
    W = hip.from_numpy(np.array([[0.5, 0.5], [0.5, -0.5]], np.float32))
    b1 = hip.from_numpy(np.array([[-0.2, -0.2]], np.float32))
    W2 = hip.from_numpy(np.array([[1.0], [-1.0]], np.float32))
    b2 = hip.from_numpy(np.array([[0.0]], np.float32))
    X = [hip.from_numpy(xs[i:i + 1].copy()) for i in range(4)]
    Y = [hip.from_numpy(ys[i:i + 1].reshape(1, 1).copy()) for i in range(4)]
    # preallocated intermediates
    z1, h, z2, p, e, ge, gz2, gW2, gh, gz1, gW = (hip.empty(s) for s in
                                                  [(1, 2), (1, 2), (1, 1), (1, 1), (1, 1), (1, 1), (1, 1),
                                                   (2, 1), (1, 2), (1, 2), (2, 2)])

    def forward(i):
        hip.matmul(X[i], W, out=z1)
        hip.add(z1, b1, out=z1)
        hip.sigmoid(z1, out=h)
        hip.matmul(h, W2, out=z2)
        hip.add(z2, b2, out=z2)
        hip.sigmoid(z2, out=p)

    for step in range(g["steps"]):
        i = step % 4
        forward(i)
        hip.sub(p, Y[i], out=e)
        hip.add(e, e, out=ge)                  # d(e*e) = de*e + e*de
        hip.sigmoid_bwd(p, ge, out=gz2)        # through sigmoid: s(1-s)
        hip.matmul(h, gz2, trans_a=True, out=gW2)   # dW2 = h^T gz2
        hip.matmul(gz2, W2, trans_b=True, out=gh)   # dh = gz2 W2^T
        hip.sigmoid_bwd(h, gh, out=gz1)
        hip.matmul(X[i], gz1, trans_a=True, out=gW)  # dW = x^T gz1
        hip.sgd_update(W, gW, g["lr"])
        hip.sgd_update(b1, gz1, g["lr"])
        hip.sgd_update(W2, gW2, g["lr"])
        hip.sgd_update(b2, gz2, g["lr"])
    preds = []
    for i in range(4):
        forward(i)
        preds.append(float(p.numpy()[0, 0]))
    assert np.allclose(preds, g["predictions"], atol=2e-6, rtol=0), preds


def test_config4_full_size_step_every_entry(hip, oracle):
    # BASELINE config 4 at full size, every gradient entry: the oracle's whole
    # step (or_mlp_step_f32 on 16 threads; its dW1 loop is blocked over rows
    # of dW1 but keeps every entry's m-ascending order) against the device's,
    # each of the 4M dW1 and 4096 dW2 entries within the GEMM bound of its
    # K = 65536 contraction, the loss within rel 1e-5, and both updated weights.
    B, D, Hd, lr = 65536, 1024, 4096, 0.01
    rng = np.random.default_rng(7)
    x = hip.fill_normal(hip.empty((B, D)), seed=71)
    yv = hip.fill_bernoulli(hip.empty(B), seed=72)
    W1 = _xavier(rng, D, Hd, (D, Hd))
    W2 = _xavier(rng, Hd, 1, Hd)
    w1, w2 = hip.from_numpy(W1), hip.from_numpy(W2)
    dw1, dw2, loss = hip.empty((D, Hd)), hip.empty(Hd), hip.empty(1)
    hip.mlp_step(x, yv, w1, w2, lr, dw1=dw1, dw2=dw2, loss=loss)
    X, y = x.numpy(), yv.numpy()
    L, g1, g2, W1n, W2n = oracle.mlp_step(X, y, W1, W2, lr, threads=16)
    assert abs(float(loss.numpy()[0]) - L) <= 1e-5 * L
    # the bound's scale: |X|^T |d1| and |H|^T |d2|, from an f32 forward pass
    # (ample for a tolerance's scale)
    H = 1.0 / (1.0 + np.exp(-(X @ W1)))
    yh = 1.0 / (1.0 + np.exp(-(H @ W2)))
    d2 = np.abs((2.0 / B) * (yh - y) * yh * (1.0 - yh)).astype(np.float32)
    a1 = np.abs(X).T @ (np.abs(W2)[None, :] * (H * (1.0 - H)) * d2[:, None])
    a2 = np.abs(H).T @ d2
    del H
    tol = 1e-5 * np.sqrt(B)
    got1, got2 = dw1.numpy(), dw2.numpy()
    e1 = np.abs(got1.astype(np.float64) - g1) / np.maximum(a1, 1e-30)
    e2 = np.abs(got2.astype(np.float64) - g2) / np.maximum(a2, 1e-30)
    assert e1.max() <= tol, f"dW1 normalised error {e1.max():.3e} > {tol:.3e}"
    assert e2.max() <= tol, f"dW2 normalised error {e2.max():.3e} > {tol:.3e}"
    # the SGD updates: W - lr * g in f32 on the device's gradients, within the
    # gradients' bound of the oracle's updated weights
    assert np.array_equal(w1.numpy(), W1 - np.float32(lr) * got1)
    assert np.array_equal(w2.numpy(), W2 - np.float32(lr) * got2)
    assert np.all(np.abs(w1.numpy().astype(np.float64) - W1n) <= lr * tol * a1 + 2.5e-7 * np.abs(W1n))


def test_config4_full_size_step(hip, oracle):
    # BASELINE config 4 at full size.  Loss and 2 x 384 sampled gradient
    # entries against the oracle's sequential restatement (or_mlp_grad_entries:
    # the forward pass of or_mlp_step_f32, then each sampled entry as its
    # m-ascending sum over the 65536 rows).  Gradients are GEMM outputs
    # (dW1 = X^T d1, dW2 = H^T d2, both K = 65536 contractions), so they get the
    # GEMM bound |g - g_ref| <= 1e-5 * sqrt(K) * sum_m |a_m||b_m|.
    B, D, Hd, lr = 65536, 1024, 4096, 0.01
    rng = np.random.default_rng(4)
    x = hip.fill_normal(hip.empty((B, D)), seed=41)
    yv = hip.fill_bernoulli(hip.empty(B), seed=42)
    W1 = _xavier(rng, D, Hd, (D, Hd))
    W2 = _xavier(rng, Hd, 1, Hd)
    w1, w2 = hip.from_numpy(W1), hip.from_numpy(W2)
    dw1, dw2, loss = hip.empty((D, Hd)), hip.empty(Hd), hip.empty(1)
    hip.mlp_step(x, yv, w1, w2, lr, dw1=dw1, dw2=dw2, loss=loss)
    X, y = x.numpy(), yv.numpy()
    srng = np.random.default_rng(44)
    k1 = np.concatenate([srng.integers(0, D, 376), [0, 0, D - 1, D - 1, 255, 256, 511, 512]])
    n1 = np.concatenate([srng.integers(0, Hd, 376), [0, Hd - 1, 0, Hd - 1, 255, 256, 2047, 2048]])
    n2 = np.concatenate([srng.integers(0, Hd, 380), [0, Hd - 1, 255, 256]])
    L, g1, a1, g2, a2 = oracle.mlp_grad_entries(X, y, W1, W2, k1, n1, n2, threads=16)
    assert abs(float(loss.numpy()[0]) - L) <= 1e-5 * L
    got1 = dw1.numpy()
    got2 = dw2.numpy()
    tol = 1e-5 * np.sqrt(B)
    e1 = np.abs(got1[k1, n1].astype(np.float64) - g1) / a1
    e2 = np.abs(got2[n2].astype(np.float64) - g2) / a2
    assert e1.max() <= tol, f"dW1 normalised error {e1.max():.3e} > {tol:.3e}"
    assert e2.max() <= tol, f"dW2 normalised error {e2.max():.3e} > {tol:.3e}"
    # the SGD update used exactly those gradients: w = w - lr * g, in f32
    assert np.array_equal(w1.numpy(), W1 - np.float32(lr) * got1)
    assert np.array_equal(w2.numpy(), W2 - np.float32(lr) * got2)


@pytest.mark.parametrize("B,D,Hd", [(512, 256, 512), (1024, 256, 768),   # fused kernels
                                    (300, 70, 130), (256, 64, 128)])      # separate kernels
def test_hidden_layer_forward_and_rule(hip, oracle, B, D, Hd):
    # z = sigmoid(X W1) w2 and its reverse rule, as the tape calls them
    rng = np.random.default_rng(B + 3 * D + Hd)
    X = rng.standard_normal((B, D)).astype(np.float32)
    W1 = _xavier(rng, D, Hd, (D, Hd))
    W2 = _xavier(rng, Hd, 1, Hd)
    x, w1, w2 = hip.from_numpy(X), hip.from_numpy(W1), hip.from_numpy(W2)
    h, z = hip.sigmoid_hidden_fwd(x, w1, w2)
    H, Z = h.numpy(), z.numpy().ravel()
    # H against sigmoid of the oracle's product: the GEMM bound through sigmoid' <= 1/4,
    # plus the maps' rel 1e-5
    Zr = oracle.matmul(X, W1, threads=16)
    Hr = oracle.sigmoid(Zr).astype(np.float64)
    tolH = 0.25 * 1e-5 * np.sqrt(D) * (np.abs(X).astype(np.float64) @ np.abs(W1)) + 1e-5 * np.abs(Hr)
    assert np.all(np.abs(H - Hr) <= tolH)
    # z against the float64 dot of the oracle's H, within the dot's bound plus H's
    zr = Hr @ W2.astype(np.float64)
    tolz = 1e-5 * np.sqrt(Hd) * (np.abs(Hr) @ np.abs(W2)) + tolH @ np.abs(W2)
    assert np.all(np.abs(Z - zr) <= tolz)
    # the rule, on the device's H and a cotangent g of z: every entry within the GEMM bound
    g = (rng.standard_normal(B) * 0.01).astype(np.float32)
    dw1, dw2 = hip.empty((D, Hd)), hip.empty((Hd, 1))
    hip.sigmoid_hidden_bwd(x, h, w2, hip.from_numpy(g.reshape(B, 1)), dw1, dw2)
    H64, g64 = H.astype(np.float64), g.astype(np.float64)
    d1 = g64[:, None] * W2.astype(np.float64)[None, :] * H64 * (1.0 - H64)
    dW1r, dW2r = X.astype(np.float64).T @ d1, H64.T @ g64
    a1 = np.abs(X).astype(np.float64).T @ np.abs(d1)
    a2 = np.abs(H64).T @ np.abs(g64)
    tol = 1e-5 * np.sqrt(B)
    assert np.all(np.abs(dw1.numpy() - dW1r) <= tol * a1 + 1e-6 * np.abs(dW1r))
    assert np.all(np.abs(dw2.numpy().ravel() - dW2r) <= tol * a2)
