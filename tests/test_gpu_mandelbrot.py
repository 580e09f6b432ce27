"""Escape-time map (examples/mandelbrot.cleave:14-26) on the GPU: counts are
bit-exact against the oracle; the u64 sum of counts is exact."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

X0, Y0, SPAN = -2.0, -1.5, 3.0


def test_special_points(hip, golden):
    pts = golden["mandelbrot_example"]
    for cr, ci in pts["never_escapes"] + pts["escapes_at_0"]:
        c = hip.escape_counts(1, 1, cr, ci, 0.0, 0.0, 1000).numpy()[0, 0]
        want = 1000 if [cr, ci] in pts["never_escapes"] else 0
        assert c == want, (cr, ci)


@pytest.mark.parametrize("w,h,it", [(1, 1, 50), (70, 25, 50), (128, 96, 200), (257, 130, 1000), (1000, 333, 300)])
def test_small_grids_bit_exact(hip, oracle, w, h, it):
    dx, dy = np.float32(SPAN / w), np.float32(SPAN / h)
    got = hip.escape_counts(w, h, X0, Y0, dx, dy, it).numpy()
    ref = oracle.mandelbrot(w, h, X0, Y0, dx, dy, it, threads=16)
    assert np.array_equal(got, ref)


def test_reference_example_window(hip, oracle):
    # examples/mandelbrot.cleave:30-33: 70 x 25 over [-2.5, 1.0] x [-1.25, 1.25], 50 iterations
    # (f64 accumulation there; here the same window in f32 with c = x0 + col*dx).
    got = hip.escape_counts(70, 25, -2.5, -1.25, 0.05, 0.1, 50).numpy()
    ref = oracle.mandelbrot(70, 25, -2.5, -1.25, 0.05, 0.1, 50)
    assert np.array_equal(got, ref)
    assert got.max() == 50 and got.min() == 0


def test_config3_full_grid(hip, oracle):
    n, it = 16384, 1000
    d = np.float32(SPAN / n)
    counts = hip.escape_counts(n, n, X0, Y0, d, d, it)
    total = hip.sum_u64(counts)
    C = counts.numpy()
    assert total == int(C.sum(dtype=np.uint64))
    # every count of the grid against the oracle, bit for bit, on 16 threads
    ref = oracle.mandelbrot(n, n, X0, Y0, d, d, it, threads=16)
    bad = np.nonzero(np.any(C != ref, axis=1))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:8]}"
    assert total == int(ref.sum(dtype=np.uint64))
    # and conjugate symmetry: row r has ci = -1.5 + r*d, and rows r and n - r
    # carry opposite ci exactly (both are k*d from the centre)
    assert np.array_equal(C[1:n // 2], C[n - 1:n // 2:-1])
