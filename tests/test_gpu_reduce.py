"""Sum / Mean / Max / argmax and the exact u64 count sum on the GPU vs the oracle.

Sum and mean: within 1e-5 * sum|x| of the reference's left fold (the tree
order differs).  max_of / argmax: exact, including the fold's NaN and signed
zero behaviour.  u32 -> u64 sums: exact.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from helpers import view

pytestmark = pytest.mark.gpu

SIZES = [1, 2, 3, 4, 5, 17, 1000, 4096, (1 << 20) + 7, (1 << 26) + 3]


def test_golden(hip, golden):
    r = golden["reductions"]
    v = hip.from_numpy(np.array(r["v"], np.float32))
    assert hip.sum(v) == r["sum"] and hip.mean(v) == r["mean"] and hip.max_of(v) == r["max_of"]


@pytest.mark.parametrize("n", SIZES)
def test_sum_mean_max(hip, oracle, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    d = hip.from_numpy(x)
    scale = float(np.sum(np.abs(x), dtype=np.float64))
    s = hip.sum(d)
    assert abs(s - oracle.sum_f32(x)) <= 1e-5 * scale
    assert abs(s - math.fsum(x.astype(np.float64))) <= 1e-6 * scale
    assert abs(hip.mean(d) - oracle.mean_f32(x)) <= 1e-5 * scale / n
    assert hip.max_of(d) == oracle.max_of(x)
    assert hip.argmax(d) == oracle.argmax(x)


def test_max_fold_semantics(hip, oracle):
    cases = [
        [np.nan, 1.0, 2.0],            # NaN at v[0] is the answer
        [1.0, np.nan, 2.0, np.nan],    # later NaNs never win
        [-0.0, 0.0, 0.0],              # +0 > -0 is false: first zero kept
        [0.0, -0.0],
        [3.0, 7.0, 7.0, 1.0, 7.0],     # first occurrence
        [-np.inf, -np.inf],
        [1.0] + [np.nan] * 9,
        [np.nan] * 6,
    ]
    for c in cases:
        x = np.array(c, np.float32)
        d = hip.from_numpy(x)
        got, ref = hip.max_of(d), oracle.max_of(x)
        if math.isnan(ref):
            assert math.isnan(got), c
        else:
            assert np.float32(got).view(np.uint32) == np.float32(ref).view(np.uint32), c
        assert hip.argmax(d) == oracle.argmax(x), c


def test_max_at_every_position_of_a_ragged_length(hip, oracle):
    n = 1031
    for pos in [0, 1, 3, 4, 511, 1024, 1027, 1030]:
        x = np.zeros(n, np.float32)
        x[pos] = 5.0
        x[(pos + 7) % n] = 5.0  # a tie later (or earlier) in the array
        d = hip.from_numpy(x)
        assert hip.argmax(d) == oracle.argmax(x)


def test_misaligned_start(hip, oracle):
    n = 100_001
    x = np.random.default_rng(1).standard_normal(n + 1).astype(np.float32)
    d = hip.from_numpy(x)
    v = view(d, 1, n)
    assert abs(hip.sum(v) - oracle.sum_f32(x[1:])) <= 1e-5 * np.abs(x[1:]).sum()
    assert hip.argmax(v) == oracle.argmax(x[1:])


@pytest.mark.parametrize("n", [0, 1, 3, 4, 5, 1 << 20, (1 << 24) + 3])
def test_u64_sum_exact(hip, oracle, n):
    x = np.random.default_rng(n).integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    if n == 0:
        d = hip.empty(1, "u32")
        d.shape = (0,)
        assert hip.sum_u64(d) == 0
        return
    d = hip.from_numpy(x)
    assert hip.sum_u64(d) == oracle.sum_u64(x) == int(x.astype(np.uint64).sum())


def test_empty_inputs_are_rejected(hip):
    d = hip.empty(1)
    d.shape = (0,)
    with pytest.raises(hip.CleaveHipError):
        hip.sum(d)
    with pytest.raises(hip.CleaveHipError):
        hip.max_of(d)


def test_one_launch_reductions_back_to_back(hip, oracle):
    # Each reduction is one launch whose last block folds the partials and
    # resets a completion counter for the next launch.  Interleave the three
    # kinds over grids of 1 to thousands of blocks, several times, and check
    # every result: a counter left non-zero would lose a result or fold early.
    sizes = [1, (1 << 24) + 5, 3, 4096, (1 << 20) + 1, 1, (1 << 22) + 17]
    rng = np.random.default_rng(77)
    for rep in range(3):
        for n in sizes:
            x = rng.standard_normal(n).astype(np.float32)
            c = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
            d, dc = hip.from_numpy(x), hip.from_numpy(c)
            scale = float(np.sum(np.abs(x), dtype=np.float64))
            assert abs(hip.sum(d) - oracle.sum_f32(x)) <= 1e-5 * scale, (rep, n)
            assert hip.max_of(d) == oracle.max_of(x), (rep, n)
            assert hip.argmax(d) == oracle.argmax(x), (rep, n)
            assert hip.sum_u64(dc) == int(c.astype(np.uint64).sum()), (rep, n)
