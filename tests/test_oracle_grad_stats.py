"""The oracle's gradient statistics (``mdq_oracle.grad_stats``) pinned on the CPU:
against the reference's own torch expression (stquant_opt_simple.py:93-98, kept as
``MDQAdamWSimple._compute_grad_stats``) and against closed forms."""
import math

import numpy as np
import pytest
import torch

from oracle import mdq_oracle as orc
from stquant_opt_simple import MDQAdamWSimple


@pytest.mark.parametrize("n,scale,seed", [(2, 1.0, 0), (129, 1e-3, 1), (4097, 1e-3, 2), (100_003, 5e-4, 3)])
def test_matches_reference_torch_expression(n, scale, seed):
    rng = np.random.default_rng(seed)
    g = (rng.standard_t(3, n) * scale).astype(np.float32)
    ref = MDQAdamWSimple._compute_grad_stats(torch.from_numpy(g)).numpy()
    got = orc.grad_stats(g)
    # the reference reduces in fp32 (rounded squares, its own summation order)
    assert np.allclose(got, ref, rtol=2e-6, atol=0), (got, ref)


def test_closed_forms():
    # constant c over n elements: mean g^2 = c^2, std = 0 -> r = 0
    s = orc.grad_stats(np.full(1000, -0.25, np.float32))
    assert s[0] == np.float32(0.25) and s[1] == 0.0 and s[2] == np.float32(0.0625)
    # +a / -a alternating, n even: mean g^2 = a^2, mean|g| = a, std^2 = n a^2 / (n - 1)
    n, a = 1000, 0.5
    s = orc.grad_stats(np.array([a, -a] * (n // 2), np.float32))
    assert s[0] == np.float32(a) and s[2] == np.float32(a * a)
    assert s[1] == np.float32(np.float32(math.sqrt(n / (n - 1)) * a) / np.float32(a + 1e-12))
    # all zero: r = 0 / 1e-12 = 0
    assert np.array_equal(orc.grad_stats(np.zeros(7, np.float32)), np.zeros(3, np.float32))


def test_degenerate_sizes_follow_torch():
    one = orc.grad_stats(np.array([3.0], np.float32))
    ref = MDQAdamWSimple._compute_grad_stats(torch.tensor([3.0])).numpy()
    assert one[0] == ref[0] == 3.0 and one[2] == ref[2] == 9.0
    assert np.isnan(one[1]) and np.isnan(ref[1])
    assert np.all(np.isnan(orc.grad_stats(np.zeros(0, np.float32))))


NONFINITE = {
    "nan": [(5, np.nan)],
    "inf": [(7, np.inf)],
    "-inf": [(7, -np.inf)],
    "inf and -inf": [(3, np.inf), (9, -np.inf)],
    "square overflows": [(2, 3e38)],
}


@pytest.mark.parametrize("case", list(NONFINITE))
def test_nonfinite_grads_follow_torch(case):
    """NaN / +-inf grads, and a grad whose square overflows fp32, give the NaN and inf entries
    the reference's torch expression gives (a NaN grad: all NaN; an infinity: inf, NaN, inf;
    an overflowing square: inf, finite, inf)."""
    g = (np.random.default_rng(0).standard_normal(1000) * 1e-3).astype(np.float32)
    for i, x in NONFINITE[case]:
        g[i] = x
    ref = MDQAdamWSimple._compute_grad_stats(torch.from_numpy(g)).numpy()
    got = orc.grad_stats(g)
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(np.isinf(got), np.isinf(ref)), (got, ref)
    fin = np.isfinite(ref)
    assert np.allclose(got[fin], ref[fin], rtol=2e-6, atol=0), (got, ref)
