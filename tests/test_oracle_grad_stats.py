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


# Expected (n_l, r_l, v_l) patterns of the reference on its GPU, where torch reduces in fp32:
# - a NaN grad makes every sum NaN;
# - an infinity makes the sums of squares and of |g| inf and the deviations NaN: (inf, NaN, inf);
# - squares that overflow fp32 (|g| > 1.8e19), or finite squares whose sum exceeds FLT_MAX, make
#   the fp32 sum of squares and the fp32 Welford M2 overflow: (inf, inf, inf).
# (torch on the CPU keeps its std accumulator in float64, so its r_l stays finite in the last
# two cases; the GPU tests compare the kernel against torch on the GPU.)
NONFINITE = {
    "nan": ([(5, np.nan)], "nan nan nan"),
    "inf": ([(7, np.inf)], "inf nan inf"),
    "-inf": ([(7, -np.inf)], "inf nan inf"),
    "inf and -inf": ([(3, np.inf), (9, -np.inf)], "inf nan inf"),
    "square overflows": ([(2, 3e38)], "inf inf inf"),
    "sum of squares overflows": ([(k, 1e19) for k in range(10)], "inf inf inf"),
}


@pytest.mark.parametrize("case", list(NONFINITE))
def test_nonfinite_grads_follow_the_fp32_reductions(case):
    g = (np.random.default_rng(0).standard_normal(1000) * 1e-3).astype(np.float32)
    where, pattern = NONFINITE[case]
    for i, x in where:
        g[i] = x
    got = orc.grad_stats(g)
    kinds = " ".join("nan" if np.isnan(v) else "inf" if np.isinf(v) else "fin" for v in got)
    assert kinds == pattern, (got, pattern)
    # n_l and v_l follow torch's elementwise fp32 squares on any backend
    ref = MDQAdamWSimple._compute_grad_stats(torch.from_numpy(g)).numpy()
    assert np.array_equal(np.isnan(got[[0, 2]]), np.isnan(ref[[0, 2]]))
    assert np.array_equal(np.isinf(got[[0, 2]]), np.isinf(ref[[0, 2]]))


@pytest.mark.parametrize("c_exp,n", [(20, 16), (30, 16), (23, 1000), (10, 3)])
def test_variance_is_exact_for_large_means(c_exp, n):
    """x_i = c + d i (i < n) with d the spacing of fp32 numbers at c: every x_i is exact in fp32,
    and the unbiased variance is d^2 n (n + 1) / 12 whatever c is.  A one-pass formula in float64
    loses about log10(c^2 / var) digits here (up to 13); the two-pass variance keeps them."""
    c = float(2 ** c_exp)
    d = float(np.spacing(np.float32(c)))
    x = (c + d * np.arange(n)).astype(np.float32)
    assert np.array_equal(x.astype(np.float64), c + d * np.arange(n))       # exact in fp32
    sd = math.sqrt(d * d * n * (n + 1) / 12.0)
    mean_abs = np.float32((c * n + d * n * (n - 1) / 2) / n)
    got = orc.grad_stats(x)
    assert got[1] == np.float32(np.float32(sd) / np.float32(mean_abs + np.float32(1e-12)))
