"""Stochastic rounding on the device: unbiased, two-valued, and the code histogram it implies.

Independent of the oracle.  Each 128-element block holds three gradient values: one element of the
largest magnitude a (it sets the block's |m| maximum and v maximum), one of the smallest b (it sets
the v minimum) and 126 equal elements c between them.  With beta1 = 0.5, beta2 = 0 and a fresh
state, one step gives m = c / 2 and v = c^2 exactly, so every middle element has the same scaled
values y_m = m / (scale_m + 1e-12) and y_v = (log(v + 1e-12) - v_min) / (scale_v + 1e-12), read
from the scales the kernel wrote.  Stochastic rounding must give floor(y) + 1 with probability
y - floor(y) and floor(y) otherwise, independently per element (Philox counters differ per
element).  Over 4096 blocks with y spread over the code range: the up-count deviates from its
expectation by less than 5 standard deviations in total and in each of 10 probability bins, every
middle code is one of the two neighbours of y, and the histogram of middle codes passes a
chi-square test against the sum of the blocks' two-point distributions.
"""
import numpy as np
import pytest
import torch

import mdq_hip

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
B, NB, MID = 128, 4096, 126


def block_grads(rng):
    a = (1e-3 * 10.0 ** rng.uniform(0.0, 1.0, NB)).astype(np.float32)
    c = (a * rng.uniform(0.05, 0.85, NB)).astype(np.float32)
    b = (c * 10.0 ** -rng.uniform(0.3, 2.0, NB)).astype(np.float32)
    sgn = np.where(rng.random(NB) < 0.5, -1.0, 1.0).astype(np.float32)
    g = np.repeat(c * sgn, B).reshape(NB, B)
    g[:, 0] = a
    g[:, 1] = b * sgn
    return g.reshape(-1).copy(), c * sgn


def check_counts(name, codes, y):
    """codes: [NB, MID] integer codes of the middle elements; y: [NB] their common scaled value."""
    fl = np.floor(y)
    p = y - fl
    clear = (p > 1e-4) & (p < 1 - 1e-4)                      # y not within rounding noise of an integer
    lo, hi = fl[:, None], fl[:, None] + 1
    two = (codes == lo) | (codes == hi)
    assert np.all(two[clear]), f"{name}: codes outside the two neighbours of y in {np.sum(~two[clear])} places"
    ups = np.sum(codes == hi, axis=1).astype(np.float64)
    exp, var = MID * p, MID * p * (1 - p)
    z = (ups[clear] - exp[clear]).sum() / np.sqrt(var[clear].sum())
    assert abs(z) < 5.0, f"{name}: total up-count off by {z:.2f} sigma"
    bins = np.minimum((p * 10).astype(int), 9)
    for k in range(10):
        sel = clear & (bins == k)
        if sel.sum() < 20:
            continue
        zk = (ups[sel] - exp[sel]).sum() / np.sqrt(var[sel].sum())
        assert abs(zk) < 5.0, f"{name}: probability bin {k}: up-count off by {zk:.2f} sigma"
    # histogram of the middle codes against the mixture of two-point distributions
    cl = clear
    vals = np.concatenate([fl[cl], fl[cl] + 1]).astype(np.int64)
    wts = np.concatenate([MID * (1 - p[cl]), MID * p[cl]])
    off = vals.min()
    expected = np.bincount(vals - off, weights=wts)
    observed = np.bincount(codes[cl].reshape(-1).astype(np.int64) - off, minlength=expected.size)
    keep = expected > 20
    chi2 = np.sum((observed[keep] - expected[keep]) ** 2 / expected[keep])
    df = max(int(keep.sum()) - 1, 1)
    assert chi2 < df + 6 * np.sqrt(2 * df), f"{name}: code histogram chi2 {chi2:.1f} over {df} dof"


@pytest.mark.parametrize("bits", [4, 8])
def test_stochastic_rounding_unbiased_two_valued_histogram(bits):
    print(f"case: stochastic rounding statistics bits={bits}", flush=True)
    rng = np.random.default_rng(31 + bits)
    g, cvals = block_grads(rng)
    n = g.size
    p = torch.zeros(n, device=DEV)
    if bits == 4:
        cm = torch.full((n,), 8, dtype=torch.uint8, device=DEV)
        cv = torch.empty(0, dtype=torch.uint8, device=DEV)
    else:
        cm = torch.zeros(n, dtype=torch.int8, device=DEV)
        cv = torch.zeros(n, dtype=torch.uint8, device=DEV)
    sm, sv = torch.zeros(NB, device=DEV), torch.zeros(NB, device=DEV)
    vm = torch.full((NB,), -20.0, device=DEV)
    tg = torch.from_numpy(g).to(DEV)
    e = mdq_hip.TensorState(p, tg, cm, cv, sm, sv, vm, 1, bits, 0.0, 0.5, 0.0, 1e-8, 0.0, 5)
    mdq_hip.multi_tensor_step([e], B, rounding="stochastic", seed=2024)
    torch.cuda.synchronize()
    if bits == 4:
        byte = cm.cpu().numpy().reshape(NB, B)
        qm = (byte & 15).astype(np.int64) - 8
        qv = (byte >> 4).astype(np.int64)
    else:
        qm = cm.cpu().numpy().reshape(NB, B).astype(np.int64)
        qv = cv.cpu().numpy().reshape(NB, B).astype(np.int64)
    s_m = sm.cpu().numpy().astype(np.float64)
    s_v = sv.cpu().numpy().astype(np.float64)
    v_min = vm.cpu().numpy().astype(np.float64)
    m_c = (np.float32(0.5) * cvals).astype(np.float64)               # exact: fma(0.5, 0, 0.5 c)
    v_c = (cvals * cvals).astype(np.float32)                          # beta2 = 0: v = (1 * c) * c
    lv_c = np.log((v_c + np.float32(1e-12)).astype(np.float64))
    y_m = m_c / (s_m + 1e-12)
    y_v = (lv_c - v_min) / (s_v + 1e-12)
    qmax = 2 ** (bits - 1)
    assert np.all(np.abs(y_m) < qmax - 1) and np.all((y_v > 0) & (y_v < 2 ** bits - 1))
    check_counts("m codes", qm[:, 2:], y_m)
    check_counts("v codes", qv[:, 2:], y_v)
