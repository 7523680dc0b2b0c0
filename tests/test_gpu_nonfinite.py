"""NaN and infinite gradients: the step kernels against the oracle, through the C ABI.

The reference reduces each block with fmaxf / fminf (stquant_kernel.cu:26-50), which skip NaN,
and converts a NaN quotient to code 0 (:113-127); tests/test_oracle_nonfinite.py pins the oracle
to that.  Here grads carry NaN, +inf and -inf elements and whole NaN blocks in the first half of
each tensor (the second half stays finite, so fast-path tiles run beside slow-path ones), over
three consecutive steps: blocks that saw an infinity decode to NaN on the next step, as in the
reference.  Codes must be bit-exact, the three scale arrays bit-exact or NaN where the oracle's
are, params NaN where the oracle's are and within the parity bar elsewhere.
"""
import numpy as np
import pytest
import torch

import mdq_hip
from oracle import mdq_oracle as orc
from test_gpu_parity import Case, assert_bits_equal, assert_params_close, resync_params

pytestmark = pytest.mark.gpu


def assert_floats_equal_or_nan(name, t, a):
    got = t.cpu().numpy()
    nan_g, nan_a = np.isnan(got), np.isnan(a)
    assert np.array_equal(nan_g, nan_a), f"{name}: NaN at {np.nonzero(nan_g != nan_a)[0][:5]} differs"
    assert np.array_equal(got[~nan_g].view(np.uint32), a[~nan_a].view(np.uint32)), f"{name} differs"


class NonfiniteCase(Case):
    def grads(self, rng):
        g = (rng.standard_normal(self.n) * 1e-3).astype(np.float32)
        half = self.n // 2
        r = rng.random(half)
        g[:half][r < 0.004] = np.nan
        g[:half][(r >= 0.004) & (r < 0.006)] = np.inf
        g[:half][(r >= 0.006) & (r < 0.008)] = -np.inf
        nb = max(1, half // self.B)
        for b in rng.choice(nb, size=max(1, nb // 20), replace=False):
            g[b * self.B:min((b + 1) * self.B, half)] = np.nan
        if self.grad_dtype == "bf16":
            tg = torch.from_numpy(g).to(torch.bfloat16)
            return tg.view(torch.int16).numpy().view(np.uint16).copy(), tg.to("cuda:0")
        return g, torch.from_numpy(g).to("cuda:0")

    def check(self, p_prev):
        torch.cuda.synchronize()
        cm, cv, sm, sv, vm = self.state
        assert_bits_equal("exp_avg", self.tcm, cm)
        if cv is not None:
            assert_bits_equal("exp_avg_sq", self.tcv, cv)
        for name, t, a in (("scale_m", self.tsm, sm), ("scale_v", self.tsv, sv), ("v_min", self.tvm, vm)):
            assert_floats_equal_or_nan(name, t, a)
        got = self.tp.cpu().numpy()
        nan_g, nan_a = np.isnan(got), np.isnan(self.p)
        assert np.array_equal(nan_g, nan_a), f"params: NaN at {np.nonzero(nan_g != nan_a)[0][:5]} differs"
        inf_a = np.isinf(self.p)
        assert np.array_equal(got[inf_a], self.p[inf_a]), "params: infinities differ"
        fin = np.isfinite(self.p)
        assert_params_close(self.tp[torch.from_numpy(fin).to(self.tp.device)], self.p[fin], p_prev[fin])
        resync_params(self.tp, self.p)


STORAGES = [(orc.STORE_P4, 4), (orc.STORE_S8, 8), (orc.STORE_S8, 5), (orc.STORE_S16, 16), (orc.STORE_S16, 12),
            (orc.STORE_S32, 32), (orc.STORE_S32, 20)]


@pytest.mark.parametrize("B", [4, 128, 1024])
@pytest.mark.parametrize("storage,bits", STORAGES)
@pytest.mark.parametrize("rounding", [orc.ROUND_NEAREST, orc.ROUND_STOCHASTIC])
def test_nonfinite_grads_match_oracle(storage, bits, B, rounding):
    gdt = "bf16" if (bits + B) % 2 else np.float32
    print(f"case: nonfinite storage={storage} bits={bits} B={B} rounding={rounding} grad={gdt}", flush=True)
    rng = np.random.default_rng(1000 * storage + 10 * bits + B + 7 * rounding)
    c = NonfiniteCase(B * 37 + 11, B, storage, rng, grad_dtype=gdt)
    for step in (1, 2, 3):
        g, tg = c.grads(rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits, rounding=rounding, seed=3, tensor_id=1)
        mdq_hip.multi_tensor_step([c.entry(tg, step, bits, tensor_id=1)], B,
                                  rounding="stochastic" if rounding else "nearest", seed=3)
        c.check(p_prev)


@pytest.mark.parametrize("storage,bits,B,rounding", [(orc.STORE_P4, 4, 128, orc.ROUND_NEAREST),
                                                     (orc.STORE_S8, 8, 64, orc.ROUND_NEAREST),
                                                     (orc.STORE_S8, 8, 256, orc.ROUND_STOCHASTIC)])
def test_nonfinite_at_one_step_then_finite(storage, bits, B, rounding):
    """A few +-inf / NaN grads at step 2 of a 2^18-element tensor, finite grads before and after:
    every block, those that held a non-finite value included, matches the oracle at every step."""
    print(f"case: non-finite at step 2 storage={storage} bits={bits} B={B} rounding={rounding}", flush=True)
    rng = np.random.default_rng(5)
    c = Case(1 << 18, B, storage, rng)
    for step in (1, 2, 3, 4):
        g = (rng.standard_normal(c.n) * 1e-3).astype(np.float32)
        if step == 2:
            idx = rng.choice(c.n, 12, replace=False)
            g[idx[:4]] = np.inf
            g[idx[4:8]] = -np.inf
            g[idx[8:]] = np.nan
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits, rounding=rounding, seed=3)
        mdq_hip.multi_tensor_step([c.entry(torch.from_numpy(g).to("cuda:0"), step, bits)], B,
                                  rounding="stochastic" if rounding else "nearest", seed=3)
        NonfiniteCase.check(c, p_prev)


def _fma32(c, s, b):
    """float32 fma(c, s, b) for |c| < 2^16: c * s and the sum are exact in float64."""
    return np.float32(np.float64(c) * np.float64(s) + np.float64(b))


def _top_scale(cmax, vmin, top):
    """The largest float32 sv with fma(cmax, sv, vmin) <= top."""
    s = np.float32((top - vmin) / cmax)
    while _fma32(cmax, s, vmin) > top:
        s = np.nextafter(s, np.float32(0))
    while _fma32(cmax, np.nextafter(s, np.float32(np.inf)), vmin) <= top:
        s = np.nextafter(s, np.float32(np.inf))
    return s


@pytest.mark.parametrize("storage,bits,B", [(orc.STORE_S8, 8, 128), (orc.STORE_S16, 16, 128), (orc.STORE_S8, 8, 64),
                                            (orc.STORE_P4, 4, 16)])
def test_exp_argument_range_edges(storage, bits, B):
    """Steps without an exp table evaluate exp(code * sv + vmin) per element, and skip the exp's
    clamps for a wave whose blocks all keep that argument inside [-104, 89].  Blocks at both ends
    of that range (vmin = -104 exactly; the largest code landing on 88 or exactly 89) and blocks
    just outside it or with negative, NaN or infinite scales, alone in a wave or beside in-range
    blocks, all match the oracle over two steps."""
    print(f"case: exp argument range edges storage={storage} bits={bits} B={B}", flush=True)
    rng = np.random.default_rng(77 + bits + B)
    lpw = {128: 4, 64: 8, 16: 32}[B]                     # quant blocks per one-wave tile
    nw = 12
    c = NonfiniteCase(B * lpw * nw, B, storage, rng)
    cm, cv, sm, sv, vm = c.state
    nb = sm.size
    cmax = {orc.STORE_P4: 15, orc.STORE_S8: 255, orc.STORE_S16: 65535}[storage]
    sm[:] = np.float32(1e-3)
    vm[:] = np.float32(-20.0)
    sv[:] = np.float32(0.05)
    if storage == orc.STORE_P4:
        cm[:] = rng.integers(0, 256, cm.size, dtype=np.uint8)
        cm[0::B] &= 0x0F                                 # v code 0 at each block's first element
        cm[B - 1::B] |= 0xF0                             # v code 15 at its last
    else:
        cm[:] = rng.integers(np.iinfo(cm.dtype).min, np.iinfo(cm.dtype).max + 1, cm.size, dtype=cm.dtype)
        cv[:] = rng.integers(0, cmax + 1, cv.size, dtype=cv.dtype)
        cv[0::B] = 0
        cv[B - 1::B] = cmax
    s88 = _top_scale(cmax, -104.0, 88.0)
    v89 = np.float32(-104.0)                             # a v_min near -104 whose top lands on 89
    while _fma32(cmax, _top_scale(cmax, v89, 89.0), v89) != np.float32(89.0):
        v89 = np.nextafter(v89, np.float32(0))
    s89 = _top_scale(cmax, v89, 89.0)
    w = lambda k: slice(k * lpw, (k + 1) * lpw)          # the blocks of wave k
    vm[w(0)], sv[w(0)] = -104.0, s88                     # in range, low end exactly -104
    vm[w(1)], sv[w(1)] = v89, s89                        # in range, top exactly 89 (exp overflows)
    vm[w(2)][1] = np.nextafter(np.float32(-104.0), np.float32(-np.inf))
    vm[w(3)][2], sv[w(3)][2] = v89, np.nextafter(s89, np.float32(np.inf))      # top just above 89
    sv[w(4)][0] = -0.01
    sv[w(5)][1] = np.nan
    vm[w(6)][2] = np.nan
    sv[w(7)][3 % lpw] = np.inf
    vm[w(8)][0], sv[w(8)][0] = -104.0, s88               # in range beside ordinary blocks
    vm[w(9)][lpw - 1], sv[w(9)][lpw - 1] = -50.0, s88
    for a, t in ((cm, c.tcm), (cv, c.tcv), (sm, c.tsm), (sv, c.tsv), (vm, c.tvm)):
        if a is not None:
            t.copy_(torch.from_numpy(a.copy()))
    assert nb == lpw * nw
    for step in (1, 2):
        g, tg = Case.grads(c, rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits)
        mdq_hip.multi_tensor_step([c.entry(tg, step, bits)], B)
        c.check(p_prev)


@pytest.mark.parametrize("rounding", [orc.ROUND_NEAREST, orc.ROUND_STOCHASTIC])
def test_huge_m_scales(rounding):
    """Blocks whose new m scale reaches 2^126 and beyond (1-bit codes dequantised with scales
    near 3e37), in the same waves as ordinary blocks: the stochastic requant's 1 / scale leaves
    its fast reciprocal, exact only below 2^126, for IEEE division there.  Two steps, against
    the oracle."""
    print(f"case: huge m scales rounding={rounding}", flush=True)
    B, bits = 128, 1
    rng = np.random.default_rng(91)
    c = NonfiniteCase(B * 4 * 6, B, orc.STORE_S8, rng)
    cm, cv, sm, sv, vm = c.state
    nb = sm.size
    cm[:] = rng.integers(-4, 5, cm.size, dtype=np.int8)
    cv[:] = rng.integers(0, 2, cv.size, dtype=np.uint8)
    sm[:] = np.float32(1e-4)
    sv[:] = np.float32(1.0)
    vm[:] = np.float32(-20.0)
    big = rng.choice(nb, nb // 3, replace=False)
    sm[big] = (10.0 ** rng.uniform(37.2, 37.6, big.size)).astype(np.float32)   # |m| up to 1.6e38
    for a, t in ((cm, c.tcm), (cv, c.tcv), (sm, c.tsm), (sv, c.tsv), (vm, c.tvm)):
        t.copy_(torch.from_numpy(a.copy()))
    for step in (1, 2):
        g, tg = Case.grads(c, rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits, rounding=rounding, seed=3)
        assert float(np.max(sm)) >= 2.0 ** 126                    # the range the guard covers
        mdq_hip.multi_tensor_step([c.entry(tg, step, bits)], B,
                                  rounding="stochastic" if rounding else "nearest", seed=3)
        c.check(p_prev)
