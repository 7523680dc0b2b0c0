"""The kernels' own exp/log (mdq_math.h, device build) against the oracle's
C implementation: bit-identical on every input of their domain, checked via
per-chunk digests over all 2^31 - 2^23 positive normals (log) and all 2^32
bit patterns (exp), plus an elementwise pass.  The stochastic requant's
reciprocal (mdq_rcp_rn) against IEEE division on every positive normal below 2^126; the hardware
sqrt and reciprocal of the parameter update within 1 ulp of IEEE on their normal range."""
import os
import re

import numpy as np
import pytest
import torch

import mdq_hip
from oracle import mdq_oracle as orc

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_device_math_elementwise():
    bits = np.arange(0x00800000, 0x7F800000, 4099, dtype=np.int64).astype(np.uint32)
    x = bits.view(np.float32)
    tx = torch.from_numpy(x).cuda()
    for which, fn in (("log", orc.logf), ("exp", orc.expf)):
        y = mdq_hip.device_math(which, tx).cpu().numpy()
        ref = fn(x)
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), which
    xe = np.linspace(-110, 95, 200_001, dtype=np.float32)
    ye = mdq_hip.device_math("exp", torch.from_numpy(xe).cuda()).cpu().numpy()
    assert np.array_equal(ye.view(np.uint32), orc.expf(xe).view(np.uint32))


@pytest.mark.parametrize("which,first,count", [
    ("log", 0x00800000, 0x7F800000 - 0x00800000 + 1),      # positive normals and +inf
    ("exp", 0, 1 << 31),
    ("exp", 1 << 31, (1 << 31) - 1),
    # the stochastic requant's 1 / d (hardware reciprocal + one Newton step) against the
    # oracle's IEEE division, every positive normal d below 2^126 (the kernel divides above)
    ("rcp", 0x00800000, 0x7E800000 - 0x00800000),
])
def test_device_math_exhaustive_digests(which, first, count):
    chunk = 1 << 22
    dev = mdq_hip.device_math_digests(which, first, count, chunk).cpu().numpy().view(np.uint64)
    ref = orc.math_chunk_digests(which, first, count, chunk)
    bad = np.nonzero(dev != ref)[0]
    assert bad.size == 0, f"{which}: chunks {bad[:8]} differ (first bit pattern {first + int(bad[0]) * chunk:#x})"


def kernel_constant(name):
    src = open(os.path.join(ROOT, "stream-mm2026_amd", "csrc", "mdq_kernel.h")).read()
    return float(re.search(rf"#define {name} ([0-9.e+-]+)f", src).group(1))


def test_hardware_log_error_bound_holds_for_every_float():
    """The step kernel's fast v-code path relies on |v_log_f32(x) ln 2 - log x| <= A + S |log x|
    (MDQ_LOG_APPROX_ERR, MDQ_LOG_APPROX_SLOPE in mdq_kernel.h) for every float x in
    [1e-12, FLT_MAX]; checked here exhaustively on the device (measured on gfx950: the difference
    stays below 1.8e-7 |log x|, and below 9.114e-6 in absolute terms)."""
    A, S = kernel_constant("MDQ_LOG_APPROX_ERR"), kernel_constant("MDQ_LOG_APPROX_SLOPE")
    lo = int(np.array([1e-12], np.float32).view(np.uint32)[0])
    n = 0x7f7fffff - lo + 1
    flat = mdq_hip.device_log_approx_error(lo, n)
    over = mdq_hip.device_log_approx_error(lo, n, S)
    print(f"max |log2_hw(x) ln2 - log x| = {flat:.6e}; max of that - {S:g} |log x| = {over:.6e}", flush=True)
    assert 0.0 < flat < 1e-4          # the probe sees the hardware log's error at all
    assert over <= A


def test_vcode_map_is_within_half_an_ulp():
    """mdq_vcode_map (the fast v-code path's c1 = ln 2 / dv and c0 = -vmin / dv) against fp64
    quotients: each within 2^-24 (1 + 2^-16) relative, as the path's error bound assumes
    (MDQ_VCODE_MAP_ERR), over dv from 1e-12 to 130 (powers of two included) and vmin over the
    logs of [1e-12, FLT_MAX] (zero and tiny values included)."""
    rng = np.random.default_rng(7)
    n = 1 << 21
    dv = (10.0 ** rng.uniform(-12, 2.1, n)).astype(np.float32)
    dv[:47] = 2.0 ** np.arange(-39, 8)                     # 1.8e-12 .. 128
    vmin = rng.uniform(-27.7, 88.8, n).astype(np.float32)
    vmin[200:1200] = 0.0
    vmin[1200:3200] = (np.sign(rng.standard_normal(2000)) * 10.0 ** rng.uniform(-8, 0, 2000)).astype(np.float32)
    x = np.stack([dv, vmin], 1).reshape(-1)
    y = mdq_hip.device_math("vcode_map", torch.from_numpy(x).cuda()).cpu().numpy().reshape(-1, 2)
    bound = 2.0 ** -24 * (1 + 2.0 ** -16)
    assert 2 * bound <= kernel_constant("MDQ_VCODE_MAP_ERR")
    d64 = dv.astype(np.float64)
    c1 = np.log(2.0) / d64
    rel1 = np.abs(y[:, 0] - c1) / c1
    assert rel1.max() <= bound, (rel1.max(), dv[rel1.argmax()])
    c0 = -vmin.astype(np.float64) / d64
    nz = vmin != 0
    rel0 = np.abs(y[nz, 1] - c0[nz]) / np.abs(c0[nz])
    assert rel0.max() <= bound, (rel0.max(), dv[nz][rel0.argmax()], vmin[nz][rel0.argmax()])
    assert np.all(y[~nz, 1] == 0.0)
    print(f"vcode map: max rel error c1 {rel1.max():.3e}, c0 {rel0.max():.3e} (bound {bound:.3e})", flush=True)


@pytest.mark.parametrize("which,first,count", [
    ("sqrt", 0x00800000, 0x7F800000 - 0x00800000),       # every positive normal
    ("rcp", 0x00800000, 0x7E800000 - 0x00800000),        # every positive normal below 2^126
])
def test_hardware_sqrt_and_reciprocal_within_one_ulp(which, first, count):
    """The step kernel's parameter update takes v_sqrt_f32 and v_rcp_f32 where the reference
    (and the oracle) take IEEE sqrtf and division; the parameter bar of the parity tests
    (tests/param_bar.py) is derived from each being within 1 ulp of the correctly rounded result.
    Checked on every float of the update's normal range (the device's fp64 sqrt / division
    rounded to fp32 is the correctly rounded result)."""
    ulps = mdq_hip.device_hw_ulp_error(which, first, count)
    print(f"{which}: max {ulps} ulp from the correctly rounded result over {count:,} floats", flush=True)
    assert ulps <= 1


def test_stochastic_fast_vcode_bound():
    """The stochastic requant's fast v-code path (mdq_sr_vfast, as the step kernel runs it) against
    the exact code's T = fl(fma(u, fl(1/dv), uv)), u = fl(log x - vmin), uv = (k + 1/2) 2^-16 (the
    oracle's definition, mdq_oracle.c): |Zh - (T - 1/2)| <= ep for blocks of 4- and 8-bit codes with
    log spans from 1e-5 to 40 over the logs of [1e-12, FLT_MAX], and rint(Zh) = floor(T) wherever
    Zh lies farther than ep from a half-integer.  A dropped term of the bound (or a wrong offset in
    c0h) shows as a bound overrun or a code mismatch here."""
    rng = np.random.default_rng(11)
    n = 1 << 20
    qv = np.where(rng.random(n) < 0.5, 15.0, 255.0).astype(np.float32)
    lmin = rng.uniform(-27.6, 85.0, n).astype(np.float32)
    span = (10.0 ** rng.uniform(-5, 1.6, n)).astype(np.float32)
    lmax = np.minimum(lmin + span, np.float32(88.7)).astype(np.float32)
    lsam = (lmin + (lmax - lmin) * rng.random(n)).astype(np.float64)
    x = np.exp(lsam).astype(np.float32)
    ok = np.isfinite(x) & (x >= np.float32(1e-12))
    x, qv, lmin, lmax = x[ok], qv[ok], lmin[ok], lmax[ok]
    l = orc.logf(x)                                          # the oracle's log of x
    vmin = np.minimum(lmin, l).astype(np.float32)
    lmax = np.maximum(lmax, l).astype(np.float32)
    dv = ((lmax - vmin + np.float32(1e-12)) / qv + np.float32(1e-12)).astype(np.float32)
    kv = rng.integers(0, 65536, x.size).astype(np.float32)
    tup = np.stack([x, kv, dv, vmin, lmax, qv], 1).astype(np.float32).reshape(-1)
    y = mdq_hip.device_math("sr_vfast", torch.from_numpy(tup).cuda()).cpu().numpy().reshape(-1, 6)
    zh, ep = y[:, 0].astype(np.float64), y[:, 1].astype(np.float64)
    u = (l - vmin).astype(np.float32)
    inv = (np.float32(1.0) / dv).astype(np.float32)
    uv = ((kv + np.float32(0.5)) * np.float32(1.0 / 65536.0)).astype(np.float32)
    t = (u.astype(np.float64) * inv.astype(np.float64) + uv.astype(np.float64)).astype(np.float32)
    err = np.abs(zh - (t.astype(np.float64) - 0.5))
    assert np.all(err <= ep), (err / ep).max()
    k = np.rint(zh)
    fast = np.abs(zh - k) < 0.5 - ep
    assert np.array_equal(k[fast], np.floor(t.astype(np.float64))[fast])
    small = ep < 1e-3                 # typical blocks: the fast path decides nearly every code
    print(f"sr fast v code: {x.size} samples, max err / ep {(err / ep).max():.3f}, fast-path share "
          f"{fast.mean():.5f} ({fast[small].mean():.5f} where ep < 1e-3, {small.mean():.3f} of samples)",
          flush=True)
    assert small.mean() > 0.25 and fast[small].mean() > 0.99
