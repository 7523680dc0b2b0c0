"""Pins the FP64 divide + round-half-away of stquant_kernel.cu:113,123 (oracle)
and the kernel's fp32 fma replacement (mdq_round_half_away, host build) on
random, constructed-tie and near-tie inputs, with the reciprocal perturbed by
up to 2 ulp as the device's v_rcp_f32 may be."""
import numpy as np
import pytest

import mdq_hip
from oracle import mdq_oracle as orc


def round_half_away_f64(q: np.ndarray) -> np.ndarray:
    # exact for any double: split off the integer part (exact), compare the fraction
    a = np.abs(q)
    r = np.floor(a)
    r = r + (a - r >= 0.5)
    return np.copysign(r, q)


def _oracle_vec(u, d):
    return np.array([orc.round_div(a, b) for a, b in zip(u.tolist(), d.tolist())])


def _cases(rng, n):
    # d across many binades, u/d in [0, 70000)
    d = (rng.uniform(1, 2, n) * np.exp2(rng.integers(-40, 10, n))).astype(np.float32)
    q = rng.uniform(0, 70000, n) * (rng.random(n) < 0.5) + rng.uniform(0, 20, n)
    u = (q * d.astype(np.float64)).astype(np.float32)
    return u, d


def _ties(rng, n):
    # d with 12 significant bits, u = (k + 1/2) d exact, plus both neighbours
    m = rng.integers(2048, 4096, n)
    e = rng.integers(-50, 5, n)
    d = np.ldexp(m.astype(np.float64), e - 11).astype(np.float32)
    k = rng.integers(0, 1 << 10, n)
    u = ((k + 0.5) * d.astype(np.float64)).astype(np.float32)
    assert np.array_equal(u.astype(np.float64), (k + 0.5) * d.astype(np.float64))
    up = np.nextafter(u, np.float32(np.inf))
    dn = np.nextafter(u, np.float32(0))
    return np.concatenate([u, up, dn]), np.concatenate([d, d, d])


def test_oracle_round_div_is_half_away():
    rng = np.random.default_rng(1)
    u, d = _ties(rng, 2000)
    ref = round_half_away_f64(u.astype(np.float64) / d.astype(np.float64))
    assert np.array_equal(_oracle_vec(u, d), ref)
    # half away, not half to even (reference quirk vs torch.round)
    assert orc.round_div(2.5, 1.0) == 3.0 and orc.round_div(-2.5, 1.0) == -3.0
    assert orc.round_div(0.5, 1.0) == 1.0 and orc.round_div(-0.5, 1.0) == -1.0


@pytest.mark.parametrize("inv_ulps", [-1, 0, 1])
def test_fp32_method_equals_fp64_round(inv_ulps):
    rng = np.random.default_rng(100 + inv_ulps)
    u1, d1 = _cases(rng, 400_000)
    u2, d2 = _ties(rng, 100_000)
    # u just below d/2 (the case that needs the u < d/2 guard) and around binade edges
    d3 = np.ldexp(np.ones(2000), rng.integers(-40, 5, 2000)).astype(np.float32)
    u3 = np.nextafter((d3 * np.float32(0.5)), np.float32(0))
    d4 = np.nextafter(d3 * np.float32(2), np.float32(0))
    u4 = (d4 * np.float32(0.5))
    u = np.concatenate([u1, u2, u3, u4, d3 * np.float32(0.5)])
    d = np.concatenate([d1, d2, d3, d4, d3])
    ref = round_half_away_f64(u.astype(np.float64) / d.astype(np.float64))
    got = mdq_hip.host_round_half_away(u, d, inv_ulps)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first u={u[bad[0]]!r} d={d[bad[0]]!r}"


def test_fp32_method_small_brute_force():
    # every u on a fine grid against a handful of awkward divisors
    rng = np.random.default_rng(7)
    for d in [np.float32(1.0), np.float32(0.1), np.nextafter(np.float32(2.0), np.float32(0)),
              np.float32(3.0), np.float32(1.1754944e-12), np.float32(1e-12) + np.float32(1.25e-13)]:
        u = (np.arange(0, 16 * 4096) / 4096.0 * float(d)).astype(np.float32)
        u = np.concatenate([u, np.nextafter(u, np.float32(np.inf)), np.nextafter(u, np.float32(0))])
        dd = np.full_like(u, d)
        ref = round_half_away_f64(u.astype(np.float64) / dd.astype(np.float64))
        for inv in (-1, 0, 1):
            assert np.array_equal(mdq_hip.host_round_half_away(u, dd, inv), ref)


@pytest.mark.parametrize("bits", list(range(1, 33)))
def test_new_v_scale_division_is_ieee(bits):
    """s_sv = X / (2^bits - 1) (stquant_kernel.cu:102): the kernel's residual-corrected
    product must equal IEEE division.  Strided over all positive floats here; the
    same check over every positive float and every bits value passed when the
    method was adopted."""
    step = 997 if bits in (4, 8, 16, 32) else 99991
    x = np.arange(1, 0x7F800000, step, dtype=np.int64).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, np.array([np.inf, 0.0], np.float32)])   # an infinite log-v range too
    D = np.float32(2.0 ** bits - 1.0)
    got = mdq_hip.host_div_code_range(x, bits)
    assert np.array_equal(got.view(np.uint32), (x / D).astype(np.float32).view(np.uint32))
    assert np.isnan(mdq_hip.host_div_code_range(np.array([np.nan], np.float32), bits)[0])


def test_centred_uniform_minus_half_is_exact():
    """The stochastic v code's fast path rounds z + (u - 1/2) to nearest, with u on the centred
    2^-16 grid (k + 1/2) / 65536 (the oracle's uniforms, mdq_oracle.c sr_uniforms): for every
    16-bit k, k * 2^-16 + (2^-17 - 1/2) is exact in fp32 (its fma and its addend too), and adding
    1/2 back gives the uniform itself exactly."""
    k = np.arange(65536, dtype=np.float32)
    c = np.float32(2.0 ** -17 - 0.5)
    assert float(c) == 2.0 ** -17 - 0.5
    exact = k.astype(np.float64) * 2.0 ** -16 + (2.0 ** -17 - 0.5)
    uh = (k.astype(np.float64) * 2.0 ** -16 + float(c)).astype(np.float32)   # the fma, one rounding
    assert np.array_equal(uh.astype(np.float64), exact)
    u = (k * np.float32(2.0 ** -16) + np.float32(2.0 ** -17)).astype(np.float32)
    assert np.array_equal(uh + np.float32(0.5), u)
    assert np.all(np.abs(uh) < 0.5)
