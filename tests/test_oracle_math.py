"""Pins the oracle's expf/logf against float64, and the library's host build of the
kernel math against the oracle, bit for bit.

The oracle's functions stand in for CUDA expf/logf (stquant_kernel.cu:75,93).
Bound: faithful rounding (< 1 ulp) everywhere the step evaluates them, checked on
every input of those ranges (mdq_oracle_max_ulp_err, against double libm) and on a
strided sample against numpy's float64 functions.
"""
import numpy as np
import pytest

import mdq_hip
from oracle import mdq_oracle as orc

POS_NORMAL_LO, POS_NORMAL_HI = 0x00800000, 0x7F800000  # bit patterns


def _ulp_err(got: np.ndarray, ref: np.ndarray) -> np.ndarray:
    # ulp of the float32 nearest to ref, measured in float64
    ref32 = np.abs(ref).astype(np.float32)
    _, e = np.frexp(ref32.astype(np.float64))
    ulp = np.ldexp(1.0, e - 24)
    ulp = np.maximum(ulp, np.ldexp(1.0, -149))
    return np.abs(got.astype(np.float64) - ref) / ulp


def _strided_bits(lo, hi, stride, offset=0):
    return np.arange(lo + offset, hi, stride, dtype=np.int64).astype(np.uint32)


@pytest.mark.parametrize("offset", [0, 1, 2])
def test_logf_faithful_over_positive_normals(offset):
    bits = _strided_bits(POS_NORMAL_LO, POS_NORMAL_HI, 3 * 61, offset * 61 + offset)
    x = bits.view(np.float32)
    got = orc.logf(x)
    err = _ulp_err(got, np.log(x.astype(np.float64)))
    assert err.max() < 1.0, f"max {err.max():.4f} ulp at x={x[err.argmax()]!r}"


def test_logf_faithful_on_every_positive_normal():
    """All 2,130,706,432 positive normal floats."""
    err = orc.max_ulp_err("log", POS_NORMAL_LO, POS_NORMAL_HI - POS_NORMAL_LO)
    print(f"logf: max {err:.4f} ulp over every positive normal float")
    assert err < 1.0


@pytest.mark.parametrize("sign", [0, 1])
def test_expf_faithful_on_every_input_in_range(sign):
    """Every float in [0, 88] (sign 0) and in [-87, 0] (sign 1): about 2.1e9 inputs each."""
    hi = int(np.float32(88.0 if sign == 0 else 87.0).view(np.uint32))
    err = orc.max_ulp_err("exp", 0x80000000 if sign else 0, hi + 1)
    print(f"expf: max {err:.4f} ulp over every input of {'[-87, 0]' if sign else '[0, 88]'}")
    assert err < 1.0


def test_logf_dense_in_step_range():
    # every float in [1e-12, 4): the arguments v + 1e-12f the step actually sees
    lo = np.float32(1e-12).view(np.uint32)
    hi = np.float32(4.0).view(np.uint32)
    bits = np.arange(lo, hi, 7, dtype=np.int64).astype(np.uint32)
    x = bits.view(np.float32)
    err = _ulp_err(orc.logf(x), np.log(x.astype(np.float64)))
    assert err.max() < 1.0


def test_logf_special_values():
    x = np.array([1.0, np.inf, np.nan, 0.0, -1.0, 1e-40], np.float32)
    y = orc.logf(x)
    assert y[0] == 0.0 and not np.signbit(y[0])          # log 1 = +0 (no -0 in the reductions)
    assert np.isposinf(y[1]) and np.isnan(y[2]) and np.isneginf(y[3]) and np.isnan(y[4])
    assert abs(float(y[5]) - np.log(1e-40)) < 1e-5        # denormal input


@pytest.mark.parametrize("sign", [0, 1])
def test_expf_faithful(sign):
    lo = 0
    hi = np.float32(87.0).view(np.uint32) if not sign else np.float32(87.0).view(np.uint32)
    bits = _strided_bits(lo, int(hi), 37, 5)
    if sign:
        bits = bits | np.uint32(0x80000000)
    x = bits.view(np.float32)
    err = _ulp_err(orc.expf(x), np.exp(x.astype(np.float64)))
    assert err.max() < 1.0, f"max {err.max():.4f} ulp at x={x[err.argmax()]!r}"


def test_expf_special_values():
    x = np.array([0.0, np.nan, 89.5, 1000.0, -104.5, -1000.0, -20.0], np.float32)
    y = orc.expf(x)
    assert y[0] == 1.0 and np.isnan(y[1]) and np.isposinf(y[2]) and np.isposinf(y[3])
    assert y[4] == 0.0 and y[5] == 0.0
    assert abs(float(y[6]) / np.exp(-20.0) - 1) < 1e-7    # the reference's initial v = e^-20


def test_host_build_of_kernel_log_matches_oracle_bitwise():
    # kernel domain: positive normals and +inf/NaN
    bits = _strided_bits(POS_NORMAL_LO, POS_NORMAL_HI, 101, 3)
    x = np.concatenate([bits.view(np.float32), np.array([np.inf, 1.0, 1e-12], np.float32)])
    a = mdq_hip.host_math("log", x)
    b = orc.logf(x)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_host_build_of_kernel_exp_matches_oracle_bitwise():
    bits = np.arange(0, 2**32, 97, dtype=np.int64).astype(np.uint32)
    x = bits.view(np.float32)
    a = mdq_hip.host_math("exp", x)
    b = orc.expf(x)
    nan = np.isnan(b)
    assert np.array_equal(np.isnan(a), nan)
    assert np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32))
