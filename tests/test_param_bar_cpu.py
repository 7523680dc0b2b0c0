"""The GPU parity tests' parameter bar (tests/param_bar.py) on planted errors: an error inside
|dp| <= 2^-20 |update| + 2^-22 |p'| passes, one just outside fails, and a parameter the oracle's
step sets to exactly 0 is reported by its absolute error, not as an infinite relative one."""
import numpy as np
import pytest

import param_bar as pb


def _case(n=4096, seed=0):
    rng = np.random.default_rng(seed)
    prev = (rng.standard_normal(n) * 0.02).astype(np.float32)
    want = (prev - rng.standard_normal(n).astype(np.float32) * 1e-3).astype(np.float32)
    return prev, want


def test_errors_inside_the_bar_pass():
    prev, want = _case()
    upd = np.abs(want.astype(np.float64) - prev)
    got = (want + 0.9 * (2.0 ** -20) * upd).astype(np.float32)      # under the update term alone
    s = pb.assert_param_bar(got, want, prev, label="inside", quiet=True)
    assert s["bar_use"] <= 1.0
    pb.RECORDS.clear()


def test_errors_outside_the_bar_fail():
    prev, want = _case(seed=1)
    upd = np.abs(want.astype(np.float64) - prev)
    bad = want.copy()
    i = int(np.argmax(upd))
    bad[i] = np.float32(want[i] + 3.0 * ((2.0 ** -20) * upd[i] + (2.0 ** -22) * abs(want[i])))
    with pytest.raises(AssertionError, match="x the bar"):
        pb.assert_param_bar(bad, want, prev, label="outside", quiet=True)
    pb.RECORDS.clear()


def test_a_zero_target_is_reported_by_its_absolute_error():
    prev = np.array([1e-3, 0.5], np.float32)
    want = np.array([0.0, 0.49], np.float32)           # the step cancels the first parameter
    got = np.array([1e-12, 0.49], np.float32)
    s = pb.param_error_stats(got, want, prev)
    assert s["zero_target"] == 1 and s["zero_target_max_abs"] == pytest.approx(1e-12, rel=1e-6)
    assert np.isfinite(s["rel_max"]) and s["rel_max"] == 0.0
    assert "p' = 0 in the oracle" in pb.format_stats(s)
    assert s["bar_use"] < 1.0                          # 1e-12 <= 2^-20 * 1e-3
