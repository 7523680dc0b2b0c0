"""log is non-decreasing over every float in [1e-12, FLT_MAX] -- the step kernel's fast
v-code path takes the block's max / min log v as the log of its max / min v, which needs
exactly this.  Checked exhaustively on the oracle's log, which tests/test_gpu_math.py shows
bit-identical to the kernel's on every input."""
import numpy as np
import pytest

from oracle import mdq_oracle as orc


@pytest.mark.slow
def test_log_is_monotonic_on_the_v_range():
    lo = int(np.array([1e-12], np.float32).view(np.uint32)[0])
    hi = 0x7F7FFFFF
    chunk = 1 << 25
    prev = None
    for a in range(lo, hi + 1, chunk):
        b = min(a + chunk, hi + 1)
        y = orc.logf(np.arange(a, b, dtype=np.uint32).view(np.float32))
        assert np.all(y[1:] >= y[:-1]), f"decrease inside [{a:#x}, {b:#x})"
        if prev is not None:
            assert y[0] >= prev, f"decrease at {a:#x}"
        prev = y[-1]
