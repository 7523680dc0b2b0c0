"""The C ABI from a C++ caller with no torch and no Python in the process
(tests/capi_driver/capi_driver.cpp, built by __graft_entry__.build()): hipMalloc'd buffers and
a hipStream of its own, multi-tensor steps (packed 4-bit / fp32 grads / nearest, 3 steps over
ragged sizes; int16 codes at 12 bits / bf16 grads / B = 64 / stochastic, 2 steps) and one
stq_fused_mdq_adamw call on int8 codes, each checked in the driver against the C oracle (codes
and block scales bit-exact, params within 1e-6), plus an argument error reported through
stq_last_error."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
DRIVER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "capi_driver", "capi_driver")


def test_cpp_caller_matches_the_oracle():
    print("case: tests/capi_driver/capi_driver (C++ caller of the C ABI)", flush=True)
    if not os.path.exists(DRIVER):
        raise RuntimeError(f"{DRIVER} is not built (python -c 'import __graft_entry__ as g; g.build()')")
    r = subprocess.run([DRIVER], capture_output=True, text=True, timeout=240)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("OK")
    assert r.stdout.count("matches the oracle") == 3 + 2 + 1
