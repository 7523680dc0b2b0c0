"""Long runs: 30 consecutive steps of one 2^21-element tensor against the oracle, through the C ABI.

The other parity tests start from fresh or drawn states and run one to ten steps.  Here the codes
and scales evolve over 30 steps under heavy-tailed gradients (Student-t with 3 degrees of
freedom, times a per-step factor between 0.1 and 10, so block ranges grow and shrink), which puts
many elements near code boundaries of the fast m- and v-code paths at 4 and 8 bits.  Codes and the
three scale arrays must be bit-exact after every step, params within the parity bar of
test_gpu_parity.py (each step starts from the oracle's params).
"""
import numpy as np
import pytest
import torch

import mdq_hip
from oracle import mdq_oracle as orc
from test_gpu_parity import Case

pytestmark = pytest.mark.gpu
STEPS = 30


class TailCase(Case):
    def grads(self, rng, scale):
        g = (rng.standard_t(3, self.n) * (1e-3 * scale)).astype(np.float32)
        if self.grad_dtype == "bf16":
            tg = torch.from_numpy(g).to(torch.bfloat16)
            return tg.view(torch.int16).numpy().view(np.uint16).copy(), tg.to("cuda:0")
        return g, torch.from_numpy(g).to("cuda:0")


@pytest.mark.parametrize("storage,bits,B,rounding,gdt", [
    (orc.STORE_P4, 4, 128, orc.ROUND_NEAREST, "bf16"),
    (orc.STORE_P4, 4, 128, orc.ROUND_STOCHASTIC, np.float32),
    (orc.STORE_S8, 8, 128, orc.ROUND_NEAREST, np.float32),
    (orc.STORE_S8, 8, 64, orc.ROUND_STOCHASTIC, "bf16"),
    (orc.STORE_S16, 16, 256, orc.ROUND_NEAREST, "bf16"),
])
def test_thirty_steps_heavy_tailed_grads(storage, bits, B, rounding, gdt):
    print(f"case: long run storage={storage} bits={bits} B={B} rounding={rounding} grad={gdt}", flush=True)
    rng = np.random.default_rng(900 + 10 * bits + B + rounding)
    c = TailCase(1 << 21, B, storage, rng, grad_dtype=gdt)
    for step in range(1, STEPS + 1):
        scale = float(10.0 ** rng.uniform(-1.0, 1.0))
        g, tg = c.grads(rng, scale)
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits, rounding=rounding, seed=11, tensor_id=2)
        mdq_hip.multi_tensor_step([c.entry(tg, step, bits, tensor_id=2)], B,
                                  rounding="stochastic" if rounding else "nearest", seed=11)
        try:
            c.check(p_prev)
        except AssertionError as e:
            raise AssertionError(f"step {step}: {e}") from None
