"""Non-finite gradients on the GPU.  The reference's codes for a block holding inf / NaN values
are undefined (a NaN quotient goes through a double -> int cast, stquant_kernel.cu:113-131), so
those blocks are not compared.  What must hold: every block without a non-finite value keeps
bit-exact codes and scales and matching params, whichever kernel path its tile takes (a tile
with a non-finite value takes the exact path, its neighbours the fast one), and the launch
completes normally."""
import numpy as np
import pytest
import torch

import mdq_hip
from oracle import mdq_oracle as orc
from test_gpu_parity import DEV, HP, STORE_TORCH, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("storage,bits,B,rounding", [(orc.STORE_P4, 4, 128, "nearest"),
                                                     (orc.STORE_S8, 8, 64, "nearest"),
                                                     (orc.STORE_S8, 8, 256, "stochastic")])
def test_nonfinite_grads_leave_finite_blocks_exact(storage, bits, B, rounding):
    print(f"case: non-finite grads storage={storage} bits={bits} B={B} {rounding}", flush=True)
    n = 1 << 18
    rng = np.random.default_rng(5)
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    cm, cv, sm, sv, vm = orc.init_state(n, B, storage)
    dm, dv = STORE_TORCH[storage]
    tp, tcm, tsm, tsv, tvm = (to_dev(a.copy()) for a in (p, cm, sm, sv, vm))
    tcv = to_dev(cv.copy()) if cv is not None else torch.empty(0, dtype=torch.uint8, device=DEV)
    rnd = orc.ROUND_STOCHASTIC if rounding == "stochastic" else orc.ROUND_NEAREST
    bad_blocks = set()
    for step in (1, 2, 3):
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        if step == 2:
            idx = rng.choice(n, 12, replace=False)
            g[idx[:4]] = np.inf
            g[idx[4:8]] = -np.inf
            g[idx[8:]] = np.nan
            bad_blocks |= set((idx // B).tolist())
        orc.step(p, g.copy(), cm, cv, sm, sv, vm, step=step, bits=bits, block_size=B, storage=storage,
                 rounding=rnd, seed=3, **HP)
        e = mdq_hip.TensorState(tp, to_dev(g), tcm, tcv, tsm, tsv, tvm, step, bits, HP["lr"], HP["beta1"],
                                HP["beta2"], HP["eps"], HP["weight_decay"], 0)
        mdq_hip.multi_tensor_step([e], B, rounding=rounding, seed=3)
        torch.cuda.synchronize()
        good = np.ones(n // B, bool)
        good[list(bad_blocks)] = False
        ge = np.repeat(good, B)
        assert np.array_equal(tcm.cpu().numpy()[ge], cm[ge]), f"m codes, step {step}"
        if cv is not None:
            assert np.array_equal(tcv.cpu().numpy()[ge], cv[ge]), f"v codes, step {step}"
        for name, t, a in (("scale_m", tsm, sm), ("scale_v", tsv, sv), ("v_min", tvm, vm)):
            assert np.array_equal(t.cpu().numpy()[good].view(np.uint32), a[good].view(np.uint32)), f"{name} {step}"
        got = tp.cpu().numpy()
        assert np.allclose(got[ge], p[ge], rtol=1e-5, atol=1e-9), f"params, step {step}"
        # later steps start from identical state everywhere (the oracle's), so only the blocks
        # that ever held a non-finite value stay excluded
        tp.copy_(torch.from_numpy(p))
        tcm.copy_(torch.from_numpy(cm))
        if cv is not None:
            tcv.copy_(torch.from_numpy(cv))
        for t, a in ((tsm, sm), (tsv, sv), (tvm, vm)):
            t.copy_(torch.from_numpy(a))
