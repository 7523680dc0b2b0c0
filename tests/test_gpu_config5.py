"""BASELINE config 5 at full size on the GPU against the oracle: 257 tensors with
log-uniform sizes (363,174,740 params, 254 ragged at B=128), Student-t(3) grads
with 5 % all-zero blocks and 0.1 % x1000 outliers, one multi-tensor launch.
Codes and scales bit-exact, params within the bar of tests/param_bar.py.

``align`` = 1 packs the tensors back to back in one buffer (views at odd
element offsets: the element-wise path of every tile); 256 starts each tensor
on a 1 KiB boundary, as separate allocations do (vector path, ragged tails)."""
import numpy as np
import pytest
import torch

import bench
import mdq_hip
from oracle import mdq_oracle as orc
from test_gpu_parity import assert_params_close

pytestmark = pytest.mark.gpu
HP = dict(beta1=0.9, beta2=0.999, lr=1e-3, weight_decay=0.01, eps=1e-8)


@pytest.mark.parametrize("bits,B,rounding,align", [(4, 128, "nearest", 256), (8, 64, "stochastic", 1),
                                                   (4, 256, "stochastic", 256)])
def test_config5_full_size(bits, B, rounding, align):
    print(f"case: config5 bits={bits} B={B} {rounding} align={align}", flush=True)
    dev = torch.device("cuda:0")
    sizes = bench.config5_sizes()
    offs = np.concatenate([[0], np.cumsum([(n + align - 1) // align * align for n in sizes])]).tolist()
    N = offs[-1]
    rng = np.random.default_rng(11)
    p = (rng.standard_normal(N) * 0.02).astype(np.float32)
    g = np.zeros(N, np.float32)
    for n, o in zip(sizes, offs):
        g[o:o + n] = bench.config5_grads_numpy(n, B, rng)
    storage = orc.STORE_P4 if bits == 4 else orc.STORE_S8
    nbs = [(n + B - 1) // B for n in sizes]
    NB = sum(nbs)
    cm, cv, _, _, _ = orc.init_state(N, B, storage)      # codes of all tensors in one buffer
    sm, sv, vm = np.zeros(NB, np.float32), np.zeros(NB, np.float32), np.full(NB, -20.0, np.float32)
    tp, tg, tcm = (torch.from_numpy(a.copy()).to(dev) for a in (p, g, cm))
    tcv = torch.from_numpy(cv.copy()).to(dev) if cv is not None else torch.empty(0, dtype=torch.uint8, device=dev)
    tsm, tsv, tvm = (torch.from_numpy(a.copy()).to(dev) for a in (sm, sv, vm))
    rnd = orc.ROUND_STOCHASTIC if rounding == "stochastic" else orc.ROUND_NEAREST
    for step in (1, 2):
        p_prev = p.copy()
        entries, ob = [], 0
        for i, (n, nb, o) in enumerate(zip(sizes, nbs, offs)):
            orc.step(p[o:o + n], g[o:o + n], cm[o:o + n], None if cv is None else cv[o:o + n],
                     sm[ob:ob + nb], sv[ob:ob + nb], vm[ob:ob + nb], step=step, bits=bits, block_size=B,
                     storage=storage, rounding=rnd, seed=99, tensor_id=i, **HP)
            entries.append(mdq_hip.TensorState(
                tp[o:o + n], tg[o:o + n], tcm[o:o + n], tcv if cv is None else tcv[o:o + n],
                tsm[ob:ob + nb], tsv[ob:ob + nb], tvm[ob:ob + nb], step, bits, HP["lr"], HP["beta1"],
                HP["beta2"], HP["eps"], HP["weight_decay"], i))
            ob += nb
        mdq_hip.multi_tensor_step(entries, B, rounding=rounding, seed=99)
        torch.cuda.synchronize()
        assert np.array_equal(tcm.cpu().numpy(), cm), f"m codes differ at step {step}"
        if cv is not None:
            assert np.array_equal(tcv.cpu().numpy(), cv), f"v codes differ at step {step}"
        for name, t, a in (("scale_m", tsm, sm), ("scale_v", tsv, sv), ("v_min", tvm, vm)):
            assert np.array_equal(t.cpu().numpy().view(np.uint32), a.view(np.uint32)), f"{name} step {step}"
        assert_params_close(tp, p, p_prev, label=f"config 5 {bits}-bit B={B} {rounding} step {step}")
        tp.copy_(torch.from_numpy(p))
