"""Parity at full size on the headline workload: the LLaMA-7B-shaped set that
bench.py times (291 tensors, 6,738,415,616 fp32 params in one flat buffer of views, bf16 grads,
packed 4-bit codes, B = 128), stepped twice through the same launch plan as the benchmark, then a
third time with stochastic rounding.

Quant blocks are independent, so the oracle judges block-aligned slices on their own: the first and
last 4096 elements of the embedding, the first decoder layer's q_proj and an RMSNorm weight, a
middle layer's down_proj, the final norm and lm_head (the last tensor, whose last tile ends the
launch).  Codes and the three scale arrays bit-exact, params within the parity bar.  In the
stochastic step each slice is judged with its start in the tensor as the oracle's elem_offset, the
tensor's index as its stream id.  About 48 GB of device memory.
"""
import numpy as np
import pytest
import torch

import bench
import mdq_hip
from oracle import mdq_oracle as orc
from test_gpu_parity import assert_bits_equal, assert_params_close

pytestmark = pytest.mark.gpu
B = 128
HP = dict(beta1=0.9, beta2=0.999, lr=1e-3, weight_decay=0.01, eps=1e-8)   # bench.build_workload's
PICK = ("embed_tokens", "layers.0.self_attn.q_proj", "layers.0.input_layernorm", "layers.16.mlp.down_proj",
        "norm", "lm_head")
W = 4096


def host(t):
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16).copy()
    return t.cpu().numpy().copy()


def test_llama7b_set_three_steps_on_slices():
    print("case: llama7b full set, 2 nearest + 1 stochastic step, slices of 6 tensors", flush=True)
    dev = torch.device("cuda:0")
    w = bench.build_workload("llama7b", dev)
    plan = w["plan"]
    p, g, codes, _vc, sm, sv, vm = w["keep"]
    shapes = bench.llama7b_shapes()
    offs, boffs, tid, o, ob = {}, {}, {}, 0, 0
    for i, (name, n) in enumerate(shapes):
        offs[name], boffs[name], tid[name] = (o, n), ob, i
        o += n
        ob += (n + B - 1) // B
    slices = []
    for name in PICK:
        o, n = offs[name]
        for s in sorted({0, max(0, n - W)}):
            e = min(n, s + W)
            slices.append((name, o + s, o + e, boffs[name] + s // B, boffs[name] + (e + B - 1) // B, s))
    sr_plan = mdq_hip.MultiTensorPlan(w["entries"], B, rounding="stochastic", seed=7)
    for step, run_plan, rounding in ((1, plan, orc.ROUND_NEAREST), (2, plan, orc.ROUND_NEAREST),
                                     (3, sr_plan, orc.ROUND_STOCHASTIC)):
        snap = [(host(p[a:b]), host(g[a:b]), host(codes[a:b]), host(sm[c:d]), host(sv[c:d]), host(vm[c:d]))
                for _n, a, b, c, d, _s in slices]
        run_plan.set_steps(step)
        run_plan.run()
        torch.cuda.synchronize()
        for (name, a, b, c, d, s), (hp, hg, hc, hsm, hsv, hvm) in zip(slices, snap):
            p_prev = hp.copy()
            orc.step(hp, hg, hc, None, hsm, hsv, hvm, step=step, bits=4, block_size=B, storage=orc.STORE_P4,
                     rounding=rounding, seed=7, tensor_id=tid[name], elem_offset=s, **HP)
            tag = f"step {step} {name} [{a}, {b})"
            assert_bits_equal(f"{tag} codes", codes[a:b], hc)
            assert_bits_equal(f"{tag} scale_m", sm[c:d], hsm)
            assert_bits_equal(f"{tag} scale_v", sv[c:d], hsv)
            assert_bits_equal(f"{tag} v_min", vm[c:d], hvm)
            assert_params_close(p[a:b], hp, p_prev, label=f"config 4 {tag}")
