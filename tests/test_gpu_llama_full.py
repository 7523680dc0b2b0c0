"""Parity at full size on the headline workload: the LLaMA-7B-shaped set that
bench.py times (291 tensors, 6,738,415,616 fp32 params in one flat buffer of views, bf16 grads,
packed 4-bit codes, B = 128), stepped twice through the same launch plan as the benchmark.

Quant blocks are independent, so the oracle judges block-aligned slices on their own: the first and
last 4096 elements of the embedding, the first decoder layer's q_proj and an RMSNorm weight, a
middle layer's down_proj, the final norm and lm_head (the last tensor, whose last tile ends the
launch).  Codes and the three scale arrays bit-exact, params within the parity bar.  About 48 GB
of device memory.
"""
import numpy as np
import pytest
import torch

import bench
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


def test_llama7b_set_two_steps_on_slices():
    print("case: llama7b full set, 2 steps, slices of 6 tensors", flush=True)
    dev = torch.device("cuda:0")
    w = bench.build_workload("llama7b", dev)
    plan = w["plan"]
    p, g, codes, _vc, sm, sv, vm = w["keep"]
    shapes = bench.llama7b_shapes()
    offs, boffs, o, ob = {}, {}, 0, 0
    for name, n in shapes:
        offs[name], boffs[name] = (o, n), ob
        o += n
        ob += (n + B - 1) // B
    slices = []
    for name in PICK:
        o, n = offs[name]
        for s in sorted({0, max(0, n - W)}):
            e = min(n, s + W)
            slices.append((name, o + s, o + e, boffs[name] + s // B, boffs[name] + (e + B - 1) // B))
    for step in (1, 2):
        snap = [(host(p[a:b]), host(g[a:b]), host(codes[a:b]), host(sm[c:d]), host(sv[c:d]), host(vm[c:d]))
                for _n, a, b, c, d in slices]
        plan.set_steps(step)
        plan.run()
        torch.cuda.synchronize()
        for (name, a, b, c, d), (hp, hg, hc, hsm, hsv, hvm) in zip(slices, snap):
            p_prev = hp.copy()
            orc.step(hp, hg, hc, None, hsm, hsv, hvm, step=step, bits=4, block_size=B, storage=orc.STORE_P4, **HP)
            tag = f"step {step} {name} [{a}, {b})"
            assert_bits_equal(f"{tag} codes", codes[a:b], hc)
            assert_bits_equal(f"{tag} scale_m", sm[c:d], hsm)
            assert_bits_equal(f"{tag} scale_v", sv[c:d], hsv)
            assert_bits_equal(f"{tag} v_min", vm[c:d], hvm)
            assert_params_close(p[a:b], hp, p_prev)
