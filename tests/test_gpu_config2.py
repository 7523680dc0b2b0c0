"""BASELINE config 2 at full size: the 148 tensors of HF GPT-2 small (124,439,808 fp32 params
~N(0, 0.02), fp32 grads ~N(0, 1e-3), packed 4-bit codes, B = 128), as the reference's drivers hand
them to the optimizer in one group (/root/reference/CUDA/Cfinetuning_timetest.py:196-200).

- The benchmark's launch plan (one multi-tensor launch per step, the set as views of one buffer)
  stepped three times; the oracle judges block-aligned slices of every tensor: the first and the
  last 4096 elements (the whole tensor when smaller), so the head and tail of wte, wpe, every
  c_attn / c_proj / c_fc weight and bias and every LayerNorm weight and bias.  Codes and scale
  arrays bit-exact, params within the parity bar.
- The drop-in optimizer (MDQAdamWSimpleFusedIO, bits=4, block_size=128) over 148 separately
  allocated params of those shapes, three steps, against the same class with the CPU oracle
  executing its launch plans: every code and scale of the whole set bit-exact after every step
  (the first step moves the fresh int16 state to nibbles through the storage-changing kernel).
"""
import numpy as np
import pytest
import torch

import bench
import mdq_hip
from oracle import mdq_oracle as orc
from stquant_opt_fused_io import MDQAdamWSimpleFusedIO
from test_gpu_parity import assert_bits_equal, assert_params_close
from test_optimizer_cpu import FusedIOCPU

pytestmark = pytest.mark.gpu
B = 128
HP = dict(beta1=0.9, beta2=0.999, lr=1e-3, weight_decay=0.01, eps=1e-8)   # bench.build_workload's
W = 4096


def host(t):
    return t.cpu().numpy().copy()


def test_gpt2_small_set_three_steps_every_tensor():
    print("case: config 2, gpt2 small set, 3 nearest steps, slices of all 148 tensors", flush=True)
    dev = torch.device("cuda:0")
    w = bench.build_workload("gpt2", dev)
    assert w["N"] == 124_439_808 and w["tensors"] == 148 and w["gdt"] == "f32"
    plan = w["plan"]
    p, g, codes, _vc, sm, sv, vm = w["keep"]
    slices, o, ob = [], 0, 0
    for name, n in bench.gpt2_small_shapes():
        for s in sorted({0, max(0, n - W)}):
            e = min(n, s + W)
            slices.append((name, o + s, o + e, ob + s // B, ob + (e + B - 1) // B))
        o += n
        ob += (n + B - 1) // B
    for step in (1, 2, 3):
        # fresh grads every step, as training produces them
        gen = torch.Generator(device=dev).manual_seed(100 + step)
        g.copy_(torch.randn(g.numel(), device=dev, generator=gen).mul_(1e-3))
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
            assert_params_close(p[a:b], hp, p_prev, label=f"config 2 {tag}")


def test_gpt2_small_set_through_the_optimizer():
    print("case: config 2, gpt2 small set through MDQAdamWSimpleFusedIO vs the oracle, 3 steps", flush=True)
    dev = torch.device("cuda:0")
    shapes = bench.gpt2_small_shapes()
    gen = torch.Generator().manual_seed(0)
    cpu = [torch.nn.Parameter(torch.randn(n, generator=gen) * 0.02) for _name, n in shapes]
    gpu = [torch.nn.Parameter(p.detach().clone().to(dev)) for p in cpu]
    oc = FusedIOCPU(cpu, bits=4, block_size=B, **{k: HP[k] for k in ("lr", "eps", "weight_decay")})
    og = MDQAdamWSimpleFusedIO(gpu, bits=4, block_size=B, **{k: HP[k] for k in ("lr", "eps", "weight_decay")})
    for step in (1, 2, 3):
        gg = torch.Generator().manual_seed(200 + step)
        for a, b in zip(cpu, gpu):
            a.grad = torch.randn(a.shape, generator=gg) * 1e-3
            b.grad = a.grad.to(dev)
        oc.step()
        og.step()
        torch.cuda.synchronize()
        lt = og.get_last_step_timings()
        assert lt["mdq_fused_io_fast_path_params"] + lt["mdq_fused_io_fallback_params"] == 148
        worst = 0.0
        for i, (a, b) in enumerate(zip(cpu, gpu)):
            sa, sb = oc.state[a], og.state[b]
            assert sa["step"] == sb["step"] and sb["current_bit"] == 4, (step, i)
            assert sb["exp_avg"].dtype == torch.uint8 and sb["exp_avg_sq"].numel() == 0
            assert torch.equal(sa["exp_avg"], sb["exp_avg"].cpu()), (step, shapes[i][0], "codes")
            for k in ("scale_m", "scale_v", "v_min"):
                assert torch.equal(sa[k].view(torch.int32), sb[k].cpu().view(torch.int32)), (step, shapes[i][0], k)
            pa, pb = a.detach().double(), b.detach().cpu().double()
            err = float((pa - pb).abs().max())
            assert err <= 1e-6 * float(pa.abs().max()), (step, shapes[i][0], err)
            worst = max(worst, err)
        print(f"step {step}: 148 tensors, codes and scales bit-exact, max |dp| = {worst:.2e}", flush=True)
