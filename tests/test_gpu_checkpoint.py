"""Checkpoint and resume of the drop-in optimizers on the GPU (stquant_opt_simple.py:361-378).

The drivers save ``optimizer.state_dict()`` with ``torch.save`` and resume with
``load_state_dict``.  Under the default MDQ schedule (scored bit widths, so the code storage
changes between steps) a run that is saved, reloaded into a fresh optimizer and continued must
match the uninterrupted run bit for bit: codes, scales, steps, bit widths and params.  A checkpoint
written on the GPU must also resume in an optimizer whose params live on the host (here the CPU
oracle in place of the kernel), including the global EMA statistics of the bit decision, which
torch's loader leaves on the device they were saved from.
"""
import io

import pytest
import torch

from stquant_opt_fused_io import MDQAdamWSimpleFusedIO
from stquant_opt_simple import MDQAdamWSimple
from test_gpu_optimizer import DEV, build, compare, grads
from test_optimizer_cpu import SimpleCPU

pytestmark = pytest.mark.gpu
SHAPES = [(300, 17), (4096,), (129,), (2, 2000)]
KW = dict(block_size=128, update_freq=3)


def checkpoint(opt):
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    return torch.load(buf, weights_only=True)


def exact_equal(opt_a, opt_b, pa, pb, tag):
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(pa, pb)):
        sa, sb = opt_a.state[a], opt_b.state[b]
        assert sa["step"] == sb["step"] and sa["current_bit"] == sb["current_bit"], (tag, i)
        for k in ("exp_avg", "exp_avg_sq", "scale_m", "scale_v", "v_min"):
            assert sa[k].dtype == sb[k].dtype and torch.equal(sa[k], sb[k]), (tag, i, k)
        assert torch.equal(a.detach(), b.detach()), (tag, i)
    for k in ("n_ema", "r_ema", "v_global_ema"):
        va, vb = getattr(opt_a, k), getattr(opt_b, k)
        assert (va is None and vb is None) or torch.equal(va, vb), (tag, k)
    assert opt_a.total_steps == opt_b.total_steps


def scaled_grads(cpu, gpu, t):
    """Seeded grads with per-tensor scales that swap between steps, so the scored bit widths
    of the tensors move between 4, 8 and 16 bits from one update step to the next."""
    grads(cpu, gpu, t)
    scales = [1.0, 30.0, 1 / 30, 3.0] if t % 2 else [3.0, 1 / 30, 30.0, 1.0]
    for p, s in zip(gpu, scales):
        p.grad.mul_(s)


@pytest.mark.parametrize("cls", [MDQAdamWSimple, MDQAdamWSimpleFusedIO])
def test_resume_matches_uninterrupted_run(cls):
    print(f"case: {cls.__name__} save at step 4, resume, 6 more steps", flush=True)
    cpu, gpu = build(SHAPES, seed=11)
    opt = cls(gpu, **KW)
    for t in range(1, 5):
        scaled_grads(cpu, gpu, t)
        opt.step()
    sd = checkpoint(opt)
    gpu2 = [torch.nn.Parameter(p.detach().clone()) for p in gpu]
    opt2 = cls(gpu2, **KW)
    opt2.load_state_dict(sd)
    exact_equal(opt, opt2, gpu, gpu2, "after load")
    changes = 0
    for t in range(5, 11):
        scaled_grads(cpu, gpu, t)
        for a, b in zip(gpu, gpu2):
            b.grad = a.grad.clone()
        before = [int(opt.state[p]["current_bit"]) for p in gpu]
        opt.step()
        opt2.step()
        exact_equal(opt, opt2, gpu, gpu2, f"step {t}")
        after = [int(opt.state[p]["current_bit"]) for p in gpu]
        changes += sum(a != b for a, b in zip(before, after))
        print(f"step {t}: bits {after}", flush=True)
    assert changes > 0, "the resumed steps should change some bit widths"


def test_gpu_checkpoint_resumes_on_host():
    print("case: GPU checkpoint loaded into a host optimizer", flush=True)
    cpu, gpu = build(SHAPES, seed=12)
    opt_g = MDQAdamWSimple(gpu, **KW)
    for t in range(1, 5):
        grads(cpu, gpu, 50 + t)
        opt_g.step()
    sd = checkpoint(opt_g)                       # device tensors, as torch.save wrote them
    host = [torch.nn.Parameter(p.detach().cpu().clone()) for p in gpu]
    opt_c = SimpleCPU(host, **KW)
    opt_c.load_state_dict(sd)
    assert opt_c.n_ema.device.type == "cpu" and opt_c.state[host[0]]["exp_avg"].device.type == "cpu"
    compare(opt_c, opt_g, host, gpu, "after load")
    for t in range(5, 9):                        # total_steps 6 is an update step: the EMAs are used
        grads(host, gpu, 50 + t)
        opt_c.step()
        opt_g.step()
        compare(opt_c, opt_g, host, gpu, f"step {t}")
    assert DEV.type == "cuda"


@pytest.mark.parametrize("bits", [4, 8, 16, 32])
def test_fixed_width_resume_on_the_gpu(bits):
    """Fixed code widths, 32-bit included (int32 / uint32 codes up to 2^32 - 1 do not survive a
    cast through float32): save after 3 steps, reload into a fresh optimizer on the GPU, and the
    next 3 steps match the uninterrupted run bit for bit."""
    print(f"case: fixed {bits}-bit save at step 3, resume, 3 more steps", flush=True)
    cpu, gpu = build(SHAPES, seed=13)
    kw = dict(block_size=128, bits=bits)
    opt = MDQAdamWSimpleFusedIO(gpu, **kw)
    for t in range(1, 4):
        grads(cpu, gpu, 70 + t)
        opt.step()
    sd = checkpoint(opt)
    gpu2 = [torch.nn.Parameter(p.detach().clone()) for p in gpu]
    opt2 = MDQAdamWSimpleFusedIO(gpu2, **kw)
    opt2.load_state_dict(sd)
    exact_equal(opt, opt2, gpu, gpu2, "after load")
    for t in range(4, 7):
        grads(cpu, gpu, 70 + t)
        for a, b in zip(gpu, gpu2):
            b.grad = a.grad.clone()
        opt.step()
        opt2.step()
        exact_equal(opt, opt2, gpu, gpu2, f"step {t}")
    assert all(int(opt.state[p]["current_bit"]) == bits for p in gpu)
