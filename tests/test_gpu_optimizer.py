"""The drop-in optimizers on the GPU (HIP kernels via the C ABI) against the same
classes with the CPU oracle in place of the kernel (tests/test_optimizer_cpu.py),
on identical params and grads: codes and scales bit-exact after every step
through bit-width transitions, two param groups, FusedIO's fast path and
stochastic rounding; params within 1e-6 of max|p|."""
import numpy as np
import pytest
import torch

from stquant_opt_fused_io import MDQAdamWSimpleFusedIO
from stquant_opt_simple import MDQAdamWSimple
from test_optimizer_cpu import FusedIOCPU, SimpleCPU

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def build(shapes, seed=0):
    g = torch.Generator().manual_seed(seed)
    cpu = [torch.nn.Parameter(torch.randn(*s, generator=g) * 0.02) for s in shapes]
    gpu = [torch.nn.Parameter(p.detach().clone().to(DEV)) for p in cpu]
    return cpu, gpu


def grads(cpu, gpu, seed):
    g = torch.Generator().manual_seed(seed)
    for a, b in zip(cpu, gpu):
        a.grad = torch.randn(a.shape, generator=g) * 1e-3
        b.grad = a.grad.to(DEV)


def compare(opt_c, opt_g, cpu, gpu, tag, p_scale=0.0):
    """Codes, scales, steps and widths identical; params within 1e-6 of the tensor's magnitude,
    max|p| or ``p_scale`` (the params' initial scale) if larger: a tensor of one or a few elements
    that its steps carried next to zero has a tiny max|p|."""
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(cpu, gpu)):
        sa, sb = opt_c.state[a], opt_g.state[b]
        assert sa["step"] == sb["step"] and sa["current_bit"] == sb["current_bit"], (tag, i)
        for k in ("exp_avg", "exp_avg_sq", "scale_m", "scale_v", "v_min"):
            x, y = sa[k], sb[k].cpu()
            assert x.dtype == y.dtype and x.shape == y.shape, (tag, i, k)
            if x.dtype.is_floating_point:
                assert torch.equal(x.view(torch.int32), y.view(torch.int32)), (tag, i, k)
            else:
                assert torch.equal(x.to(torch.int64), y.to(torch.int64)), (tag, i, k)
        pa, pb = a.detach().double(), b.detach().cpu().double()
        assert (pa - pb).abs().max() <= 1e-6 * max(pa.abs().max().item(), p_scale), (tag, i)


@pytest.mark.parametrize("cls_c,cls_g", [(SimpleCPU, MDQAdamWSimple), (FusedIOCPU, MDQAdamWSimpleFusedIO)])
def test_transitions_and_groups(cls_c, cls_g):
    print(f"case: {cls_g.__name__} transitions", flush=True)
    shapes = [(700, 13), (4096,), (129,), (3, 1000)]
    cpu, gpu = build(shapes)

    def groups(ps):
        return [{"params": ps[:2], "lr": 2e-3, "weight_decay": 0.01},
                {"params": ps[2:], "lr": 1e-3, "weight_decay": 0.0}]
    kw = dict(bits=4, block_size=128)
    opt_c, opt_g = cls_c(groups(cpu), **kw), cls_g(groups(gpu), **kw)
    for t, bits in enumerate([4, 4, 8, 16, 4, 32, 8, 4], start=1):
        for o in (opt_c, opt_g):
            for g in o.param_groups:
                g["bits"] = bits
        grads(cpu, gpu, t)
        opt_c.step()
        opt_g.step()
        compare(opt_c, opt_g, cpu, gpu, f"step {t} bits {bits}")


@pytest.mark.parametrize("cls_c,cls_g", [(SimpleCPU, MDQAdamWSimple), (FusedIOCPU, MDQAdamWSimpleFusedIO)],
                         ids=["simple", "fused_io"])
def test_hundreds_of_tensors_through_width_changes(cls_c, cls_g):
    """400 params of 1 to 2000 elements (1-D and 2-D) in two groups, widths forced through
    4 -> 4 -> 8 -> 16 -> 4 -> 4 (steady steps, storage changes, the steady plan rebuilt), some
    params without a grad on some steps; the GPU optimizer against its oracle-driven twin after
    every step."""
    print(f"case: {cls_g.__name__} 400 tensors", flush=True)
    rng = np.random.default_rng(400)
    shapes = []
    for _ in range(400):
        n = int(np.floor(np.exp(rng.uniform(0, np.log(2000)))))
        shapes.append((n,) if rng.random() < 0.5 or n < 4 else (n // 4, 4))
    cpu, gpu = build(shapes, seed=11)

    def groups(ps):
        return [{"params": ps[:250], "lr": 2e-3, "weight_decay": 0.01},
                {"params": ps[250:], "lr": 1e-3, "weight_decay": 0.0}]
    kw = dict(bits=4, block_size=128)
    opt_c, opt_g = cls_c(groups(cpu), **kw), cls_g(groups(gpu), **kw)
    for t, bits in enumerate([4, 4, 8, 16, 4, 4], start=1):
        for o in (opt_c, opt_g):
            for g in o.param_groups:
                g["bits"] = bits
        grads(cpu, gpu, 500 + t)
        if t == 5:                                   # a step where some params have no grad
            for i in range(0, 400, 7):
                cpu[i].grad = None
                gpu[i].grad = None
        opt_c.step()
        opt_g.step()
        compare(opt_c, opt_g, cpu, gpu, f"step {t} bits {bits}", p_scale=0.02)


def test_stochastic_rounding_matches_oracle():
    print("case: optimizer stochastic", flush=True)
    shapes = [(1000, 7), (333,)]
    cpu, gpu = build(shapes, seed=3)
    kw = dict(bits=4, block_size=64, rounding="stochastic", seed=77)
    opt_c, opt_g = SimpleCPU(cpu, **kw), MDQAdamWSimple(gpu, **kw)
    for t in range(1, 5):
        grads(cpu, gpu, 100 + t)
        opt_c.step()
        opt_g.step()
        compare(opt_c, opt_g, cpu, gpu, f"step {t}")


def test_default_schedule_runs_on_gpu():
    print("case: optimizer default MDQ schedule", flush=True)
    cpu, gpu = build([(512, 64), (2048,), (64,)], seed=5)
    opt = MDQAdamWSimpleFusedIO(gpu, block_size=256, update_freq=4)
    for t in range(1, 10):
        grads(cpu, gpu, t)
        opt.step()
    lt = opt.get_last_step_timings()
    assert lt["mdq_fused_kernel_ms"] > 0
    assert abs(sum(opt.get_bit_distribution().values()) - 100.0) < 1e-6
    for p in gpu:
        assert torch.isfinite(p).all()
        st = opt.state[p]
        assert st["step"] >= 9 and st["current_bit"] in (4, 8, 16, 32)
