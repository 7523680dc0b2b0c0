"""The allocation-free entry point (stq_multi_tensor_mdq_adamw_noalloc) against the ordinary
multi-tensor entry point (stq_multi_tensor_mdq_adamw), through the C ABI: the same tensors
stepped by each from identical states give bit-identical codes, scales and params.  Two calls in
a row, the second with fewer and smaller tensors (the fixed descriptor array keeps the first
call's table, which the second must not read); nearest and stochastic rounding, packed 4-bit and
int8 codes.  A list longer than STQ_NOALLOC_MAX_TENSORS is refused before any device work."""
import numpy as np
import pytest
import torch

import mdq_hip

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
B = 128


def make_set(sizes, bits, seed):
    """Two identical copies of a tensor set: params, bf16 grads, codes and scales."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    copies = ([], [])
    for n in sizes:
        p = torch.randn(n, device=DEV, generator=g) * 0.02
        gr = (torch.randn(n, device=DEV, generator=g) * 1e-3).to(torch.bfloat16)
        nb = (n + B - 1) // B
        if bits == 4:
            m = torch.randint(0, 256, (n,), device=DEV, generator=g).to(torch.uint8)
            v = torch.empty(0, dtype=torch.uint8, device=DEV)
        else:
            m = torch.randint(-128, 128, (n,), device=DEV, generator=g).to(torch.int8)
            v = torch.randint(0, 256, (n,), device=DEV, generator=g).to(torch.uint8)
        sm = torch.rand(nb, device=DEV, generator=g) * 1e-4
        sv = torch.rand(nb, device=DEV, generator=g)
        vm = -20.0 + torch.rand(nb, device=DEV, generator=g)
        for c in copies:
            c.append([x.clone() for x in (p, gr, m, v, sm, sv, vm)])
    return copies


def entries(ts, bits, step):
    return [mdq_hip.TensorState(p, gr, m, v, sm, sv, vm, step, bits, 1e-3, 0.9, 0.999, 1e-8, 0.01, i)
            for i, (p, gr, m, v, sm, sv, vm) in enumerate(ts)]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
def test_noalloc_matches_the_ordinary_entry_point(bits, rounding):
    print(f"case: noalloc vs multi-tensor entry, bits={bits} {rounding}", flush=True)
    rng = np.random.default_rng(bits)
    first = [int(x) for x in rng.integers(1, 300_000, 37)] + [1 << 20, 4096, 1]
    second = [int(x) for x in rng.integers(1, 50_000, 5)]
    for call, sizes in enumerate((first, second), start=1):
        ref, got = make_set(sizes, bits, 10 * call + bits)
        mdq_hip.MultiTensorPlan(entries(ref, bits, call), B, rounding=rounding, seed=3).run()
        mdq_hip.MultiTensorPlan(entries(got, bits, call), B, rounding=rounding, seed=3).run(noalloc=True)
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(ref, got)):
            for name, x, y in zip(("p", "grad", "exp_avg", "exp_avg_sq", "scale_m", "scale_v", "v_min"), a, b):
                assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), (call, i, name)
        print(f"call {call}: {len(sizes)} tensors, {sum(sizes):,} params bit-identical", flush=True)


def test_noalloc_refuses_too_many_tensors():
    ts = make_set([8] * (mdq_hip.NOALLOC_MAX_TENSORS + 1), 4, 0)[0]
    plan = mdq_hip.MultiTensorPlan(entries(ts, 4, 1), B)
    before = [x.clone() for x in ts[0]]
    with pytest.raises(RuntimeError, match="STQ_NOALLOC_MAX_TENSORS"):
        plan.run(noalloc=True)
    torch.cuda.synchronize()
    for x, y in zip(ts[0], before):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))
