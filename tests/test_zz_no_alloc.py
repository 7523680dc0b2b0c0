"""The allocation-free entry point (stq_multi_tensor_mdq_adamw_noalloc) against the ordinary
multi-tensor entry point (stq_multi_tensor_mdq_adamw), through the C ABI: the same tensors
stepped by each from identical states give bit-identical codes, scales and params.  Two calls in
a row, the second with fewer and smaller tensors (the fixed descriptor array keeps the first
call's table, which the second must not read); nearest and stochastic rounding, packed 4-bit and
int8 codes.  Calls queued back to back with no synchronisation between them, the first long
enough that its kernel still runs when the second call's table is copied, on one stream and
alternating between two streams (every call on a GPU shares the one descriptor array, so the
library orders each copy after the previous call's kernel).  A list longer than
STQ_NOALLOC_MAX_TENSORS is refused before any device work."""
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


def test_noalloc_at_the_tensor_limit():
    """Exactly STQ_NOALLOC_MAX_TENSORS tensors (the whole fixed descriptor array), sizes 1 to
    2000 elements, then a call over 3 tensors; both bit-identical to the ordinary entry point."""
    print(f"case: noalloc with {mdq_hip.NOALLOC_MAX_TENSORS} tensors", flush=True)
    rng = np.random.default_rng(4096)
    full = [int(x) for x in rng.integers(1, 2001, mdq_hip.NOALLOC_MAX_TENSORS)]
    for call, sizes in enumerate((full, [300, 1, 70_000]), start=1):
        ref, got = make_set(sizes, 4, 40 + call)
        mdq_hip.MultiTensorPlan(entries(ref, 4, call), B).run()
        mdq_hip.MultiTensorPlan(entries(got, 4, call), B).run(noalloc=True)
        torch.cuda.synchronize()
        _assert_same(ref, got, f"call {call}")
        print(f"call {call}: {len(sizes)} tensors bit-identical", flush=True)


def test_noalloc_refuses_too_many_tensors():
    ts = make_set([8] * (mdq_hip.NOALLOC_MAX_TENSORS + 1), 4, 0)[0]
    plan = mdq_hip.MultiTensorPlan(entries(ts, 4, 1), B)
    before = [x.clone() for x in ts[0]]
    with pytest.raises(RuntimeError, match="STQ_NOALLOC_MAX_TENSORS"):
        plan.run(noalloc=True)
    torch.cuda.synchronize()
    for x, y in zip(ts[0], before):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))


def _assert_same(ref, got, what):
    for i, (a, b) in enumerate(zip(ref, got)):
        for name, x, y in zip(("p", "grad", "exp_avg", "exp_avg_sq", "scale_m", "scale_v", "v_min"), a, b):
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), (what, i, name)


@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
def test_noalloc_calls_back_to_back_without_a_sync(rounding):
    """A large set (four 2^24-element tensors) then a small one, queued on one stream with no
    synchronisation in between: the second table copy must wait for the first kernel.  The
    ordinary entry point steps identical copies; the noalloc calls upload nothing to its ring."""
    print(f"case: noalloc back to back on one stream, {rounding}", flush=True)
    big = [1 << 24] * 4 + [12_345]
    small = [700, 5, 65_536]
    ref_a, got_a = make_set(big, 4, 21)
    ref_b, got_b = make_set(small, 4, 22)
    mdq_hip.MultiTensorPlan(entries(ref_a, 4, 3), B, rounding=rounding, seed=5).run()
    mdq_hip.MultiTensorPlan(entries(ref_b, 4, 4), B, rounding=rounding, seed=5).run()
    plan_a = mdq_hip.MultiTensorPlan(entries(got_a, 4, 3), B, rounding=rounding, seed=5)
    plan_b = mdq_hip.MultiTensorPlan(entries(got_b, 4, 4), B, rounding=rounding, seed=5)
    torch.cuda.synchronize()
    before = mdq_hip.step_table_uploads()
    plan_a.run(noalloc=True)
    plan_b.run(noalloc=True)
    after = mdq_hip.step_table_uploads()
    torch.cuda.synchronize()
    assert after == before, "the noalloc calls must not take the ordinary entry point's ring"
    _assert_same(ref_a, got_a, "large set")
    _assert_same(ref_b, got_b, "small set")
    print(f"{sum(big):,} then {sum(small):,} params bit-identical, uploads {before} -> {after}", flush=True)


def test_noalloc_calls_alternating_between_two_streams():
    """Two tensor sets of identical shapes, one per stream, stepped alternately for four steps
    with no synchronisation: a kernel that read the other stream's table would step the other
    set (valid memory, wrong result).  Both sets must equal the ordinary entry point's steps."""
    print("case: noalloc alternating between two streams", flush=True)
    sizes = [1 << 23, 1 << 23, 33_333, 129]
    ref_a, got_a = make_set(sizes, 8, 31)
    ref_b, got_b = make_set(sizes, 8, 32)
    for step in range(1, 5):
        for ref in (ref_a, ref_b):
            mdq_hip.MultiTensorPlan(entries(ref, 8, step), B, rounding="stochastic", seed=9).run()
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(DEV), torch.cuda.Stream(DEV)
    s1.wait_stream(torch.cuda.current_stream(DEV))
    s2.wait_stream(torch.cuda.current_stream(DEV))
    plans = [(s1, mdq_hip.MultiTensorPlan(entries(got_a, 8, 1), B, rounding="stochastic", seed=9)),
             (s2, mdq_hip.MultiTensorPlan(entries(got_b, 8, 1), B, rounding="stochastic", seed=9))]
    for step in range(1, 5):
        for stream, plan in plans:
            plan.set_steps(step)
            with torch.cuda.stream(stream):
                plan.run(noalloc=True)
    torch.cuda.synchronize()
    _assert_same(ref_a, got_a, "stream 1 set")
    _assert_same(ref_b, got_b, "stream 2 set")
    print(f"2 x {sum(sizes):,} params, 4 alternating steps bit-identical", flush=True)
