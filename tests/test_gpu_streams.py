"""Calls on several streams and from several host threads, through the C ABI.

The descriptor table of each call lives in a library-owned ring of 8 device slots per device; a
slot is reused only after the event recorded behind its last launch has completed, small launches
(< 2^24 elements) upload on the caller's stream and large ones on a copy stream.  Here two tensor
sets are stepped in interleaved launches on two streams (one set small, one large, so both upload
routes alternate), for enough steps to wrap the ring several times, and then from two host
threads at once.  Every result must equal the same steps run one after the other on the current
stream, bit for bit (each set's steps see only its own tensors, so the order between the sets does
not matter)."""
import threading

import numpy as np
import pytest
import torch

import mdq_hip

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
B = 128


def make_set(sizes, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    out = []
    for i, n in enumerate(sizes):
        nb = (n + B - 1) // B
        p = torch.randn(n, device=DEV, generator=g) * 0.02
        cm = torch.full((n,), 8, dtype=torch.uint8, device=DEV)
        out.append([p, cm, torch.zeros(nb, device=DEV), torch.zeros(nb, device=DEV),
                    torch.full((nb,), -20.0, device=DEV), i])
    return out


def clone_set(s):
    return [[t.clone() for t in x[:5]] + [x[5]] for x in s]


def grads_for(sizes, step, seed):
    g = torch.Generator(device=DEV).manual_seed(seed * 1000 + step)
    return [(torch.randn(n, device=DEV, generator=g) * 1e-3).to(torch.bfloat16) for n in sizes]


def step_set(s, grads, step, rounding):
    empty = torch.empty(0, dtype=torch.uint8, device=DEV)
    entries = [mdq_hip.TensorState(p, gr, cm, empty, sm, sv, vm, step, 4, 1e-3, 0.9, 0.999, 1e-8, 0.01, tid)
               for (p, cm, sm, sv, vm, tid), gr in zip(s, grads)]
    mdq_hip.multi_tensor_step(entries, B, rounding=rounding, seed=3)


def assert_sets_equal(a, b, tag):
    for k, (x, y) in enumerate(zip(a, b)):
        for name, u, w in zip(("p", "codes", "scale_m", "scale_v", "v_min"), x[:5], y[:5]):
            assert torch.equal(u.view(torch.uint8), w.view(torch.uint8)), f"{tag}: tensor {k} {name}"


SMALL = [4097, 100_000, 1_000_003]            # 1.1M elements: uploads on the caller's stream
LARGE = [9_000_001, 12_000_000]               # 21M elements: uploads on the copy stream
STEPS = 12                                     # 24 launches: the 8-slot ring wraps three times


@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
def test_interleaved_streams_equal_sequential(rounding):
    print(f"case: two streams interleaved, {STEPS} steps each, {rounding}", flush=True)
    small, large = make_set(SMALL, 1), make_set(LARGE, 2)
    small_ref, large_ref = clone_set(small), clone_set(large)
    gs = [grads_for(SMALL, t, 1) for t in range(1, STEPS + 1)]
    gl = [grads_for(LARGE, t, 2) for t in range(1, STEPS + 1)]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(device=DEV), torch.cuda.Stream(device=DEV)
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    for t in range(1, STEPS + 1):
        with torch.cuda.stream(s1):
            step_set(small, gs[t - 1], t, rounding)
        with torch.cuda.stream(s2):
            step_set(large, gl[t - 1], t, rounding)
    torch.cuda.synchronize()
    for t in range(1, STEPS + 1):
        step_set(small_ref, gs[t - 1], t, rounding)
        step_set(large_ref, gl[t - 1], t, rounding)
    torch.cuda.synchronize()
    assert_sets_equal(small, small_ref, "small set")
    assert_sets_equal(large, large_ref, "large set")


def test_two_host_threads_equal_sequential():
    print(f"case: two host threads, own streams, {STEPS} steps each", flush=True)
    small, large = make_set(SMALL, 3), make_set(LARGE, 4)
    small_ref, large_ref = clone_set(small), clone_set(large)
    gs = [grads_for(SMALL, t, 3) for t in range(1, STEPS + 1)]
    gl = [grads_for(LARGE, t, 4) for t in range(1, STEPS + 1)]
    torch.cuda.synchronize()
    errors = []

    def worker(s, grads):
        try:
            st = torch.cuda.Stream(device=DEV)
            with torch.cuda.stream(st):
                for t in range(1, STEPS + 1):
                    step_set(s, grads[t - 1], t, "nearest")
            st.synchronize()
        except Exception as e:       # surfaced below
            errors.append(e)

    th = [threading.Thread(target=worker, args=(small, gs)), threading.Thread(target=worker, args=(large, gl))]
    for x in th:
        x.start()
    for x in th:
        x.join(timeout=120)
    assert not any(x.is_alive() for x in th), "worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for t in range(1, STEPS + 1):
        step_set(small_ref, gs[t - 1], t, "nearest")
        step_set(large_ref, gl[t - 1], t, "nearest")
    torch.cuda.synchronize()
    assert_sets_equal(small, small_ref, "small set")
    assert_sets_equal(large, large_ref, "large set")
