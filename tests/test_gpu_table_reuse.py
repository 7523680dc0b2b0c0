"""Steady steps launch from the device copy of their descriptor table.

When every tensor of a launch has the same step count and AdamW constants, the step-dependent
constants travel as kernel arguments, the table of a fixed tensor set is the same at every step,
and a call whose table equals one an earlier call on the same stream left on the device launches
from it without an upload (stq_step_table_uploads counts the uploads).  Every case here is held
bit-exact (codes, scales) and within the parity bar (params) against the oracle after each step:
steady steps in both rounding modes, tensors with different step counts (no kernel-argument
constants), two tensor sets alternating, a grad buffer that moves, another stream, and ring
slots taken in between by other entry points.
"""
import numpy as np
import pytest
import torch

import mdq_hip
from oracle import mdq_oracle as orc
from test_gpu_parity import DEV, Case, resync_params

pytestmark = pytest.mark.gpu
SIZES = [4096, 1000, 70_001]
B = 128


class Set:
    """Tensors with persistent device grad buffers, refilled in place every step.  Tensor ids
    start at 1000 * seed, so no two sets share a table even where the allocator hands a set the
    addresses of an earlier one (the device copy of an identical table would be launched from,
    correctly, and the upload counts below would not show the first upload)."""

    def __init__(self, seed, sizes=SIZES, storage=orc.STORE_P4, bits=4):
        self.rng = np.random.default_rng(seed)
        self.id0 = 1000 * seed
        self.cases = [Case(n, B, storage, self.rng) for n in sizes]
        self.bits = bits
        self.tg = [torch.zeros(c.n, dtype=torch.float32, device=DEV) for c in self.cases]

    def step(self, steps, rounding=orc.ROUND_NEAREST, seed=5, stream=None, tg=None):
        """One launch over the set, the oracle stepped alongside; returns the uploads it made."""
        tg = tg or self.tg
        entries, prevs = [], []
        for i, (c, t, s) in enumerate(zip(self.cases, tg, steps)):
            g, g_dev = c.grads(self.rng)
            t.copy_(g_dev)
            prevs.append(c.p.copy())
            c.oracle_step(g, s, self.bits, rounding=rounding, seed=seed, tensor_id=self.id0 + i)
            entries.append(c.entry(t, s, self.bits, tensor_id=self.id0 + i))
        before = mdq_hip.step_table_uploads()
        mode = "stochastic" if rounding == orc.ROUND_STOCHASTIC else "nearest"
        if stream is None:
            mdq_hip.multi_tensor_step(entries, B, rounding=mode, seed=seed)
        else:
            stream.wait_stream(torch.cuda.current_stream(DEV))   # the grads were filled there
            with torch.cuda.stream(stream):
                mdq_hip.multi_tensor_step(entries, B, rounding=mode, seed=seed)
            stream.synchronize()
        uploads = mdq_hip.step_table_uploads() - before
        for c, p_prev in zip(self.cases, prevs):
            c.check(p_prev)
            resync_params(c.tp, c.p)
        return uploads


@pytest.mark.parametrize("rounding", [orc.ROUND_NEAREST, orc.ROUND_STOCHASTIC])
def test_steady_steps_launch_without_uploads(rounding):
    print(f"case: steady steps 1-6, rounding {rounding}", flush=True)
    s = Set(1 + rounding)
    ups = [s.step([t] * len(SIZES), rounding=rounding) for t in range(1, 7)]
    print(f"uploads per step: {ups}", flush=True)
    assert ups[0] == 1 and ups[1:] == [0] * 5


def test_tensors_at_different_steps_upload_every_call():
    print("case: per-tensor step counts differ", flush=True)
    s = Set(3)
    ups = [s.step([t, t + 3, 2 * t]) for t in range(1, 5)]
    print(f"uploads per step: {ups}", flush=True)
    assert ups == [1, 1, 1, 1]
    # then all equal again: one upload, then none
    ups = [s.step([t] * len(SIZES)) for t in (9, 10, 11)]
    assert ups == [1, 0, 0]


def test_two_sets_alternate():
    print("case: sets A and B alternate on one stream, 8-bit and packed 4-bit", flush=True)
    a = Set(4)
    b = Set(5, sizes=[513, 20_000], storage=orc.STORE_S8, bits=8)
    ups = []
    for t in range(1, 5):
        ups.append(a.step([t] * 3, rounding=orc.ROUND_STOCHASTIC))
        ups.append(b.step([t] * 2))
    print(f"uploads: {ups}", flush=True)
    assert ups[:2] == [1, 1] and ups[2:] == [0] * 6


def test_moved_grad_buffer_and_other_stream_upload():
    print("case: a grad buffer moves; a second stream", flush=True)
    s = Set(6)
    assert s.step([1] * 3) == 1
    assert s.step([2] * 3) == 0
    moved = [torch.zeros_like(t) for t in s.tg]
    assert s.step([3] * 3, tg=moved) == 1
    assert s.step([4] * 3) == 0                 # back to the first buffers: that table is still held
    other = torch.cuda.Stream(DEV)
    assert s.step([5] * 3, stream=other) == 1   # a table held for another stream is not used
    assert s.step([6] * 3, stream=other) == 0
    torch.cuda.current_stream(DEV).wait_stream(other)
    assert s.step([7] * 3) == 0


def test_ring_slots_taken_in_between():
    """Grad statistics and code conversions take ring slots; a step table they overwrite is
    uploaded again, and every step stays exact."""
    print("case: grad_stats / convert_codes between steps", flush=True)
    s = Set(7)
    x = torch.randn(50_000, device=DEV)
    src = torch.randint(0, 256, (4096,), dtype=torch.uint8, device=DEV)
    dst_m = torch.empty(4096, dtype=torch.int8, device=DEV)
    dst_v = torch.empty(4096, dtype=torch.uint8, device=DEV)
    total = 0
    for t in range(1, 13):
        total += s.step([t] * 3)
        for _ in range(t % 3):
            mdq_hip.grad_stats([x])
            mdq_hip.convert_codes([(src, torch.empty(0, dtype=torch.uint8, device=DEV), dst_m, dst_v)])
    torch.cuda.synchronize()
    print(f"uploads over 12 steps: {total}", flush=True)
    assert 1 <= total <= 12


def test_random_sequence_of_launches():
    """A seeded random sequence of 36 launches over three tensor sets (packed 4-bit nearest,
    int8 stochastic, int16 at 12 bits nearest), on two streams, with per-tensor or shared step
    counts, grad buffers that move now and then, and grad statistics / conversions in between:
    every launch exact against the oracle, whatever mix of uploads and device copies it takes."""
    print("case: random sequence of 36 launches", flush=True)
    rng = np.random.default_rng(99)
    sets = [Set(11), Set(12, sizes=[700, 9000], storage=orc.STORE_S8, bits=8),
            Set(13, sizes=[256, 5000, 128], storage=orc.STORE_S16, bits=12)]
    rounding = [orc.ROUND_NEAREST, orc.ROUND_STOCHASTIC, orc.ROUND_NEAREST]
    steps = [0, 0, 0]
    other = torch.cuda.Stream(DEV)
    x = torch.randn(10_000, device=DEV)
    ups = 0
    for op in range(36):
        k = int(rng.integers(0, 3))
        s = sets[k]
        steps[k] += 1
        n = len(s.cases)
        per_tensor = rng.random() < 0.25
        st = [steps[k] + (3 * i if per_tensor else 0) for i in range(n)]
        if rng.random() < 0.15:
            s.tg = [torch.zeros_like(t) for t in s.tg]       # the grads move
        stream = other if rng.random() < 0.3 else None
        if stream is None:
            torch.cuda.current_stream(DEV).wait_stream(other)
        ups += s.step(st, rounding=rounding[k], seed=40 + k, stream=stream)
        if rng.random() < 0.2:
            mdq_hip.grad_stats([x])
    print(f"uploads over 36 launches: {ups}", flush=True)
    assert 3 <= ups < 36
