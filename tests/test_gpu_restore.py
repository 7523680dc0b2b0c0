"""Storage-changing steps (stq_multi_tensor_mdq_adamw_restore) against the separate passes.

When a tensor's bit width changes, MDQAdamWSimple aligns its codes to the new width, runs the
kernel, and packs 4-bit codes into nibbles (stquant_opt_simple.py:231-280, storage rules
:140-210).  The restore kernel does the three in one pass.  Here every (source, destination)
storage pair, at block sizes 64 / 128 / 256, nearest and stochastic rounding and fp32 / bf16 /
fp16 grads, must give exactly what the separate passes give on the GPU: the conversion kernel
(itself bit-exact against the reference's torch restatement, test_gpu_convert.py), the step
kernel (bit-exact against the oracle, test_gpu_parity.py), then the nibble packing.  Codes,
scales and params are compared bit for bit (both routes run the same device arithmetic).  Source
codes span the source type's whole range, so the clamps of the alignment are exercised.

The optimizer then runs bit-width sequences with the fused transitions on and off.
"""
import numpy as np
import pytest
import torch

import mdq_hip
from mdq_hip import storage
from stquant_opt_fused_io import MDQAdamWSimpleFusedIO
from stquant_opt_simple import MDQAdamWSimple
from test_gpu_optimizer import build, grads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
NAMES = {mdq_hip.STORE_P4: "p4", mdq_hip.STORE_S8: "s8", mdq_hip.STORE_S16: "s16", mdq_hip.STORE_S32: "s32"}
BITS = {mdq_hip.STORE_P4: 4, mdq_hip.STORE_S8: 8, mdq_hip.STORE_S16: 16, mdq_hip.STORE_S32: 32}
SIZES = [4096 * 2, 1000, 129, 3 * 777]          # whole tiles, ragged tails, and (last) an unaligned p view
PAIRS = [(s, d) for s in NAMES for d in NAMES if s != d]
GDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def src_state(src, n, B, rng):
    """A state in storage ``src`` as a run at that width leaves it: codes over the full range,
    scale_m = M / 2^(w-1) and scale_v = (Lmax - Lmin) / (2^w - 1) for that width w."""
    w = BITS[src]
    nb = (n + B - 1) // B
    if src == mdq_hip.STORE_P4:
        cm = torch.from_numpy(rng.integers(0, 256, n, dtype=np.uint8))
        cv = torch.empty(0, dtype=torch.uint8)
    else:
        tm, tv = {1: (torch.int8, torch.uint8), 2: (torch.int16, torch.uint16), 3: (torch.int32, torch.uint32)}[src]
        im, iv = torch.iinfo(tm), torch.iinfo(tv)
        # half the codes near zero, half over the type's whole range
        m = np.where(rng.random(n) < 0.5, rng.integers(-20, 20, n), rng.integers(im.min, im.max, n, endpoint=True))
        v = np.where(rng.random(n) < 0.5, rng.integers(0, 20, n), rng.integers(0, iv.max, n, endpoint=True))
        cm = torch.from_numpy(m.astype(np.int64)).to(tm)
        cv = torch.from_numpy(v.astype(np.int64)).to(tv)
    sm = (rng.uniform(0.2, 1.0, nb) * 1e-3 / 2.0 ** (w - 1)).astype(np.float32)
    sv = (rng.uniform(0.5, 1.0, nb) * 28.0 / (2.0 ** w - 1)).astype(np.float32)
    vm = rng.uniform(-30.0, -22.0, nb).astype(np.float32)
    return cm, cv, sm, sv, vm


class Tensors:
    """Device tensors of one call; ``clone()`` gives an independent copy for the other route."""

    def __init__(self, src, B, gdt, seed, sizes=SIZES, offsets=None):
        """``offsets``: per tensor, the element offsets of the p and grad views in their buffers
        (default: p of the last tensor at 1, everything else at 0)."""
        rng = np.random.default_rng(seed)
        if offsets is None:
            offsets = [(1 if k == len(sizes) - 1 else 0, 0) for k in range(len(sizes))]
        self.items = []
        for n, (off, goff) in zip(sizes, offsets):
            cm, cv, sm, sv, vm = src_state(src, n, B, rng)
            pbuf = torch.from_numpy((rng.standard_normal(n + off) * 0.02).astype(np.float32)).to(DEV)
            g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(DEV).to(GDT[gdt])
            if goff:
                gbuf = torch.zeros(n + goff, dtype=g.dtype, device=DEV)
                gbuf[goff:] = g
                g = gbuf[goff:]
            self.items.append([pbuf[off:], g, cm.to(DEV), cv.to(DEV), *(torch.from_numpy(a).to(DEV) for a in (sm, sv, vm))])

    def clone(self):
        c = Tensors.__new__(Tensors)
        c.items = []
        for p, g, cm, cv, sm, sv, vm in self.items:
            pb = torch.empty(p.numel() + p.storage_offset(), dtype=p.dtype, device=DEV)
            pv = pb[p.storage_offset():]
            pv.copy_(p)
            c.items.append([pv, g, cm.clone(), cv.clone(), sm.clone(), sv.clone(), vm.clone()])
        return c

    def entries(self, bits, step):
        return [mdq_hip.TensorState(p, g, cm, cv, sm, sv, vm, step, bits, 2e-3, 0.9, 0.999, 1e-8, 0.01, i)
                for i, (p, g, cm, cv, sm, sv, vm) in enumerate(self.items)]


def separate_passes(t, dst, B, rounding, seed, step):
    """convert to the aligned storage -> step kernel at the new width -> pack nibbles."""
    bits = BITS[dst]
    aligned = storage.kernel_layout(bits)
    moves = []
    for it in t.items:
        if mdq_hip.storage_of(it[2], it[3]) != aligned:
            nm, nv = mdq_hip.empty_codes(it[2], aligned)
            moves.append((it, nm, nv))
    mdq_hip.convert_codes([(it[2], it[3], nm, nv) for it, nm, nv in moves])
    for it, nm, nv in moves:
        it[2], it[3] = nm, nv
    mdq_hip.multi_tensor_step(t.entries(bits, step), B, rounding=rounding, seed=seed)
    if dst == mdq_hip.STORE_P4:
        outs = [mdq_hip.empty_codes(it[2], mdq_hip.STORE_P4) for it in t.items]
        mdq_hip.convert_codes([(it[2], it[3], nm, nv) for it, (nm, nv) in zip(t.items, outs)])
        for it, (nm, nv) in zip(t.items, outs):
            it[2], it[3] = nm, nv


def fused(t, dst, B, rounding, seed, step):
    outs = [mdq_hip.empty_codes(it[2], dst) for it in t.items]
    mdq_hip.multi_tensor_restore(t.entries(BITS[dst], step), outs, B, rounding=rounding, seed=seed)
    for it, (nm, nv) in zip(t.items, outs):
        it[2], it[3] = nm, nv


def assert_same(a, b, tag):
    torch.cuda.synchronize()
    for k, (x, y) in enumerate(zip(a.items, b.items)):
        for name, u, w in zip(("p", "grad", "exp_avg", "exp_avg_sq", "scale_m", "scale_v", "v_min"), x, y):
            assert u.dtype == w.dtype and u.shape == w.shape, (tag, k, name, u.dtype, w.dtype)
            if u.numel() == 0:
                continue
            assert torch.equal(u.cpu().view(torch.uint8), w.cpu().view(torch.uint8)), f"{tag}: tensor {k} {name} differs"


@pytest.mark.parametrize("B", [64, 128, 256])
@pytest.mark.parametrize("src,dst", PAIRS, ids=[f"{NAMES[s]}-{NAMES[d]}" for s, d in PAIRS])
def test_restore_matches_separate_passes(src, dst, B):
    for gdt, rounding in (("f32", "nearest"), ("bf16", "stochastic"), ("f16", "nearest")):
        tag = f"restore {NAMES[src]} -> {NAMES[dst]} B={B} {gdt} {rounding}"
        print(f"case: {tag}", flush=True)
        a = Tensors(src, B, gdt, seed=1000 * src + 100 * dst + B + len(gdt))
        b = a.clone()
        separate_passes(a, dst, B, rounding, 99, step=7)
        fused(b, dst, B, rounding, 99, step=7)
        assert_same(a, b, tag)


@pytest.mark.parametrize("seed", range(6))
def test_restore_random_sweep(seed):
    """Seeded random cases crossing the axes above: storage pair, B, rounding, grad dtype, one to
    three tensors of random sizes (whole tiles and ragged tails), params and grads as views at
    independent element offsets (inside a 128-byte line, 16-byte aligned or not), a random step."""
    rng = np.random.default_rng(500 + seed)
    for case in range(12):
        src, dst = PAIRS[rng.integers(len(PAIRS))]
        B = int(rng.choice([64, 128, 256]))
        rounding = "stochastic" if rng.random() < 0.5 else "nearest"
        gdt = str(rng.choice(list(GDT)))
        k = int(rng.integers(1, 4))
        sizes = [int(rng.integers(1, 40 * 512)) if rng.random() < 0.7 else 512 * int(rng.integers(1, 40))
                 for _ in range(k)]
        offsets = [(int(rng.choice([0, 0, 1, 4, 5, 16, 33])), int(rng.choice([0, 0, 2, 4, 8, 31]))) for _ in range(k)]
        step = int(rng.integers(1, 50))
        tag = (f"restore sweep seed={seed} #{case} {NAMES[src]} -> {NAMES[dst]} B={B} {gdt} {rounding} "
               f"sizes={sizes} offsets={offsets} step={step}")
        print(f"case: {tag}", flush=True)
        a = Tensors(src, B, gdt, seed=10_000 * seed + case, sizes=sizes, offsets=offsets)
        b = a.clone()
        separate_passes(a, dst, B, rounding, 5, step=step)
        fused(b, dst, B, rounding, 5, step=step)
        assert_same(a, b, tag)


@pytest.mark.parametrize("src,dst", [(mdq_hip.STORE_S16, mdq_hip.STORE_P4), (mdq_hip.STORE_S8, mdq_hip.STORE_S16)],
                         ids=["s16-p4", "s8-s16"])
def test_restore_thousands_of_small_tensors(src, dst):
    """1500 tensors of 1 to 3000 elements (log-uniform) changing storage in one launch (a
    1500-entry descriptor table), against the separate passes."""
    print(f"case: restore 1500 tensors {NAMES[src]} -> {NAMES[dst]}", flush=True)
    rng = np.random.default_rng(1500 + src)
    sizes = [int(x) for x in np.floor(np.exp(rng.uniform(0, np.log(3000), 1500)))]
    a = Tensors(src, 128, "bf16", seed=77, sizes=sizes, offsets=[(0, 0)] * len(sizes))
    b = a.clone()
    separate_passes(a, dst, 128, "nearest", 3, step=9)
    fused(b, dst, 128, "nearest", 3, step=9)
    assert_same(a, b, f"restore 1500 tensors {NAMES[src]} -> {NAMES[dst]}")


@pytest.mark.parametrize("cls", [MDQAdamWSimple, MDQAdamWSimpleFusedIO])
@pytest.mark.parametrize("B", [64, 256, 512])
def test_optimizer_fused_transitions_match_separate_passes(cls, B):
    """Bit-width changes 16 -> 4 -> 8 -> 16 -> 4 -> 32 -> 8 -> 4 with the fused transitions on,
    off, and with the codes moved by torch passes on the device (``_device_transitions = False``),
    identical params and grads; B = 512 has no restore kernels (separate passes)."""
    print(f"case: {cls.__name__} fused transitions B={B}", flush=True)
    shapes = [(700, 13), (4096,), (129,), (3, 1000)]
    cpu, gpu = build(shapes, seed=21)
    gpu2 = [torch.nn.Parameter(p.detach().clone()) for p in gpu]
    gpu3 = [torch.nn.Parameter(p.detach().clone()) for p in gpu]
    on, off, tor = (cls(g, bits=4, block_size=B) for g in (gpu, gpu2, gpu3))
    off._fused_transitions = False
    tor._device_transitions = False
    for t, bits in enumerate([4, 8, 16, 4, 32, 8, 4, 4], start=1):
        for o in (on, off, tor):
            o.param_groups[0]["bits"] = bits
        grads(cpu, gpu, 300 + t)
        for a, b, c in zip(gpu, gpu2, gpu3):
            b.grad = a.grad.clone()
            c.grad = a.grad.clone()
        for o in (on, off, tor):
            o.step()
        torch.cuda.synchronize()
        for other, params in ((off, gpu2), (tor, gpu3)):
            for i, (a, b) in enumerate(zip(gpu, params)):
                sa, sb = on.state[a], other.state[b]
                assert sa["step"] == sb["step"] and sa["current_bit"] == sb["current_bit"] == bits
                for k in ("exp_avg", "exp_avg_sq", "scale_m", "scale_v", "v_min"):
                    assert sa[k].dtype == sb[k].dtype and torch.equal(sa[k], sb[k]), (t, bits, i, k)
                assert torch.equal(a.detach(), b.detach()), (t, bits, i)


@pytest.mark.parametrize("src,dst", [(2, 0), (0, 1), (1, 2), (3, 0)],
                         ids=["s16-p4", "p4-s8", "s8-s16", "s32-p4"])
def test_restore_with_nonfinite_grads_matches_separate_passes(src, dst):
    """NaN and +-inf grads (the reference's NaN-skipping reductions, code 0 for a NaN quotient):
    the storage-changing step still equals the separate passes bit for bit."""
    B = 128
    tag = f"restore {NAMES[src]} -> {NAMES[dst]} B={B} non-finite grads"
    print(f"case: {tag}", flush=True)
    a = Tensors(src, B, "f32", seed=77 + 10 * src + dst)
    rng = np.random.default_rng(5)
    for it in a.items:
        g = it[1].clone()
        n = g.numel()
        idx = torch.from_numpy(rng.choice(n, size=max(1, n // 50), replace=False)).to(DEV)
        vals = torch.tensor([float("nan"), float("inf"), float("-inf")], device=DEV)
        g[idx] = vals[torch.arange(idx.numel(), device=DEV) % 3]
        it[1] = g
    b = a.clone()
    separate_passes(a, dst, B, "nearest", 99, step=7)
    fused(b, dst, B, "nearest", 99, step=7)
    assert_same(a, b, tag)
