"""Seeded random sweeps of the step kernels against the oracle, through the C ABI.

Each case draws a code storage and a bit width it can hold (any width, not only 4/8/16/32), a
block size 1 .. 2048 (min(B, 1024) is used, as the reference clamps it), a grad dtype, the rounding
mode, 1-3 tensors of ragged sizes (some of them unaligned views), per-tensor AdamW
hyper-parameters (including lr = 0 and wd = 0) and a starting step up to 5000, then runs two
consecutive steps in one multi-tensor launch each.  Codes and all three scale arrays must be
bit-exact after every step, params within the parity bar of test_gpu_parity.py.

The storage-changing step (stq_multi_tensor_mdq_adamw_restore) is swept the same way against the
oracle run as the reference runs a bit-width change (stquant_opt_simple.py:140-280): the old codes
decoded and clamped to the int8 / int16 range of the new width (old scales kept), the oracle step
on those codes, and 4-bit codes packed into nibbles.
"""
import numpy as np
import pytest
import torch

import mdq_hip
from oracle import mdq_oracle as orc
from test_gpu_parity import DEV, Case, assert_bits_equal, assert_params_close
from test_gpu_restore import src_state

pytestmark = pytest.mark.gpu
N_CASES = 96
WIDTH = {orc.STORE_P4: 4, orc.STORE_S8: 8, orc.STORE_S16: 16, orc.STORE_S32: 32}


def draw(k):
    rng = np.random.default_rng(10_000 + k)
    storage = int(rng.choice([orc.STORE_P4, orc.STORE_S8, orc.STORE_S16, orc.STORE_S32]))
    bits = 4 if storage == orc.STORE_P4 else int(rng.integers(1, WIDTH[storage] + 1))
    block = int(2 ** rng.integers(0, 12))                     # 1 .. 2048
    gdt = [np.float32, "bf16", np.float16][int(rng.integers(0, 3))]
    rounding = orc.ROUND_STOCHASTIC if rng.random() < 0.4 else orc.ROUND_NEAREST
    B = min(block, 1024)
    tensors = []
    for _ in range(int(rng.integers(1, 4))):
        n = int(np.clip(np.exp(rng.uniform(0, np.log(40_000))), 1, 40_000))
        if rng.random() < 0.25:
            n = max(B, (n // B) * B)                          # whole blocks
        hp = dict(lr=float(rng.choice([0.0, 1e-4, 1e-3, 3e-2])),
                  weight_decay=float(rng.choice([0.0, 0.01, 0.1])),
                  beta1=float(rng.choice([0.9, 0.8, 0.5])),
                  beta2=float(rng.choice([0.999, 0.99, 0.95])),
                  eps=float(rng.choice([1e-8, 1e-6, 1e-3])))
        tensors.append(dict(n=n, offset=int(rng.random() < 0.2), hp=hp,
                            step=int(rng.choice([1, 2, 7, 100, 5000]))))
    return rng, storage, bits, block, B, gdt, rounding, tensors


@pytest.mark.parametrize("k", range(N_CASES))
def test_random_case_matches_oracle(k):
    rng, storage, bits, block, B, gdt, rounding, tensors = draw(k)
    seed = 77 + k
    print(f"case {k}: storage={storage} bits={bits} block={block} grad={gdt} rounding={rounding} "
          f"tensors={[(t['n'], t['offset'], t['step']) for t in tensors]} "
          f"hp={[tuple(t['hp'].values()) for t in tensors]}", flush=True)
    cases = [Case(t["n"], B, storage, rng, grad_dtype=gdt, offset=t["offset"]) for t in tensors]
    for rep in range(2):
        entries, prevs = [], []
        for i, (c, t) in enumerate(zip(cases, tensors)):
            g, tg = c.grads(rng)
            prevs.append(c.p.copy())
            step = t["step"] + rep
            c.oracle_step(g, step, bits, rounding=rounding, seed=seed, tensor_id=i, **t["hp"])
            entries.append(c.entry(tg, step, bits, tensor_id=i, **t["hp"]))
        mdq_hip.multi_tensor_step(entries, block, rounding="stochastic" if rounding else "nearest", seed=seed)
        for c, p_prev in zip(cases, prevs):
            c.check(p_prev)


N_RESTORE = 48
NP_CODES = {orc.STORE_S8: (np.int8, np.uint8), orc.STORE_S16: (np.int16, np.uint16),
            orc.STORE_S32: (np.int32, np.uint32)}


def host_codes(cm, cv, src):
    """(m, v) of a source state as int64 numpy arrays (P4: m = (b & 15) - 8, v = b >> 4)."""
    if src == orc.STORE_P4:
        b = cm.numpy().astype(np.int64)
        return (b & 15) - 8, b >> 4
    m = cm.numpy().astype(np.int64)
    v = cv.view({orc.STORE_S8: torch.uint8, orc.STORE_S16: torch.int16, orc.STORE_S32: torch.int32}[src])
    v = v.numpy().astype(np.int64) & ((1 << (8 * v.element_size())) - 1)
    return m, v


@pytest.mark.parametrize("k", range(N_RESTORE))
def test_random_restore_matches_oracle(k):
    rng = np.random.default_rng(20_000 + k)
    src, dst = (int(x) for x in rng.choice(4, size=2, replace=False))
    bits = WIDTH[dst]
    aligned = orc.STORE_S8 if bits <= 8 else orc.STORE_S16 if bits <= 16 else orc.STORE_S32
    B = int(rng.choice([64, 128, 256]))
    gdt = [torch.float32, torch.bfloat16, torch.float16][int(rng.integers(0, 3))]
    rounding = orc.ROUND_STOCHASTIC if rng.random() < 0.4 else orc.ROUND_NEAREST
    seed = 500 + k
    sizes = [int(np.clip(np.exp(rng.uniform(0, np.log(30_000))), 1, 30_000)) for _ in range(int(rng.integers(1, 4)))]
    hps = [dict(lr=float(rng.choice([0.0, 1e-3, 3e-2])), weight_decay=float(rng.choice([0.0, 0.01])),
                beta1=float(rng.choice([0.9, 0.5])), beta2=float(rng.choice([0.999, 0.95])),
                eps=float(rng.choice([1e-8, 1e-3]))) for _ in sizes]
    steps = [int(rng.choice([1, 3, 50])) for _ in sizes]
    print(f"case {k}: src={src} dst={dst} bits={bits} B={B} grad={gdt} rounding={rounding} sizes={sizes}",
          flush=True)
    entries, outs, checks = [], [], []
    for i, (n, hp, step) in enumerate(zip(sizes, hps, steps)):
        cm, cv, sm, sv, vm = src_state(src, n, B, rng)
        p = (rng.standard_normal(n) * 0.02).astype(np.float32)
        g32 = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32))
        tg = g32.to(gdt)
        g_host = (tg.view(torch.int16).numpy().view(np.uint16).copy() if gdt == torch.bfloat16
                  else tg.numpy().copy())
        # the reference's route on the host: align (clamp to the aligned storage's range), step, pack
        m, v = host_codes(cm, cv, src)
        lo_m, hi_m = np.iinfo(NP_CODES[aligned][0]).min, np.iinfo(NP_CODES[aligned][0]).max
        am = np.clip(m, lo_m, hi_m).astype(NP_CODES[aligned][0])
        av = np.clip(v, 0, np.iinfo(NP_CODES[aligned][1]).max).astype(NP_CODES[aligned][1])
        hp_, hsm, hsv, hvm = p.copy(), sm.copy(), sv.copy(), vm.copy()
        orc.step(hp_, g_host, am, av, hsm, hsv, hvm, step=step, bits=bits, block_size=B, storage=aligned,
                 rounding=rounding, seed=seed, tensor_id=i, **hp)
        want = ((am.astype(np.int64) + 8) | (av.astype(np.int64) << 4)).astype(np.uint8) if dst == orc.STORE_P4 \
            else (am, av)
        tp = torch.from_numpy(p.copy()).to(DEV)
        ts = [torch.from_numpy(a.copy()).to(DEV) for a in (sm, sv, vm)]
        e = mdq_hip.TensorState(tp, tg.to(DEV), cm.to(DEV), cv.to(DEV), *ts, step, bits, hp["lr"], hp["beta1"],
                                hp["beta2"], hp["eps"], hp["weight_decay"], i)
        out = mdq_hip.empty_codes(tp, dst)
        entries.append(e)
        outs.append(out)
        checks.append((tp, ts, out, want, hp_, (hsm, hsv, hvm), p))
    mdq_hip.multi_tensor_restore(entries, outs, B, rounding="stochastic" if rounding else "nearest", seed=seed)
    torch.cuda.synchronize()
    for i, (tp, ts, (om, ov), want, hp_, hs, p_prev) in enumerate(checks):
        if dst == orc.STORE_P4:
            assert_bits_equal(f"tensor {i} packed codes", om, want)
        else:
            assert_bits_equal(f"tensor {i} m codes", om, want[0])
            assert_bits_equal(f"tensor {i} v codes", ov, want[1])
        for name, t, a in zip(("scale_m", "scale_v", "v_min"), ts, hs):
            assert_bits_equal(f"tensor {i} {name}", t, a)
        assert_params_close(tp, hp_, p_prev)


class WideCase(Case):
    """Grads with magnitudes log-uniform over 1e-30 .. 1e3 (so v spans denormals to 1e6 and
    x = v + 1e-12 straddles the fast v-code path's range), random signs, 10 % of quant blocks
    all zero."""

    def grads(self, rng):
        g = (np.sign(rng.standard_normal(self.n)) * 10.0 ** rng.uniform(-30, 3, self.n)).astype(np.float32)
        nb = (self.n + self.B - 1) // self.B
        for b in np.nonzero(rng.random(nb) < 0.1)[0]:
            g[b * self.B:(b + 1) * self.B] = 0.0
        if self.grad_dtype == "bf16":
            tg = torch.from_numpy(g).to(torch.bfloat16)
            return tg.view(torch.int16).numpy().view(np.uint16).copy(), self._dev_view_t(tg)
        return g, self._dev_view(g)


WIDE = [(orc.STORE_P4, 4, 128, orc.ROUND_NEAREST), (orc.STORE_P4, 4, 64, orc.ROUND_STOCHASTIC),
        (orc.STORE_S8, 8, 256, orc.ROUND_NEAREST), (orc.STORE_S8, 8, 128, orc.ROUND_STOCHASTIC),
        (orc.STORE_S8, 3, 16, orc.ROUND_NEAREST), (orc.STORE_S16, 16, 128, orc.ROUND_NEAREST),
        (orc.STORE_S16, 16, 1024, orc.ROUND_STOCHASTIC), (orc.STORE_S32, 32, 128, orc.ROUND_NEAREST),
        (orc.STORE_S32, 24, 2, orc.ROUND_NEAREST)]


@pytest.mark.parametrize("gdt", [np.float32, "bf16"])
@pytest.mark.parametrize("storage,bits,B,rounding", WIDE)
def test_extreme_gradient_magnitudes(storage, bits, B, rounding, gdt):
    print(f"case: wide grads storage={storage} bits={bits} B={B} rounding={rounding} grad={gdt}", flush=True)
    rng = np.random.default_rng(30_000 + 100 * storage + bits + B)
    c = WideCase(B * 45 + 7, B, storage, rng, grad_dtype=gdt)
    for step in range(1, 5):
        g, tg = c.grads(rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits, rounding=rounding, seed=5, tensor_id=3)
        mdq_hip.multi_tensor_step([c.entry(tg, step, bits, tensor_id=3)], B,
                                  rounding="stochastic" if rounding else "nearest", seed=5)
        c.check(p_prev)
