"""Sharding at quant-block boundaries keeps the step bit-exact (the one-GPU part of the sharded
design): every tensor cut into `world` block-aligned pieces (mdq_hip.shard_states), one launch per
piece set, must leave p, codes and scales exactly as one launch over the whole tensors does.
Ragged tensors, tensors smaller than world x B (empty pieces), packed and int8 storage, nearest and
stochastic rounding (each piece's elem_offset continues the whole tensor's random stream), block
sizes from 2 (lanes own single elements, pieces start off the 4-element Philox quads) to 1024 (two
waves per block), and the storage-changing step."""
import numpy as np
import pytest
import torch

import mdq_hip
from test_gpu_restore import src_state

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def make(sizes, B, bits, gdt, rng):
    out = []
    for i, n in enumerate(sizes):
        nb = (n + B - 1) // B
        p = torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)).to(DEV)
        g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(DEV).to(gdt)
        if bits == 4:
            cm, cv = torch.full((n,), 8, dtype=torch.uint8, device=DEV), torch.empty(0, dtype=torch.uint8, device=DEV)
        else:
            cm, cv = torch.zeros(n, dtype=torch.int8, device=DEV), torch.zeros(n, dtype=torch.uint8, device=DEV)
        sc = [torch.zeros(nb, device=DEV), torch.zeros(nb, device=DEV), torch.full((nb,), -20.0, device=DEV)]
        out.append(mdq_hip.TensorState(p, g, cm, cv, *sc, 1, bits, 1e-3, 0.9, 0.999, 1e-8, 0.01, i))
    return out


def clone(entries):
    return [mdq_hip.TensorState(e.p.clone(), e.grad, e.exp_avg.clone(), e.exp_avg_sq.clone(), e.scale_m.clone(),
                                e.scale_v.clone(), e.v_min.clone(), e.step, e.bits, e.lr, e.beta1, e.beta2, e.eps,
                                e.weight_decay, e.tensor_id) for e in entries]


def assert_equal_states(whole, parts, sizes, step):
    for i, (a, b) in enumerate(zip(whole, parts)):
        for name in ("p", "exp_avg", "exp_avg_sq", "scale_m", "scale_v", "v_min"):
            x, y = getattr(a, name), getattr(b, name)
            assert torch.equal(x.view(torch.uint8) if x.numel() else x, y.view(torch.uint8) if y.numel() else y), \
                (step, i, sizes[i], name)


@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
@pytest.mark.parametrize("bits,B,gdt", [(4, 128, torch.bfloat16), (8, 64, torch.float32), (4, 256, torch.float32),
                                        (8, 2, torch.float16), (4, 1024, torch.bfloat16)])
@pytest.mark.parametrize("world", [3, 8])
def test_shards_equal_the_whole_launch(bits, B, gdt, world, rounding):
    print(f"case: shards world={world} bits={bits} B={B} grad={gdt} rounding={rounding}", flush=True)
    rng = np.random.default_rng(world * 100 + bits + B)
    sizes = [int(x) for x in np.clip(np.floor(np.exp(rng.uniform(0, np.log(300_000), 19))), 1, None)] + [B * 8 * 40]
    whole = make(sizes, B, bits, gdt, rng)
    parts = clone(whole)
    for step in (1, 2):
        for e in whole + parts:
            e.step = step
        mdq_hip.multi_tensor_step(whole, B, rounding=rounding, seed=11)
        for rank in range(world):
            mine = mdq_hip.shard_states(parts, B, world, rank)
            if mine:
                mdq_hip.multi_tensor_step(mine, B, rounding=rounding, seed=11)
        torch.cuda.synchronize()
        assert_equal_states(whole, parts, sizes, step)


@pytest.mark.parametrize("src,dst", [(2, 0), (0, 1), (1, 3)])
def test_sharded_storage_change_equals_the_whole(src, dst):
    """stq_multi_tensor_mdq_adamw_restore over the pieces (stochastic rounding) equals it over the
    whole tensors; each piece writes its slice of the destination codes."""
    B, world = 128, 3
    print(f"case: sharded restore src={src} dst={dst} B={B} world={world}", flush=True)
    rng = np.random.default_rng(40 + 10 * src + dst)
    bits = {0: 4, 1: 8, 2: 16, 3: 32}[dst]
    sizes = [5000, 129, B * 3 * 7 + 5]
    whole, parts = [], []
    for i, n in enumerate(sizes):
        cm, cv, sm, sv, vm = src_state(src, n, B, rng)
        p = torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)).to(DEV)
        g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(DEV)
        for lst in (whole, parts):
            lst.append(mdq_hip.TensorState(p.clone(), g, cm.to(DEV), cv.to(DEV),
                                           *(torch.from_numpy(a.copy()).to(DEV) for a in (sm, sv, vm)),
                                           3, bits, 1e-3, 0.9, 0.999, 1e-8, 0.01, i))
    outs_w = [mdq_hip.empty_codes(e.p, dst) for e in whole]
    outs_p = [mdq_hip.empty_codes(e.p, dst) for e in parts]
    mdq_hip.multi_tensor_restore(whole, outs_w, B, rounding="stochastic", seed=5)
    for rank in range(world):
        mine = mdq_hip.shard_states(parts, B, world, rank)
        outs = []
        for e, (om, ov) in zip(parts, outs_p):
            s, t = mdq_hip.block_aligned_ranges(e.p.numel(), B, world)[rank]
            if s < t:
                outs.append((om[s:t], ov if ov.numel() == 0 else ov[s:t]))
        if mine:
            mdq_hip.multi_tensor_restore(mine, outs, B, rounding="stochastic", seed=5)
    torch.cuda.synchronize()
    for i, ((wm, wv), (pm, pv)) in enumerate(zip(outs_w, outs_p)):
        assert torch.equal(wm.view(torch.uint8), pm.view(torch.uint8)), (i, "m codes")
        assert torch.equal(wv.view(torch.uint8), pv.view(torch.uint8)), (i, "v codes")
    assert_equal_states(whole, parts, sizes, 3)          # p, scales (and the unchanged source codes)
