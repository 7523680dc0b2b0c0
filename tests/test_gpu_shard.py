"""Sharding at quant-block boundaries keeps the step bit-exact (the one-GPU part of the sharded
design): every tensor cut into `world` block-aligned pieces (mdq_hip.shard_states), one launch per
piece set, must leave p, codes and scales exactly as one launch over the whole tensors does.
Ragged tensors, tensors smaller than world x B (empty pieces), packed and int8 storage."""
import numpy as np
import pytest
import torch

import mdq_hip

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


@pytest.mark.parametrize("bits,B,gdt", [(4, 128, torch.bfloat16), (8, 64, torch.float32), (4, 256, torch.float32)])
@pytest.mark.parametrize("world", [3, 8])
def test_shards_equal_the_whole_launch(bits, B, gdt, world):
    print(f"case: shards world={world} bits={bits} B={B} grad={gdt}", flush=True)
    rng = np.random.default_rng(world * 100 + bits + B)
    sizes = [int(x) for x in np.clip(np.floor(np.exp(rng.uniform(0, np.log(300_000), 19))), 1, None)] + [B * 8 * 40]
    whole = make(sizes, B, bits, gdt, rng)
    parts = clone(whole)
    for step in (1, 2):
        for e in whole + parts:
            e.step = step
        mdq_hip.multi_tensor_step(whole, B)
        for rank in range(world):
            mine = mdq_hip.shard_states(parts, B, world, rank)
            if mine:
                mdq_hip.multi_tensor_step(mine, B)
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(whole, parts)):
            for name in ("p", "exp_avg", "exp_avg_sq", "scale_m", "scale_v", "v_min"):
                x, y = getattr(a, name), getattr(b, name)
                assert torch.equal(x.view(torch.uint8) if x.numel() else x, y.view(torch.uint8) if y.numel() else y), \
                    (step, i, sizes[i], name)
