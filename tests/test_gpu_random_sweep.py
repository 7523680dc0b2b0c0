"""Seeded random sweep of steps that keep their storage, against the oracle.

Each case draws a code storage and width, a block size (1..1024), the rounding mode, the grads'
dtype, an element offset of the params/grads views inside their buffers, one or two tensors per
launch (the by-value one-tensor kernel, through the reference's single-tensor entry point or a
list of one, or the descriptor-table kernel), code arrays aligned or views at the same offset
(the guarded tile mode), and ragged sizes up to a few thousand tiles (several XCD chunks); two
steps each, codes and scales bit-exact and params within the bar after every step, padding
around the views untouched.  The fixed cases elsewhere pin each of these axes alone; this one
crosses them."""
import numpy as np
import pytest

import mdq_hip
from oracle import mdq_oracle as orc
from test_gpu_parity import HP, Case

pytestmark = pytest.mark.gpu

STORAGES = [(orc.STORE_P4, 4), (orc.STORE_S8, 8), (orc.STORE_S8, 4), (orc.STORE_S16, 16), (orc.STORE_S16, 8),
            (orc.STORE_S32, 16), (orc.STORE_S32, 32)]
GRAD_DTYPES = [np.float32, "bf16", np.float16]
OFFSETS = [0, 0, 1, 3, 4, 5, 16, 31, 33]


def _draw(rng, max_tiles):
    storage, bits = STORAGES[rng.integers(len(STORAGES))]
    B = int(2 ** rng.integers(0, 11))
    stochastic = bool(rng.integers(2))     # at 32 bits the step rounds to nearest either way
    gdt = GRAD_DTYPES[rng.integers(len(GRAD_DTYPES))]
    offset = int(rng.choice(OFFSETS))
    tiles = int(np.exp(rng.uniform(0, np.log(max_tiles))))
    sizes = []
    for _ in range(int(rng.integers(1, 3))):
        n = tiles * 512
        if rng.random() < 0.5:
            n += int(rng.integers(-B, B))
        sizes.append(max(1, n))
    codes_aligned = offset == 0 or rng.random() < 0.75   # else the code arrays are views at the offset too
    single_entry = len(sizes) == 1 and rng.random() < 0.5  # the reference's fused_mdq_adamw entry point
    return storage, bits, B, stochastic, gdt, offset, sizes, codes_aligned, single_entry


@pytest.mark.parametrize("seed,n_cases,max_tiles", [(1, 60, 12), (2, 60, 12), (3, 40, 600), (4, 12, 5000),
                                                     (5, 80, 40)])
def test_random_sweep(seed, n_cases, max_tiles):
    rng = np.random.default_rng(seed)
    for case in range(n_cases):
        storage, bits, B, stochastic, gdt, offset, sizes, codes_aligned, single_entry = _draw(rng, max_tiles)
        print(f"case: sweep seed={seed} #{case} storage={storage} bits={bits} B={B} stochastic={stochastic} "
              f"grad={getattr(gdt, '__name__', gdt)} offset={offset} codes_aligned={codes_aligned} sizes={sizes} "
              f"{'fused_mdq_adamw' if single_entry else 'multi_tensor_step'}", flush=True)
        cases = [Case(n, B, storage, rng, grad_dtype=gdt, offset=offset, codes_aligned=codes_aligned, tail=7)
                 for n in sizes]
        rmode = orc.ROUND_STOCHASTIC if stochastic else orc.ROUND_NEAREST
        for step in (1, 2):
            grads = [c.grads(rng) for c in cases]
            prev = [c.p.copy() for c in cases]
            for k, (c, (g, _)) in enumerate(zip(cases, grads)):
                c.oracle_step(g, step, bits, rounding=rmode, seed=seed, tensor_id=k)
            rounding = "stochastic" if stochastic else "nearest"
            if single_entry:
                c, tg = cases[0], grads[0][1]
                mdq_hip.fused_step(c.tp, tg, c.tcm, c.tcv, c.tsm, c.tsv, c.tvm, HP["beta1"], HP["beta2"], HP["lr"],
                                   HP["weight_decay"], HP["eps"], step, bits, B, rounding=rounding, seed=seed,
                                   tensor_id=0)
            else:
                mdq_hip.multi_tensor_step([c.entry(tg, step, bits, tensor_id=k) for k, (c, (_, tg)) in
                                           enumerate(zip(cases, grads))], B, rounding=rounding, seed=seed)
            for c, p_prev in zip(cases, prev):
                c.padding_intact()
                c.check(p_prev)
