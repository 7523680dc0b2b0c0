"""Seeded random sweep of steps that keep their storage, against the oracle.

Each case draws a code storage and width, a block size (1..1024), the rounding mode, the grads'
dtype, an element offset of the params/grads views inside their buffers, one or two tensors per
launch (the by-value one-tensor kernel, or the descriptor-table kernel) and ragged sizes up to a
few thousand tiles (several XCD chunks); two steps each, codes and scales bit-exact and params
within the bar after every step, padding around the views untouched.  The fixed cases elsewhere
pin each of these axes alone; this one crosses them."""
import numpy as np
import pytest

import mdq_hip
from oracle import mdq_oracle as orc
from test_gpu_parity import Case

pytestmark = pytest.mark.gpu

STORAGES = [(orc.STORE_P4, 4), (orc.STORE_S8, 8), (orc.STORE_S8, 4), (orc.STORE_S16, 16), (orc.STORE_S16, 8),
            (orc.STORE_S32, 16), (orc.STORE_S32, 32)]
GRAD_DTYPES = [np.float32, "bf16", np.float16]
OFFSETS = [0, 0, 1, 3, 4, 5, 16, 31, 33]


def _draw(rng, max_tiles):
    storage, bits = STORAGES[rng.integers(len(STORAGES))]
    B = int(2 ** rng.integers(0, 11))
    stochastic = bool(rng.integers(2)) and bits <= 16
    gdt = GRAD_DTYPES[rng.integers(len(GRAD_DTYPES))]
    offset = int(rng.choice(OFFSETS))
    tiles = int(np.exp(rng.uniform(0, np.log(max_tiles))))
    sizes = []
    for _ in range(int(rng.integers(1, 3))):
        n = tiles * 512
        if rng.random() < 0.5:
            n += int(rng.integers(-B, B))
        sizes.append(max(1, n))
    return storage, bits, B, stochastic, gdt, offset, sizes


@pytest.mark.parametrize("seed,n_cases,max_tiles", [(1, 60, 12), (2, 60, 12), (3, 40, 600), (4, 12, 5000)])
def test_random_sweep(seed, n_cases, max_tiles):
    rng = np.random.default_rng(seed)
    for case in range(n_cases):
        storage, bits, B, stochastic, gdt, offset, sizes = _draw(rng, max_tiles)
        print(f"case: sweep seed={seed} #{case} storage={storage} bits={bits} B={B} stochastic={stochastic} "
              f"grad={getattr(gdt, '__name__', gdt)} offset={offset} sizes={sizes}", flush=True)
        cases = [Case(n, B, storage, rng, grad_dtype=gdt, offset=offset, codes_aligned=True, tail=7) for n in sizes]
        rmode = orc.ROUND_STOCHASTIC if stochastic else orc.ROUND_NEAREST
        for step in (1, 2):
            grads = [c.grads(rng) for c in cases]
            prev = [c.p.copy() for c in cases]
            for k, (c, (g, _)) in enumerate(zip(cases, grads)):
                c.oracle_step(g, step, bits, rounding=rmode, seed=seed, tensor_id=k)
            mdq_hip.multi_tensor_step([c.entry(tg, step, bits, tensor_id=k) for k, (c, (_, tg)) in
                                       enumerate(zip(cases, grads))], B,
                                      rounding="stochastic" if stochastic else "nearest", seed=seed)
            for c, p_prev in zip(cases, prev):
                c.padding_intact()
                c.check(p_prev)
