"""Edge inputs of the step against the oracle, through the C ABI, in both rounding modes:

- empty tensors at the start, in the middle and at the end of a multi-tensor list;
- beta1 = 0 (m is this step's grad) and beta2 = 0 (v is its square);
- eps = 0 (grads nonzero, so v > 0 and no 0 / 0);
- a step count of one million (both bias corrections are 1 in fp32);
- lr = 0 with weight decay (the params stay as they are; the codes still move);
- one-element tensors and a tensor of exactly one quant block.

Bar as in test_gpu_parity.py: codes and scales bit-exact, params within 1e-6."""
import numpy as np
import pytest

import mdq_hip
from oracle import mdq_oracle as orc
from test_gpu_parity import Case

pytestmark = pytest.mark.gpu
ROUNDINGS = [orc.ROUND_NEAREST, orc.ROUND_STOCHASTIC]


def _run(cases, steps, hps, rounding, bits, B, seed=17):
    mode = "stochastic" if rounding == orc.ROUND_STOCHASTIC else "nearest"
    for rep in range(2):
        entries, prevs = [], []
        for i, (c, st, hp) in enumerate(zip(cases, steps, hps)):
            g, tg = c.grads(np.random.default_rng(1000 * rep + i))
            prevs.append(c.p.copy())
            c.oracle_step(g, st + rep, bits, rounding=rounding, seed=seed, tensor_id=i, **hp)
            entries.append(c.entry(tg, st + rep, bits, tensor_id=i, **hp))
        mdq_hip.multi_tensor_step(entries, B, rounding=mode, seed=seed)
        for c, p_prev in zip(cases, prevs):
            if c.n:
                c.check(p_prev)


@pytest.mark.parametrize("rounding", ROUNDINGS)
def test_empty_tensors_inside_a_list(rounding):
    print(f"case: empty tensors in the list, rounding {rounding}", flush=True)
    rng = np.random.default_rng(5)
    sizes = [0, 1000, 0, 0, 4096, 1, 0]
    cases = [Case(n, 128, orc.STORE_P4, rng) for n in sizes]
    _run(cases, [3] * len(sizes), [{}] * len(sizes), rounding, 4, 128)


@pytest.mark.parametrize("rounding", ROUNDINGS)
@pytest.mark.parametrize("storage,bits", [(orc.STORE_P4, 4), (orc.STORE_S8, 8), (orc.STORE_S16, 12)])
def test_edge_hyper_parameters(storage, bits, rounding):
    print(f"case: edge hyper-parameters storage={storage} bits={bits} rounding={rounding}", flush=True)
    rng = np.random.default_rng(6 + bits)
    hps = [dict(beta1=0.0), dict(beta2=0.0), dict(eps=0.0), dict(), dict(lr=0.0, weight_decay=0.1),
           dict(beta1=0.0, beta2=0.0, eps=0.0)]
    steps = [1, 4, 2, 10 ** 6, 7, 1]
    sizes = [3000, 128, 777, 5000, 1000, 1]
    cases = [Case(n, 128, storage, rng) for n in sizes]
    before = cases[4].p.copy()
    _run(cases, steps, hps, rounding, bits, 128)
    assert np.array_equal(cases[4].p, before)            # lr = 0: the oracle leaves p as it was


@pytest.mark.parametrize("B", [64, 128, 1024])
def test_stochastic_stream_across_the_2_32_quad_boundary(B):
    """Pieces whose stochastic-rounding stream starts just below, at and above element 2^34 (quad
    index 2^32), as a shard of a tensor that large would: the tiles that straddle quad 2^32 draw
    with a per-lane high counter word, the others with a wave-uniform one; every code bit-exact."""
    print(f"case: stochastic stream around quad 2^32, B={B}", flush=True)
    rng = np.random.default_rng(B)
    n = 3 * 1024 + 77
    for origin in (2 ** 34 - 2048, 2 ** 34 - B, 2 ** 34, 2 ** 35 - 1024):
        c = Case(n, B, orc.STORE_P4, rng)
        for step in (1, 2):
            g, tg = c.grads(rng)
            p_prev = c.p.copy()
            c.oracle_step(g, step, 4, rounding=orc.ROUND_STOCHASTIC, seed=5, tensor_id=9, elem_offset=origin)
            e = c.entry(tg, step, 4, tensor_id=9)
            e.elem_offset = origin
            mdq_hip.multi_tensor_step([e], B, rounding="stochastic", seed=5)
            c.check(p_prev)
