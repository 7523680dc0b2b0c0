"""Fused multi-tensor gradient statistics and the vectorised bit decision on the GPU.

- ``mdq_hip.grad_stats`` against the oracle (float64 sums, tests/test_oracle_grad_stats.py)
  within 1e-6 relative, over ragged sizes (tile edges at 16384 and 32768), fp32/bf16/fp16 and
  unaligned views; NaN where torch gives NaN (numel 0 and 1), NaN / inf where NaN / inf grads or
  overflowing squares make them;
- deterministic (bit-identical on repeat), and within 1e-5 of the reference's fp32 torch
  reductions run on the same device;
- ``MDQAdamWSimple._scores`` (one [n] vector) bit-identical to the reference's per-tensor
  0-dim expressions (stquant_opt_simple.py:446-466) on the same stats;
- the optimizer's default MDQ schedule with ``grad_stats="fused"`` picks the same bits and
  produces the same codes as with ``grad_stats="reference"``."""
import numpy as np
import pytest
import torch

import mdq_hip
from oracle import mdq_oracle as orc
from stquant_opt_simple import MDQAdamWSimple

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SIZES = [1, 2, 3, 0, 16383, 16384, 16385, 32767, 32768, 32769, 49153, 100_003, (1 << 20) + 7, 64]


def views(dtype, offset, seed):
    g = torch.Generator().manual_seed(seed)
    flat = (torch.distributions.StudentT(3.0).sample((sum(SIZES) + offset + 8,)) * 1e-3)
    flat[torch.rand(flat.shape, generator=g) < 0.001] *= 1000.0
    flat = flat.to(dtype).to(DEV)
    out, o = [], offset
    for n in SIZES:
        out.append(flat[o:o + n])
        o += n
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("offset", [0, 1])
def test_kernel_matches_oracle(dtype, offset):
    print(f"case: grad_stats {dtype} offset={offset}", flush=True)
    vs = views(dtype, offset, 0)
    got = mdq_hip.grad_stats(vs).cpu().numpy()
    again = mdq_hip.grad_stats(vs).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "not deterministic"
    for i, v in enumerate(vs):
        ref = orc.grad_stats(v.float().cpu().numpy())
        np.testing.assert_allclose(got[i], ref, rtol=1e-6, atol=0, equal_nan=True, err_msg=f"tensor {i} n={v.numel()}")
        if v.numel() >= 2:
            tr = MDQAdamWSimple._compute_grad_stats(v.float()).cpu().numpy()
            np.testing.assert_allclose(got[i], tr, rtol=1e-5, atol=0, err_msg=f"torch, tensor {i}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_nonfinite_grads_match_oracle(dtype):
    """NaN, +-inf and (fp32) overflowing squares in some tensors of a launch: the kernel gives the
    oracle's NaN / inf entries (pinned to the reference's torch expression on the CPU), finite
    entries within 1e-6, and the tensors without such values are unaffected."""
    print(f"case: grad_stats non-finite {dtype}", flush=True)
    vs = [v.clone() for v in views(dtype, 0, 3)]
    vs[4][100] = float("nan")
    vs[5][7] = float("inf")
    vs[6][3], vs[6][9] = float("inf"), float("-inf")
    vs[10][50] = float("-inf")
    if dtype == torch.float32:
        vs[11][2] = 3e38
    got = mdq_hip.grad_stats(vs).cpu().numpy()
    for i, v in enumerate(vs):
        ref = orc.grad_stats(v.float().cpu().numpy())
        assert np.array_equal(np.isnan(got[i]), np.isnan(ref)) and np.array_equal(np.isinf(got[i]), np.isinf(ref)), \
            (i, got[i], ref)
        fin = np.isfinite(ref)
        np.testing.assert_allclose(got[i][fin], ref[fin], rtol=1e-6, atol=0, err_msg=f"tensor {i}")


def test_mixed_dtypes_scatter_back():
    a = views(torch.float32, 0, 1)[4:7]
    b = views(torch.bfloat16, 0, 2)[4:7]
    mixed = [a[0], b[0], a[1], b[1], a[2], b[2]]
    got = mdq_hip.grad_stats(mixed).cpu().numpy()
    for i, v in enumerate(mixed):
        np.testing.assert_allclose(got[i], orc.grad_stats(v.float().cpu().numpy()), rtol=1e-6)


def test_rejects_bad_arguments():
    with pytest.raises(RuntimeError):
        mdq_hip.grad_stats([torch.zeros(4)])                       # CPU tensor
    with pytest.raises(RuntimeError):
        mdq_hip.grad_stats([torch.zeros(4, dtype=torch.int32, device=DEV)])


def test_vectorised_score_is_the_reference_expression():
    params = [torch.nn.Parameter(torch.zeros(8, device=DEV)) for _ in range(37)]
    opt = MDQAdamWSimple(params, layer_count=12, batch_size=8)
    g = torch.Generator(device=DEV).manual_seed(3)
    stats = torch.rand(37, 3, device=DEV, generator=g) * 1e-3 + 1e-5
    opt.n_ema, opt.r_ema, opt.v_global_ema = stats.mean(0).unbind(0)
    tau = opt.param_groups[0]["tau"]
    steps = [int(s) for s in np.random.default_rng(0).integers(1, 5000, 37)]
    vec = opt._scores(stats, steps, tau)
    for i in range(37):
        n_l, r_l, v_l = stats[i]
        s_t = 1.0 + (1.0 / torch.cosh(torch.tensor(steps[i] / tau, device=DEV, dtype=torch.float32)))
        ref = (7.2 + torch.log2(r_l / (opt.r_ema + 1e-12)) + torch.log2(n_l / (opt.n_ema + 1e-12))
               + torch.log2(s_t) + torch.log2(v_l / (opt.v_global_ema + 1e-12)))
        assert torch.equal(vec[i].view(torch.int32), ref.view(torch.int32)), i
        assert opt._score_to_bits(float(vec[i].item())) == opt._score_to_bits(ref)


def test_optimizer_fused_stats_same_decisions():
    print("case: optimizer grad_stats fused vs reference", flush=True)
    shapes = [(700, 13), (4096,), (129,), (3, 1000), (50_000,)]
    gen = torch.Generator().manual_seed(9)
    init = [torch.randn(*s, generator=gen) * 0.02 for s in shapes]
    pa = [torch.nn.Parameter(t.clone().to(DEV)) for t in init]
    pb = [torch.nn.Parameter(t.clone().to(DEV)) for t in init]
    oa = MDQAdamWSimple(pa, block_size=128, update_freq=2, grad_stats="fused")
    ob = MDQAdamWSimple(pb, block_size=128, update_freq=2, grad_stats="reference")
    for t in range(1, 9):
        gg = torch.Generator().manual_seed(100 + t)
        for a, b in zip(pa, pb):
            scale = 1e-3 * (1 + 10 * (t % 3))
            a.grad = (torch.randn(a.shape, generator=gg) * scale).to(DEV)
            b.grad = a.grad.clone()
        oa.step()
        ob.step()
        for a, b in zip(pa, pb):
            sa, sb = oa.state[a], ob.state[b]
            assert sa["current_bit"] == sb["current_bit"], (t, sa["current_bit"], sb["current_bit"])
            assert abs(float(sa["last_score"]) - float(sb["last_score"])) < 1e-4
            assert torch.equal(sa["exp_avg"], sb["exp_avg"]) and torch.equal(sa["scale_m"], sb["scale_m"])
        lt = oa.get_last_step_timings()
        assert lt["mdq_update_decision"] == (t % 2 == 0 or t < 5)
    bits = {oa.state[p]["current_bit"] for p in pa}
    print(f"bits chosen: {sorted(bits)}", flush=True)
