"""GPT-2 pretraining with the fused 4-bit optimizer on the GPU: stochastic
rounding against nearest rounding (the reference's arithmetic, bit-exact to the oracle per
tests/test_gpu_optimizer.py) on identical seeded batches, on a 2-layer model and at the config's
stated size (the ``test_config3_*`` tests at the end).

- uniform tokens over the full vocabulary (the config's data): loss curves within 1 %;
- tokens from the first 256 ids (a learnable unigram task whose loss floor is log 256): every
  optimizer brings the loss from log 50257 + (excess of the random init) to within 0.25 nats of
  the floor, and the 4-bit runs end within 2 % of fp32 AdamW's final loss;
- the MDQ score-based bit schedule (bits change on update steps) with the storage-changing kernel
  and with separate conversion passes: the same loss curve (up to the run-to-run variation of
  autograd's atomic accumulations)."""
import math

import numpy as np
import pytest
import torch

import gpt2_pretrain as gp

pytestmark = pytest.mark.gpu
SMALL = dict(n_layer=2, n_embd=128, n_head=4, seq_len=128, batch=4)


def _run(name, rounding, steps, **kw):
    print(f"case: gpt2 {name} {rounding} {kw}", flush=True)
    return gp.train(name, steps=steps, rounding=rounding, **SMALL, **kw)


def test_uniform_tokens_stochastic_vs_nearest_within_1pct():
    a = _run("MDQAdamW-Simple-FusedIO", "stochastic", 40, lr=1e-3)
    b = _run("MDQAdamW-Simple-FusedIO", "nearest", 40, lr=1e-3)
    gap = gp.compare_loss_curves(a["History"]["loss"], b["History"]["loss"], window=1)
    print(f"uniform: max per-step gap {gap:.2e}", flush=True)
    assert gap <= 0.01
    assert a["Avg_FusedIO_FastPath_Ratio"] > 0.9 and a["Avg_MDQ_FusedKernel_ms"] > 0
    assert a["Optimizer_State_GB"] < 0.2 * (4 * 2 * a["Params"] / 2 ** 30)


def test_learnable_tokens_all_optimizers_learn():
    runs = {k: _run(n, r, 60, lr=2e-3, vocab_used=256)
            for k, (n, r) in {"sr": ("MDQAdamW-Simple-FusedIO", "stochastic"),
                              "rn": ("MDQAdamW-Simple", "nearest"),
                              "adamw": ("AdamW-32bit", "nearest")}.items()}
    first = {k: v["History"]["loss"][0] for k, v in runs.items()}
    last = {k: sum(v["History"]["loss"][-5:]) / 5 for k, v in runs.items()}
    print(f"learnable: first {first} last {last} (log 256 = {math.log(256):.3f})", flush=True)
    floor = math.log(256)
    for k in runs:
        assert first[k] > floor + 5.0 and last[k] < floor + 0.25, k
    for k in ("sr", "rn"):
        assert abs(last[k] - last["adamw"]) <= 0.02 * last["adamw"], k
    assert gp.compare_loss_curves(runs["sr"]["History"]["loss"], runs["rn"]["History"]["loss"], 5) <= 0.05


def test_default_schedule_fused_transitions_match_separate_passes():
    kw = dict(bits=None, lr=1e-3, vocab_used=256)
    a = _run("MDQAdamW-Simple-FusedIO", "nearest", 24, fused_transitions=True, **kw)
    b = _run("MDQAdamW-Simple-FusedIO", "nearest", 24, fused_transitions=False, **kw)
    fa, fb = a["History"]["mdq_fused_io_fallback_params"], b["History"]["mdq_fused_io_fallback_params"]
    print(f"tensors changing storage per step: {fa}", flush=True)
    # step 1 moves every tensor not scored at 16 bits out of the initial int16 storage
    assert 0 < fa[0] <= a["Params_Tensors"] and sum(x > 0 for x in fa) >= 2
    gap = gp.compare_loss_curves(a["History"]["loss"], b["History"]["loss"], window=1)
    print(f"default schedule: max per-step loss gap fused vs separate {gap:.2e}", flush=True)
    assert gap <= 2e-3


# BASELINE config 3 at its stated size: GPT-2 small (12 layers, 768 wide, 124M params), seq 1024,
# micro-batch 8, bf16 autocast, fused 4-bit AdamW (B = 128), 300 steps; the reference's training and
# timing loop is /root/reference/CUDA/Cfinetuning_timetest.py:359-501.
FULL = dict(n_layer=12, n_embd=768, n_head=12, seq_len=1024, batch=8)


def _run_full(name, rounding, **kw):
    print(f"case: gpt2 small (config 3 size) {name} {rounding} {kw}", flush=True)
    return gp.train(name, steps=300, rounding=rounding, log_every=100, **FULL, **kw)


def test_config3_uniform_tokens_stochastic_vs_nearest():
    """The config's data (tokens uniform over the 50257-token vocabulary): the stochastic-rounding
    loss curve within 1 % of the nearest-rounding one (the reference's arithmetic) at every step."""
    a = _run_full("MDQAdamW-Simple-FusedIO", "stochastic")
    b = _run_full("MDQAdamW-Simple-FusedIO", "nearest")
    gap = gp.compare_loss_curves(a["History"]["loss"], b["History"]["loss"], window=1)
    print(f"config 3 uniform: max per-step loss gap SR vs nearest {gap:.2e}; optimizer "
          f"{a['Avg_OptimizerStep_ms']:.2f} ms of a {a['Avg_Step_Wall_ms']:.1f} ms step "
          f"({100 * a['Optimizer_Share_of_Step']:.1f} %), state {a['Optimizer_State_GB']:.3f} GB", flush=True)
    assert a["Params"] == 124_439_808 and len(a["History"]["loss"]) == 300
    assert gap <= 0.01
    assert a["Avg_FusedIO_FastPath_Ratio"] > 0.99


def test_config3_learnable_tokens_stochastic_vs_nearest_vs_adamw():
    """Tokens from the first 256 ids: a unigram task the model learns (the loss falls from about
    log 50257 towards log 256), so the curves move and a biased rounding would show.

    While the loss falls steeply (steps 10-80), the 4-bit runs trail fp32 AdamW, nearest more
    than stochastic rounding: nearest rounds the many small m entries of a block to 0, and
    stochastic rounding keeps them in expectation.  Measured: stochastic ahead of nearest by up
    to 4 % at a step there.  The bars: the mean per-step gap between stochastic and nearest
    within 1 %; from step 100 on, where the loss still moves but no longer steeply (from about
    5.60 down to 5.55), the stochastic curve within 1 % of the nearest one and of AdamW's at
    every step; final losses (last 50 steps) within 1 % of each other and of AdamW; and the
    stochastic curve no farther from AdamW's (sum of losses) than the nearest one."""
    runs = {k: _run_full(n, r, vocab_used=256)
            for k, (n, r) in {"sr": ("MDQAdamW-Simple-FusedIO", "stochastic"),
                              "rn": ("MDQAdamW-Simple-FusedIO", "nearest"),
                              "adamw": ("AdamW-32bit", "nearest")}.items()}
    loss = {k: np.asarray(v["History"]["loss"], np.float64) for k, v in runs.items()}
    first = {k: float(v[0]) for k, v in loss.items()}
    final = {k: float(v[-50:].mean()) for k, v in loss.items()}
    rel = np.abs(loss["sr"] - loss["rn"]) / loss["rn"]
    rel_adamw = np.abs(loss["sr"] - loss["adamw"]) / loss["adamw"]
    late = slice(99, None)                               # steps 100 .. 300
    area = {k: abs(loss[k].sum() - loss["adamw"].sum()) / loss["adamw"].sum() for k in ("sr", "rn")}
    print(f"config 3 learnable: first {first} final (last 50) {final} (log 256 = {math.log(256):.3f}); "
          f"SR vs nearest per-step gap mean {rel.mean():.2e} max {rel.max():.2e} (step {int(rel.argmax()) + 1}); "
          f"summed-loss gap to AdamW: SR {area['sr']:.2e}, nearest {area['rn']:.2e}; steps 100-300: SR vs nearest "
          f"max {rel[late].max():.2e}, SR vs AdamW max {rel_adamw[late].max():.2e}, loss moving "
          f"{loss['sr'][99]:.4f} -> {loss['sr'][-1]:.4f}", flush=True)
    for k in loss:
        assert first[k] > math.log(256) + 4.0 and final[k] < first[k] - 4.0, k
    assert len(set(first.values())) == 1                 # same init and data
    assert rel.mean() <= 0.01
    assert rel[late].max() <= 0.01 and rel_adamw[late].max() <= 0.01
    assert abs(final["sr"] - final["rn"]) <= 0.01 * final["rn"]
    for k in ("sr", "rn"):
        assert abs(final[k] - final["adamw"]) <= 0.01 * final["adamw"], k
    assert area["sr"] <= area["rn"]
