"""GPT-2 pretraining on synthetic tokens with the fused MDQ optimizer.

The counterpart of the reference's timing harness (``CUDA/Cfinetuning_timetest.py:340-560``) and
pretraining loop (``baseline/pretrain_gpt.py:214-290``): HF ``GPT2LMHeadModel`` built from a local
``GPT2Config`` (random init, no hub access), bf16 autocast, ``labels=input_ids``, one optimizer
step per micro-batch. Each step records the harness's per-step history (loss, forward/backward/
optimizer-step ms with a device synchronisation around each phase, as
``Cfinetuning_timetest.py:368-390`` does, plus the optimizer's ``get_last_step_timings()`` keys),
and ``train`` returns the harness's summary keys (``Avg_Loss``, ``Avg_OptimizerStep_ms``,
``Avg_MDQ_FusedKernel_ms``, ``Throughput_tokens_per_s`` ... ``Cfinetuning_timetest.py:523-590``).

Tokens are drawn uniformly from the 50257-token vocabulary by a device generator seeded per run,
so two runs with the same seed see identical batches (and identical dropout masks: the optimizers
draw nothing from torch's generators).

Attention runs in fp32 through a registered attention function (``stq_fp32_causal``): bf16
batched products against transposed operands are avoided on this platform, so the scores, softmax
and the product with V are computed in float32 and the result is cast back to the activations'
dtype. The linear layers, the LM head and the loss run under bf16 autocast as in the reference.
Batches carry no padding, so the causal mask is the whole mask.

Usage::

    python gpt2_pretrain.py --optimizer MDQAdamW-Simple-FusedIO --rounding stochastic --steps 300
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

from stquant_opt_fused_io import MDQAdamWSimpleFusedIO  # noqa: E402
from stquant_opt_simple import MDQAdamWSimple  # noqa: E402

VOCAB = 50257
ATTN_NAME = "stq_fp32_causal"
OPTIMIZERS = ("MDQAdamW-Simple-FusedIO", "MDQAdamW-Simple", "AdamW-32bit")

# the MDQ timing keys the harness copies into its history (Cfinetuning_timetest.py:440-478)
MDQ_KEYS = {
    "unpack_ms": "mdq_unpack_ms", "pack_ms": "mdq_pack_ms",
    "mdq_fused_kernel_ms": "mdq_fused_kernel_ms", "mdq_extra_stats_ms": "mdq_extra_stats_ms",
    "mdq_grad_stats_ms": "mdq_grad_stats_ms", "mdq_allreduce_ms": "mdq_allreduce_ms",
    "mdq_score_bits_ms": "mdq_score_bits_ms", "mdq_update_decision": "mdq_update_decision",
    "mdq_kernel_dequant_ms": "mdq_kernel_dequant_ms", "mdq_kernel_adam_mv_ms": "mdq_kernel_adam_mv_ms",
    "mdq_kernel_scale_reduce_ms": "mdq_kernel_scale_reduce_ms",
    "mdq_kernel_quant_ms": "mdq_kernel_quant_ms", "mdq_kernel_update_p_ms": "mdq_kernel_update_p_ms",
}


def fp32_causal_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """Causal softmax attention computed in float32; returns (output [B, T, H, D], None)."""
    if scaling is None:
        scaling = query.size(-1) ** -0.5
    with torch.autocast(device_type=query.device.type, enabled=False):
        q, k, v = query.float(), key.float(), value.float()
        scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scaling
        T, S = scores.shape[-2], scores.shape[-1]
        causal = torch.ones(T, S, dtype=torch.bool, device=scores.device).triu(S - T + 1)
        scores = scores.masked_fill(causal, float("-inf"))
        w = torch.softmax(scores, dim=-1)
        w = torch.nn.functional.dropout(w, p=dropout, training=module.training)
        out = torch.matmul(w, v)
    return out.transpose(1, 2).to(query.dtype), None


def register_attention() -> None:
    from transformers import AttentionInterface
    AttentionInterface.register(ATTN_NAME, fp32_causal_attention)


def build_model(device, n_layer: int = 12, n_embd: int = 768, n_head: int = 12, n_positions: int = 1024,
                seed: int = 42):
    """GPT-2 small by default (124,439,808 params with wte tied to the LM head)."""
    from transformers import GPT2Config, GPT2LMHeadModel
    register_attention()
    torch.manual_seed(seed)
    cfg = GPT2Config(vocab_size=VOCAB, n_positions=n_positions, n_embd=n_embd, n_layer=n_layer,
                     n_head=n_head)
    cfg._attn_implementation = ATTN_NAME
    model = GPT2LMHeadModel(cfg).to(device)
    model.train()
    return model


def build_optimizer(name: str, model, lr: float, layer_count: int, global_batch: int, *, bits=4,
                    block_size: int = 128, rounding: str = "stochastic", seed: int = 0):
    """As ``Cfinetuning_timetest.py:96-200``: the MDQ classes over ``model.parameters()``
    (wd 0.01), torch AdamW for the 32-bit baseline."""
    if name == "AdamW-32bit":
        return torch.optim.AdamW(model.parameters(), lr=lr, weight_decay=0.01)
    cls = {"MDQAdamW-Simple": MDQAdamWSimple, "MDQAdamW-Simple-FusedIO": MDQAdamWSimpleFusedIO}[name]
    return cls(model.parameters(), lr=lr, weight_decay=0.01, layer_count=layer_count,
               batch_size=global_batch, block_size=block_size, bits=bits, rounding=rounding, seed=seed)


def _avg(xs):
    xs = [float(x) for x in xs]
    return sum(xs) / len(xs) if xs else 0.0


def optimizer_state_bytes(opt) -> int:
    """Bytes of device tensors in ``opt.state`` (``Cfinetuning_timetest.py:242-250``)."""
    return sum(v.numel() * v.element_size() for st in opt.state.values() for v in st.values()
               if isinstance(v, torch.Tensor))


def train(optimizer_name: str = "MDQAdamW-Simple-FusedIO", *, steps: int = 300, warmup: int = 0,
          batch: int = 8, seq_len: int = 1024, lr: float = 2e-4, bits=4, block_size: int = 128,
          rounding: str = "stochastic", data_seed: int = 1234, model_seed: int = 42, opt_seed: int = 0,
          n_layer: int = 12, n_embd: int = 768, n_head: int = 12, vocab_used: int = VOCAB,
          device="cuda:0", log_every: int = 0, fused_transitions: bool = True):
    """Run ``warmup`` untimed-history steps then ``steps`` measured steps; return the summary.

    Tokens are uniform over ``[0, vocab_used)`` (the full vocabulary by default; a smaller range
    gives a learnable unigram task whose loss falls towards ``log(vocab_used)``).  ``bits=None``
    runs the MDQ score-based bit schedule; ``fused_transitions=False`` steps tensors whose bit
    width changes with separate conversion passes instead of the storage-changing kernel."""
    dev = torch.device(device)
    model = build_model(dev, n_layer=n_layer, n_embd=n_embd, n_head=n_head, n_positions=seq_len,
                        seed=model_seed)
    opt = build_optimizer(optimizer_name, model, lr, n_layer, batch, bits=bits, block_size=block_size,
                          rounding=rounding, seed=opt_seed)
    is_mdq = optimizer_name.startswith("MDQ")
    if is_mdq:
        opt._fused_transitions = fused_transitions
    gen = torch.Generator(device=dev).manual_seed(data_seed)
    torch.manual_seed(model_seed)
    hist = {k: [] for k in ("loss", "forward_ms", "backward_ms", "step_wall_ms", "optimizer_step_ms")}
    if is_mdq:
        for k in MDQ_KEYS:
            hist[k] = []
        if optimizer_name == "MDQAdamW-Simple-FusedIO":
            hist["mdq_fused_io_fast_path_ratio"] = []
            hist["mdq_fused_io_fallback_params"] = []
    sync = torch.cuda.synchronize
    measure_start = None
    torch.cuda.reset_peak_memory_stats(dev)
    for it in range(warmup + steps):
        if it == warmup:
            sync()
            measure_start = time.perf_counter()
        t_step = time.perf_counter()
        ids = torch.randint(0, vocab_used, (batch, seq_len), device=dev, generator=gen)
        sync()
        t0 = time.perf_counter()
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            out = model(ids, labels=ids)
        sync()
        t1 = time.perf_counter()
        out.loss.backward()
        sync()
        t2 = time.perf_counter()
        opt.step()
        sync()
        t3 = time.perf_counter()
        opt.zero_grad(set_to_none=True)
        if it < warmup:
            continue
        hist["loss"].append(float(out.loss.item()))
        hist["forward_ms"].append((t1 - t0) * 1e3)
        hist["backward_ms"].append((t2 - t1) * 1e3)
        hist["optimizer_step_ms"].append((t3 - t2) * 1e3)
        hist["step_wall_ms"].append((time.perf_counter() - t_step) * 1e3)
        if is_mdq:
            lt = opt.get_last_step_timings()
            for hk, tk in MDQ_KEYS.items():
                hist[hk].append(lt.get(tk, 0.0))
            if "mdq_fused_io_fast_path_ratio" in hist:
                hist["mdq_fused_io_fast_path_ratio"].append(lt.get("mdq_fused_io_fast_path_ratio", 0.0))
                hist["mdq_fused_io_fallback_params"].append(lt.get("mdq_fused_io_fallback_params", 0))
        if log_every and (it - warmup + 1) % log_every == 0:
            print(f"[gpt2] {optimizer_name} step {it - warmup + 1}/{steps} loss {hist['loss'][-1]:.4f} "
                  f"step {hist['step_wall_ms'][-1]:.1f} ms opt {hist['optimizer_step_ms'][-1]:.2f} ms",
                  file=sys.stderr, flush=True)
    sync()
    wall_ms = (time.perf_counter() - measure_start) * 1e3
    n_params = sum(p.numel() for p in model.parameters())
    res = {
        "Opt": optimizer_name,
        "Rounding": rounding if is_mdq else None,
        "Bits": bits if is_mdq else 32,
        "Block_Size": block_size if is_mdq else None,
        "Params": n_params,
        "Params_Tensors": sum(1 for _ in model.parameters()),
        "Avg_Loss": _avg(hist["loss"]),
        "Final_Loss_Avg10": _avg(hist["loss"][-10:]),
        "Measure_Train_Wall_ms": wall_ms,
        "Avg_Step_Wall_ms": _avg(hist["step_wall_ms"]),
        "Throughput_tokens_per_s": steps * batch * seq_len / (wall_ms / 1e3),
        "Peak_GPU_Memory_GB": torch.cuda.max_memory_allocated(dev) / 2 ** 30,
        "Optimizer_State_GB": optimizer_state_bytes(opt) / 2 ** 30,
        "Warmup_Steps": warmup,
        "Measured_Steps": steps,
        "Avg_Forward_ms": _avg(hist["forward_ms"]),
        "Avg_Backward_ms": _avg(hist["backward_ms"]),
        "Avg_OptimizerStep_ms": _avg(hist["optimizer_step_ms"]),
        "Optimizer_Share_of_Step": _avg(hist["optimizer_step_ms"]) / max(_avg(hist["step_wall_ms"]), 1e-9),
    }
    if is_mdq:
        res.update({
            "Avg_Unpack_ms": _avg(hist["unpack_ms"]),
            "Avg_Pack_ms": _avg(hist["pack_ms"]),
            "Avg_MDQ_FusedKernel_ms": _avg(hist["mdq_fused_kernel_ms"]),
            "Avg_Kernel_Dequant_ms": _avg(hist["mdq_kernel_dequant_ms"]),
            "Avg_Kernel_Adam_mv_ms": _avg(hist["mdq_kernel_adam_mv_ms"]),
            "Avg_Kernel_ScaleReduce_ms": _avg(hist["mdq_kernel_scale_reduce_ms"]),
            "Avg_Kernel_Quant_ms": _avg(hist["mdq_kernel_quant_ms"]),
            "Avg_Kernel_UpdateP_ms": _avg(hist["mdq_kernel_update_p_ms"]),
            "Avg_MDQ_Extra_Stats_ms": _avg(hist["mdq_extra_stats_ms"]),
        })
        if "mdq_fused_io_fast_path_ratio" in hist:
            res["Avg_FusedIO_FastPath_Ratio"] = _avg(hist["mdq_fused_io_fast_path_ratio"])
        res["Bit_Distribution_Final"] = opt.get_bit_distribution()
        res["Avg_Bits_Param_Weighted_Final"] = opt.get_avg_bit_param_weighted()
    res["History"] = hist
    return res


def compare_loss_curves(a, b, window: int = 10):
    """Max relative gap between two loss histories, each smoothed by a trailing mean of ``window``."""
    import numpy as np
    la, lb = np.asarray(a, np.float64), np.asarray(b, np.float64)
    n = min(la.size, lb.size)
    k = np.ones(window) / window
    sa = np.convolve(la[:n], k, mode="valid")
    sb = np.convolve(lb[:n], k, mode="valid")
    return float(np.max(np.abs(sa - sb) / np.abs(sb)))


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--optimizer", choices=OPTIMIZERS, default="MDQAdamW-Simple-FusedIO")
    ap.add_argument("--rounding", choices=("nearest", "stochastic"), default="stochastic")
    ap.add_argument("--bits", type=int, default=4)
    ap.add_argument("--block-size", type=int, default=128)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=0)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--seq-len", type=int, default=1024)
    ap.add_argument("--lr", type=float, default=2e-4)
    ap.add_argument("--out", default=None, help="write the summary (with history) as JSON here")
    a = ap.parse_args(argv)
    res = train(a.optimizer, steps=a.steps, warmup=a.warmup, batch=a.batch, seq_len=a.seq_len, lr=a.lr,
                bits=a.bits, block_size=a.block_size, rounding=a.rounding, log_every=25)
    if a.out:
        with open(a.out, "w") as f:
            json.dump(res, f, indent=1)
    print(json.dumps({k: v for k, v in res.items() if k != "History"}))


if __name__ == "__main__":
    main()
