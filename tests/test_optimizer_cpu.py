"""Host logic of the drop-in optimizers on CPU tensors.

The fused kernel needs a GPU, so these tests swap the kernel call
(``_run_kernels``) for the CPU oracle on the same state tensors; everything
else -- state init (stquant_opt_simple.py:212-225), the MDQ bit decision
(:93-109, :427-482), storage alignment / packing on bit changes (:114-210),
FusedIO's fast path and double step increment (stquant_opt_fused_io.py:39-54),
timing keys and state_dict -- runs as shipped.
"""
import io

import numpy as np
import pytest
import torch

from oracle import mdq_oracle as orc
from stquant_opt_fused_io import MDQAdamWSimpleFusedIO
from stquant_opt_simple import MDQAdamWSimple


def _np(t):
    if t.dtype == torch.uint16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.uint32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.numpy()


def oracle_run_kernels(self, items):
    for p, group in items:
        st = self.state[p]
        ea, easq = st["exp_avg"], st["exp_avg_sq"]
        bits = int(st["current_bit"])
        if bits == 4 and ea.dtype == torch.uint8 and easq.numel() == 0:
            storage, cv = orc.STORE_P4, None
        else:
            storage = {torch.int8: orc.STORE_S8, torch.int16: orc.STORE_S16, torch.int32: orc.STORE_S32}[ea.dtype]
            cv = _np(easq.view(-1))
        b1, b2 = group["betas"]
        orc.step(_np(p.data.view(-1)), _np(p.grad.view(-1)), _np(ea.view(-1)), cv,
                 _np(st["scale_m"]), _np(st["scale_v"]), _np(st["v_min"]),
                 beta1=b1, beta2=b2, lr=group["lr"], weight_decay=group["weight_decay"], eps=group["eps"],
                 step=st["step"], bits=bits, block_size=min(int(group["block_size"]), 1024), storage=storage,
                 rounding=0 if group.get("rounding", "nearest") == "nearest" else 1,
                 seed=int(group.get("seed", 0)), tensor_id=self._tensor_ids.get(p, 0))


class SimpleCPU(MDQAdamWSimple):
    _run_kernels = oracle_run_kernels


class FusedIOCPU(MDQAdamWSimpleFusedIO):
    _run_kernels = oracle_run_kernels


def make_params(shapes, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.nn.Parameter(torch.randn(*s, generator=g) * 0.02) for s in shapes]


def set_grads(params, seed):
    g = torch.Generator().manual_seed(seed)
    for p in params:
        p.grad = torch.randn(p.shape, generator=g) * 1e-3


def test_fixed_4bit_matches_direct_packed_run():
    """bits=4 through the optimizer == the packed-4 kernel stepped directly from a fresh state
    (the first step goes int16 -> int8/uint8 kernel -> nibbles, as the reference does)."""
    shapes = [(300, 7), (128,), (1000,)]
    params = make_params(shapes)
    ref = [p.detach().clone().view(-1).numpy() for p in params]
    states = [orc.init_state(r.size, 128, orc.STORE_P4) for r in ref]
    opt = SimpleCPU(params, bits=4, block_size=128)
    for t in range(1, 6):
        set_grads(params, t)
        opt.step()
        for r, s, p in zip(ref, states, params):
            orc.step(r, p.grad.view(-1).numpy().copy(), s[0], None, s[2], s[3], s[4], beta1=0.9, beta2=0.999,
                     lr=1e-3, weight_decay=0.01, eps=1e-8, step=t, bits=4, block_size=128, storage=orc.STORE_P4)
    for r, s, p in zip(ref, states, params):
        st = opt.state[p]
        assert st["exp_avg"].dtype == torch.uint8 and st["exp_avg_sq"].numel() == 0
        assert np.array_equal(st["exp_avg"].view(-1).numpy(), s[0])
        for k, a in (("scale_m", s[2]), ("scale_v", s[3]), ("v_min", s[4])):
            assert np.array_equal(st[k].numpy().view(np.uint32), a.view(np.uint32))
        assert np.array_equal(p.detach().view(-1).numpy(), r)
        assert st["step"] == 5


def test_default_schedule_first_step_picks_8_bits():
    # single tensor, step 1: score = 7.2 + 0 + 0 + log2(1 + 1/cosh(1/tau)) + 0 ~ 8.2 -> 8 bits
    params = make_params([(512,)])
    opt = SimpleCPU(params)
    set_grads(params, 1)
    opt.step()
    st = opt.state[params[0]]
    assert st["current_bit"] == 8
    assert st["exp_avg"].dtype == torch.int8 and st["exp_avg_sq"].dtype == torch.uint8
    assert abs(float(st["last_score"]) - (7.2 + np.log2(1 + 1 / np.cosh(1 / opt.param_groups[0]["tau"])))) < 1e-5
    lt = opt.get_last_step_timings()
    for key in ("mdq_fused_kernel_ms", "mdq_unpack_ms", "mdq_pack_ms", "mdq_quant_dequant_ms",
                "mdq_grad_stats_ms", "mdq_bit_decision_ms", "mdq_update_decision", "mdq_kernel_dequant_ms"):
        assert key in lt
    assert lt["mdq_update_decision"] is True


def test_update_decision_schedule():
    params = make_params([(64,)])
    opt = SimpleCPU(params, update_freq=3)
    seen = []
    for t in range(1, 8):
        set_grads(params, t)
        opt.step()
        seen.append(opt.get_last_step_timings()["mdq_update_decision"])
    # steps 1-4 always, then every update_freq-th step (stquant_opt_simple.py:407)
    assert seen == [True, True, True, True, False, True, False]


@pytest.mark.parametrize("seq", [(16, 4, 8, 32, 16, 4), (32, 8, 4, 16)])
def test_storage_follows_bit_changes(seq):
    params = make_params([(256,)])
    opt = SimpleCPU(params, bits=seq[0], block_size=64)
    expect = {4: (torch.uint8, 0), 8: (torch.int8, 256), 16: (torch.int16, 256), 32: (torch.int32, 256)}
    for t, b in enumerate(seq, start=1):
        opt.param_groups[0]["bits"] = b
        set_grads(params, t)
        opt.step()
        st = opt.state[params[0]]
        dt, n_sq = expect[b]
        assert st["exp_avg"].dtype == dt and st["exp_avg_sq"].numel() == n_sq
        assert st["current_bit"] == b and st["step"] == t
        if b == 4:
            codes = st["exp_avg"].to(torch.int32)
            assert int(codes.max()) <= 255
        else:
            qm = 2 ** (b - 1)
            assert int(st["exp_avg"].to(torch.int64).min()) >= -qm
            assert int(st["exp_avg"].to(torch.int64).max()) <= qm - 1
            assert int(st["exp_avg_sq"].to(torch.int64).max()) <= 2 ** b - 1


def test_bit_decrease_clamps_codes_and_keeps_scales():
    # stquant_opt_simple.py:166-168: int16 codes -> int8 by clamping, scales untouched (quirk Q4)
    st = {"exp_avg": torch.tensor([300, -300, 5], dtype=torch.int16),
          "exp_avg_sq": torch.tensor([1000, 3, 255], dtype=torch.uint16)}
    MDQAdamWSimple._align_momentum_storage(st, 8)
    assert st["exp_avg"].tolist() == [127, -128, 5] and st["exp_avg"].dtype == torch.int8
    assert st["exp_avg_sq"].tolist() == [255, 3, 255] and st["exp_avg_sq"].dtype == torch.uint8
    MDQAdamWSimple._pack_momentum_storage(st, 4)
    # nibbles: m = clamp(q + 8, 0, 15), v = clamp(q, 0, 15)
    assert st["exp_avg"].tolist() == [15 | (15 << 4), 0 | (3 << 4), 13 | (15 << 4)]
    assert st["exp_avg_sq"].numel() == 0
    MDQAdamWSimple._align_momentum_storage(st, 8)
    assert st["exp_avg"].tolist() == [7, -8, 5] and st["exp_avg_sq"].tolist() == [15, 3, 15]


def test_fused_io_fast_path_and_double_increment():
    params = make_params([(256,), (128,)])
    opt = FusedIOCPU(params, bits=4, block_size=128)
    set_grads(params, 1)
    opt.step()
    lt = opt.get_last_step_timings()
    # first step: int16 state != packed -> fallback, which increments step twice (quirk Q5)
    assert lt["mdq_fused_io_fallback_params"] == 2 and lt["mdq_fused_io_fast_path_params"] == 0
    assert all(opt.state[p]["step"] == 2 for p in params)
    set_grads(params, 2)
    opt.step()
    lt = opt.get_last_step_timings()
    assert lt["mdq_fused_io_fast_path_params"] == 2 and lt["mdq_fused_io_fast_path_ratio"] == 1.0
    assert all(opt.state[p]["step"] == 3 for p in params)


def test_state_dict_round_trip_restores_code_dtypes():
    params = make_params([(256,), (300,)])
    opt = SimpleCPU(params, bits=4, block_size=128)
    for t in (1, 2):
        set_grads(params, t)
        opt.step()
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)              # a checkpoint, as the drivers write it
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    assert "mdq_global_stats" in sd and sd["mdq_global_stats"]["total_steps"] == 2
    params2 = [torch.nn.Parameter(p.detach().clone()) for p in params]
    opt2 = SimpleCPU(params2, bits=4, block_size=128)
    opt2.load_state_dict(sd)
    for p, q in zip(params, params2):
        a, b = opt.state[p], opt2.state[q]
        # torch's Optimizer.load_state_dict would leave these as float32 (quirk Q8)
        assert b["exp_avg"].dtype == torch.uint8 and torch.equal(a["exp_avg"], b["exp_avg"])
        assert b["exp_avg_sq"].dtype == torch.uint8
        assert torch.equal(a["scale_m"], b["scale_m"]) and b["step"] == a["step"]
    assert opt2.total_steps == 2
    # both continue identically
    set_grads(params, 3)
    set_grads(params2, 3)
    opt.step()
    opt2.step()
    for p, q in zip(params, params2):
        assert torch.equal(p.detach(), q.detach())


def test_bit_distribution_getters():
    params = make_params([(100,), (300,)])
    opt = SimpleCPU(params)
    opt.param_groups[0]["bits"] = None
    set_grads(params, 1)
    opt.step()
    d = opt.get_bit_distribution()
    assert abs(sum(d.values()) - 100.0) < 1e-9
    w = opt.get_bit_distribution_param_weighted()
    assert abs(sum(w.values()) - 100.0) < 1e-9
    assert opt.get_avg_bit_param_weighted() in (4.0, 8.0, 16.0, 32.0) or 4 <= opt.get_avg_bit_param_weighted() <= 32
    assert len(opt.get_all_raw_scores()) == 2


def test_rejects_bad_options():
    with pytest.raises(ValueError):
        MDQAdamWSimple(make_params([(4,)]), bits=5)
    with pytest.raises(ValueError):
        MDQAdamWSimple(make_params([(4,)]), rounding="up")
