"""Host logic of the drop-in optimizers on CPU tensors.

The fused kernel needs a GPU, so these tests swap the launch of each
multi-tensor plan for the CPU oracle stepping every planned descriptor row on
the same state tensors; everything else -- the bucketing and plan cache of
``_run_kernels``, the steady-state path, state init (stquant_opt_simple.py:212-225), the MDQ bit decision
(:93-109, :427-482), storage alignment / packing on bit changes (:114-210),
FusedIO's fast path and double step increment (stquant_opt_fused_io.py:39-54),
timing keys and state_dict -- runs as shipped.  (The value map of the storage changes is
pinned against the reference's rules in test_storage_cpu.py.)
"""
import ctypes
import io

import numpy as np
import pytest
import torch

import mdq_hip
from oracle import mdq_oracle as orc
from stquant_opt_fused_io import MDQAdamWSimpleFusedIO
from stquant_opt_simple import MDQAdamWSimple


def _np(t):
    if t.dtype == torch.uint16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.uint32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.numpy()


_NP_DT = {0: np.float32, 1: np.uint16, 2: np.float16, 3: np.uint8, 4: np.int8, 5: np.int16,
          6: np.uint16, 7: np.int32, 8: np.uint32}


def _host_view(ptr, n, dt):
    """numpy view of ``n`` elements at a CPU tensor's address (a planned descriptor pointer)."""
    dt = np.dtype(dt)
    if n == 0 or ptr == 0:
        return np.zeros(0, dt)
    return np.ctypeslib.as_array((ctypes.c_char * (n * dt.itemsize)).from_address(int(ptr))).view(dt)


class OraclePlan(mdq_hip.MultiTensorPlan):
    """The optimizer's real launch plan, executed row by row by the CPU oracle:
    whatever the host code wrote into the ``stq_tensor`` descriptors (pointers,
    sizes, steps, hyper-parameters, bits, tensor ids) is what gets stepped."""

    def run(self, profile_cycles=None):
        gdt, eadt, _ = self.codes
        for r in self.arr:
            n = int(r["numel"])
            p4 = eadt == 3 and int(r["exp_avg_sq_numel"]) == 0
            storage = orc.STORE_P4 if p4 else {4: orc.STORE_S8, 5: orc.STORE_S16, 7: orc.STORE_S32}[eadt]
            dm, dv = orc.STORAGE_DTYPES[storage]
            nb = int(r["scale_m_numel"])
            orc.step(_host_view(r["p"], n, np.float32), _host_view(r["grad"], n, _NP_DT[gdt]),
                     _host_view(r["exp_avg"], n, dm), None if p4 else _host_view(r["exp_avg_sq"], n, dv),
                     _host_view(r["scale_m"], nb, np.float32), _host_view(r["scale_v"], nb, np.float32),
                     _host_view(r["v_min"], nb, np.float32),
                     beta1=float(r["beta1"]), beta2=float(r["beta2"]), lr=float(r["lr"]),
                     weight_decay=float(r["weight_decay"]), eps=float(r["eps"]), step=int(r["step"]),
                     bits=int(r["bits"]), block_size=self.block_size, storage=storage,
                     rounding=self.rounding, seed=self.seed, tensor_id=int(r["tensor_id"]))


class SimpleCPU(MDQAdamWSimple):
    _plan_cls = OraclePlan


class FusedIOCPU(MDQAdamWSimpleFusedIO):
    _plan_cls = OraclePlan


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


class _CountSteady:
    def _steady_step(self, sc):
        ok = super()._steady_step(sc)
        if ok:
            self.__dict__.setdefault("steady_at", []).append(self.total_steps)
        return ok


class SimpleSteady(_CountSteady, SimpleCPU):
    pass


class FusedIOSteady(_CountSteady, FusedIOCPU):
    pass


class SimpleSlow(SimpleCPU):
    def _steady_lookup(self, update_decision):
        return None


class FusedIOSlow(FusedIOCPU):
    def _steady_lookup(self, update_decision):
        return None


def _same_state(oa, ob, pa, pb, tag):
    for a, b in zip(pa, pb):
        assert torch.equal(a.detach(), b.detach()), tag
        sa, sb = oa.state[a], ob.state[b]
        assert sa["step"] == sb["step"] and sa["current_bit"] == sb["current_bit"], tag
        for k in ("exp_avg", "exp_avg_sq", "scale_m", "scale_v", "v_min"):
            assert sa[k].dtype == sb[k].dtype and torch.equal(sa[k], sb[k]), (tag, k)


@pytest.mark.parametrize("fast_cls,slow_cls", [(SimpleSteady, SimpleSlow), (FusedIOSteady, FusedIOSlow)])
def test_steady_path_matches_slow_path(fast_cls, slow_cls):
    """Reusing last step's plans (same tensors, storage, bits) gives byte-identical results
    to rebuilding everything, through lr changes, a non-contiguous grad, a bit-width change,
    a param without grad, scored bit decisions and a checkpoint reload."""
    shapes = [(300, 7), (128,), (1000,), (5, 5)]
    pa, pb = make_params(shapes, seed=4), make_params(shapes, seed=4)

    def groups(ps):
        return [{"params": ps[:2], "lr": 2e-3, "bits": 4}, {"params": ps[2:], "weight_decay": 0.0, "bits": 4}]
    kw = dict(block_size=64, rounding="stochastic", seed=5, update_freq=3)
    oa, ob = fast_cls(groups(pa), **kw), slow_cls(groups(pb), **kw)
    for t in range(1, 19):
        set_grads(pa, 50 + t)
        set_grads(pb, 50 + t)
        if t == 5:                                       # scheduler-style lr change
            for o in (oa, ob):
                o.param_groups[0]["lr"] = 5e-4
        if t == 7:                                       # a non-contiguous grad
            for ps in (pa, pb):
                ps[0].grad = ps[0].grad.t().contiguous().t()
        if t == 9:                                       # bit width change in one group
            for o in (oa, ob):
                o.param_groups[1]["bits"] = 8
        if t == 11:                                      # one param without grad this step
            pa[1].grad = None
            pb[1].grad = None
        if t == 13:                                      # scored bits from here on
            for o in (oa, ob):
                for g in o.param_groups:
                    g["bits"] = None
        if t == 16:                                      # checkpoint round trip
            buf = io.BytesIO()
            torch.save(oa.state_dict(), buf)
            buf.seek(0)
            oa.load_state_dict(torch.load(buf, weights_only=True))
        oa.step()
        ob.step()
        _same_state(oa, ob, pa, pb, f"step {t}")
        lt = oa.get_last_step_timings()
        assert lt["mdq_fused_kernel_ms"] >= 0 and "mdq_quant_dequant_ms" in lt
        if isinstance(oa, FusedIOSteady):
            assert lt["mdq_fused_io_fast_path_params"] + lt["mdq_fused_io_fallback_params"] >= 3
    # slow: 1-2 (first step re-packs int16 -> nibbles), 7 (non-contiguous grad), 9-10 (bits
    # change re-packs), 11-12 (set of params with grads changes), 13 (group config changes),
    # 15 and 18 (scored bit decisions), 16 (reload); steady everywhere else
    assert oa.steady_at == [3, 4, 5, 6, 8, 14, 17], oa.steady_at


def test_mixed_fixed_and_scored_groups():
    """A group with a fixed ``bits`` keeps its width while the other groups are scored, against
    global statistics over every tensor with a grad: the scored tensors get the widths and scores
    they get when the fixed group is scored too (same statistics, same step counts)."""
    shapes = [(300,), (64, 9), (1000,), (37,)]
    runs = []
    for fixed in (False, True):
        params = make_params(shapes, seed=5)
        groups = [{"params": params[:2]}, {"params": params[2:], "bits": 4 if fixed else None}]
        opt = SimpleCPU(groups, block_size=64)
        for t in range(1, 4):
            set_grads(params, 40 + t)
            params[0].grad.mul_(100.0)           # a wide score spread: the scored widths differ
            opt.step()
        runs.append([(opt.state[p]["current_bit"], float(opt.state[p]["last_score"])) for p in params])
    scored_free, scored_mixed = runs[0][:2], runs[1][:2]
    assert scored_mixed == scored_free
    assert [b for b, _s in runs[1][2:]] == [4, 4]
    assert len({b for b, _s in runs[0]}) > 1


@pytest.mark.parametrize("cls,slow_cls", [(SimpleSteady, SimpleSlow), (FusedIOSteady, FusedIOSlow)])
def test_param_data_replaced_between_steps(cls, slow_cls):
    """``p.data = ...`` (as Module.to() does) gives the same Parameter new storage: the next
    step must update the new storage, on the steady path and on the full path, and the result
    equals a run whose params never moved."""
    shapes = [(300, 7), (128,), (1000,)]
    pa, pb = make_params(shapes, seed=8), make_params(shapes, seed=8)
    oa, ob = cls(pa, bits=4, block_size=64), slow_cls(pb, bits=4, block_size=64)
    for t in range(1, 9):
        if t in (4, 6):                       # steady steps follow both moves
            for p in pa:
                old = p.data
                p.data = old.clone()
                old.fill_(123.0)              # the old storage must not be stepped any more
        set_grads(pa, 70 + t)
        set_grads(pb, 70 + t)
        oa.step()
        ob.step()
        for a, b in zip(pa, pb):
            assert torch.equal(a.detach(), b.detach()), f"step {t}"
    assert 4 in oa.steady_at and 6 in oa.steady_at, oa.steady_at


@pytest.mark.parametrize("bits", [4, 8, 16, 32])
def test_checkpoint_keeps_codes_bit_identical(bits):
    """A save / load round trip keeps every code value and dtype, 32-bit codes included (a cast
    through float32 would lose their low bits: up to 2^32 - 1 for v codes)."""
    params = make_params([(256,), (300,)], seed=9)
    opt = SimpleCPU(params, bits=bits, block_size=64)
    for t in (1, 2, 3):
        set_grads(params, 80 + t)
        opt.step()
    for p in params:                          # extreme codes the float32 cast would corrupt
        st = opt.state[p]
        if bits == 32:
            st["exp_avg"][:4] = torch.tensor([2 ** 31 - 1, -2 ** 31, 2 ** 24 + 1, -(2 ** 24) - 1], dtype=torch.int32)
            st["exp_avg_sq"][:3] = torch.tensor([2 ** 32 - 1, 2 ** 31 + 1, 2 ** 24 + 1]).to(torch.uint32)
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    buf.seek(0)
    params2 = [torch.nn.Parameter(p.detach().clone()) for p in params]
    opt2 = SimpleCPU(params2, bits=bits, block_size=64)
    opt2.load_state_dict(torch.load(buf, weights_only=True))
    for p, q in zip(params, params2):
        a, b = opt.state[p], opt2.state[q]
        for k in ("exp_avg", "exp_avg_sq"):
            assert b[k].dtype == a[k].dtype
            assert torch.equal(b[k].to(torch.int64), a[k].to(torch.int64)), k
    set_grads(params, 90)
    set_grads(params2, 90)
    opt.step()
    opt2.step()
    for p, q in zip(params, params2):
        assert torch.equal(p.detach(), q.detach())
