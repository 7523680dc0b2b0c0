"""MDQAdamWSimple -- drop-in for /root/reference/CUDA/stquant_opt_simple.py on MI355X.

Kept from the reference, because callers and checkpoints depend on it:
- the constructor and param groups, ``step()``;
- the per-param state: ``step``, the ``exp_avg`` / ``exp_avg_sq`` integer codes (packed
  nibbles and an empty ``exp_avg_sq`` at 4 bits), ``scale_m``, ``scale_v``, ``v_min`` per quant
  block, ``current_bit``, ``last_score``;
- the ``state_dict`` extras, the bit-distribution getters and the timing keys.

The machinery underneath is different:
- ``step()`` makes one multi-tensor HIP launch per bucket of tensors, through the C ABI of
  ``libstquant_hip.so`` (``mdq_hip.MultiTensorPlan``). The reference launches once per tensor,
  with a device synchronisation on either side (:242-265).
- Launch plans are cached. A step over the same tensors as the last one only refreshes
  pointers, steps and hyper-parameters (the steady path).
- A tensor whose bit width changed has its codes moved to the new layout (``mdq_hip.storage``)
  inside the step kernel: ``mdq_hip.multi_tensor_restore`` reads the old layout and writes the
  new one in one pass. Block sizes other than 64 / 128 / 256 get one conversion launch before
  the step and one after.
- The MDQ bit decision takes its gradient statistics from one fused launch
  (``mdq_hip.grad_stats``) and reads all scores back to the host once.

Results per element are those of the reference kernel (:246-263 -> stquant_kernel.cu).

New optional param-group keys (the defaults keep the reference's behaviour):
- ``bits``: a fixed code width 4/8/16/32 instead of the score-based choice. Tensors in such
  groups still count in the global gradient statistics that score the other groups.
- ``rounding``: 'nearest' or 'stochastic'.
- ``seed``: the seed of the stochastic-rounding stream.

New constructor options:
- ``sync_timing=False`` skips the device synchronisations that fill the timing dict and the
  kernel phase profile, so ``step()`` issues its work asynchronously on the current stream.
- ``grad_stats`` chooses where the bit decision's statistics come from. ``'fused'`` (the default):
  one fused launch for all tensors, exact to fp64; the tensors whose score lies within
  ``SETTLE_MARGIN`` of a width threshold, and the near-constant ones (spread below
  ``NEAR_CONSTANT_R`` of the mean magnitude, where the reference's fp32 ``torch.std`` loses digits),
  are then scored on the reference's own torch reductions, so the widths are the reference's.
  ``'reference'``: the reference's per-tensor torch reductions for every tensor.  ``'exact'``: the
  fused statistics alone.
"""
from __future__ import annotations

import math
import time
from collections import Counter, OrderedDict

import numpy as np
import torch
import torch.distributed as dist
from torch.optim import Optimizer

import mdq_hip
from mdq_hip import storage as codes

# Timing-dict keys of the reference (stquant_opt_simple.py:392-405, :486-493, :282-316).
_PHASE_KEYS = ("mdq_kernel_dequant_ms", "mdq_kernel_adam_mv_ms", "mdq_kernel_scale_reduce_ms",
               "mdq_kernel_quant_ms", "mdq_kernel_update_p_ms")
_DECISION_KEYS = ("mdq_stats_ms", "mdq_bit_decision_ms", "mdq_grad_stats_ms", "mdq_allreduce_ms",
                  "mdq_score_bits_ms")
_KERNEL_WALL_KEYS = ("quant_dequant_unpack_ms", "quant_dequant_kernel_ms", "quant_dequant_pack_ms")
# score thresholds of the widths above 4 bits, widest first (stquant_opt_simple.py:100-109)
_WIDTH_THRESHOLDS = ((32, 24.0), (16, 12.0), (8, 6.8))
_REPORTED_WIDTHS = (4, 8, 16, 32)


class _PhaseProfile:
    """The kernel's five phase cycle sums (dequant, moments, scale reduction, requant, param
    update) in an int64 device buffer, and their split of a measured kernel wall time
    (the reference's ``profile_cycles``, stquant_opt_simple.py:56-83)."""

    SLOTS = len(_PHASE_KEYS)

    def __init__(self):
        self.buf = None

    def on(self, device) -> torch.Tensor:
        if self.buf is None or self.buf.device != device:
            self.buf = torch.zeros(self.SLOTS, dtype=torch.int64, device=device)
        return self.buf

    def active(self, device):
        """The buffer if it lives on ``device``, else None (profiling off)."""
        buf = self.buf
        return buf if buf is not None and buf.device == device else None

    def cycles(self, device):
        return self.on(device).double().cpu().tolist()

    def split(self, device, wall_ms: float):
        """``wall_ms`` shared out in proportion to the phases' cycles."""
        if wall_ms <= 0:
            return [0.0] * self.SLOTS
        cyc = self.cycles(device)
        total = sum(cyc)
        return [wall_ms * (c / total) for c in cyc] if total > 0 else [0.0] * self.SLOTS


class _Stopwatch:
    """Milliseconds between entry and exit, with a device synchronisation at both ends when
    ``sync`` is set (the reference brackets every timed phase that way)."""

    def __init__(self, device, sync: bool = True):
        self.device, self.sync, self.ms = device, sync, 0.0

    def __enter__(self):
        if self.sync and self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        self._t = time.perf_counter()
        return self

    def __exit__(self, *exc):
        if exc[0] is None and self.sync and self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        self.ms = (time.perf_counter() - self._t) * 1000.0
        return False


class MDQAdamWSimple(Optimizer):
    def __init__(
        self,
        params,
        lr=1e-3,
        betas=(0.9, 0.999),
        eps=1e-8,
        weight_decay=0.01,
        alpha=0.9,
        layer_count=24,
        batch_size=32,
        update_freq=20,
        block_size=256,
        bits=None,
        rounding="nearest",
        seed=0,
        sync_timing=True,
        grad_stats="fused",
    ):
        if bits is not None and int(bits) not in _REPORTED_WIDTHS:
            raise ValueError(f"bits must be one of 4, 8, 16, 32 or None, got {bits}")
        mdq_hip.rounding_code(rounding)
        if grad_stats not in ("fused", "reference", "exact"):
            raise ValueError(f"grad_stats must be 'fused', 'reference' or 'exact', got {grad_stats!r}")
        # the schedule's time constant, stquant_opt_simple.py:33
        tau = 300 * math.log(layer_count) * math.sqrt(batch_size)
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, alpha=alpha,
                                      tau=tau, update_freq=update_freq, block_size=block_size, bits=bits,
                                      rounding=rounding, seed=seed))
        # global EMAs of the bit decision (0-d tensors once the first decision ran)
        self.n_ema = self.r_ema = self.v_global_ema = None
        self.total_steps = 0
        self.last_step_timings = {}
        self.sync_timing = sync_timing
        self.grad_stats = grad_stats
        self._settled = 0                   # rows of the last decision taken from torch's reductions
        self._profile = _PhaseProfile()

    # launch-plan class of ``_run_kernels`` (a test harness substitutes its own executor)
    _plan_cls = mdq_hip.MultiTensorPlan
    # False: layout changes of CUDA tensors run as torch ops per tensor instead of device launches
    _device_transitions = True
    # False: a layout change always takes the separate convert -> step -> convert launches,
    # even where the storage-changing step kernel exists (block sizes 64 / 128 / 256)
    _fused_transitions = True
    _RESTORE_GRAD_DTYPES = (torch.float32, torch.bfloat16, torch.float16)

    def add_param_group(self, param_group):
        self.__dict__["_steady"] = None
        super().add_param_group(param_group)

    def get_last_step_timings(self):
        return dict(self.last_step_timings)

    # ------------------------------------------------------------------
    # bit decision (stquant_opt_simple.py:93-109, :407-482)
    # ------------------------------------------------------------------
    @staticmethod
    def _compute_grad_stats(grad: torch.Tensor) -> torch.Tensor:
        # the reference's fp32 torch expression (stquant_opt_simple.py:93-98); its op order fixes
        # the statistics' rounding and so the widths chosen near a threshold
        n_l = torch.sqrt(torch.mean(grad * grad))
        r_l = torch.std(grad) / (grad.abs().mean() + 1e-12)
        v_l = torch.mean(grad * grad)
        return torch.stack([n_l, r_l, v_l])

    # Scores this close to a width threshold, and tensors whose spread is below this fraction of
    # their mean magnitude (r_l), take the reference's torch statistics in the default mode.  The
    # fused statistics are exact to fp64; torch's fp32 reductions differ from them by less than
    # 1e-4 in the score except for near-constant tensors, where torch.std loses digits (up to
    # ~1e-2 in the score at r_l ~ 1e-5; tests/test_gpu_grad_stats.py).
    SETTLE_MARGIN = 1e-2
    NEAR_CONSTANT_R = 5e-2

    def _all_grad_stats(self, grads, steps=None, tau=None):
        """``[n, 3]`` stats of all grads: one fused launch per grad dtype (``'fused'``, settled on
        the reference's torch reductions near the thresholds, and ``'exact'``), or the reference's
        per-tensor torch reductions (``'reference'``, stquant_opt_simple.py:427-431)."""
        if self.grad_stats != "reference" and grads and grads[0].is_cuda:
            stats = mdq_hip.grad_stats(grads)
            if self.grad_stats == "fused" and steps is not None:
                stats = self._settle(stats, grads, steps, tau)
            return stats
        return torch.stack([self._compute_grad_stats(g.float()) for g in grads])

    def _settle(self, stats, grads, steps, tau):
        """The fused statistics, with the rows of the tensors whose width the fused and the
        reference statistics could decide differently replaced by the reference's torch
        reductions: scores within SETTLE_MARGIN of a threshold (provisional scores against the
        EMAs this decision would fold in), near-constant tensors, and non-finite rows."""
        prov = self._scores(stats, steps, tau, ema=self._folded_ema(stats.mean(dim=0)))
        host = torch.cat((prov, stats[:, 1])).cpu().numpy()
        sc, r = host[:len(grads)], host[len(grads):]
        near = np.zeros(len(grads), dtype=bool)
        for _bits, lo in _WIDTH_THRESHOLDS:
            near |= np.abs(sc - lo) < self.SETTLE_MARGIN
        redo = np.nonzero(near | (r < self.NEAR_CONSTANT_R) | ~np.isfinite(sc) | ~np.isfinite(r))[0].tolist()
        if not redo:
            return stats
        stats = stats.clone()
        stats[torch.as_tensor(redo, device=stats.device)] = torch.stack(
            [self._compute_grad_stats(grads[i].float()) for i in redo])
        self._settled = len(redo)
        return stats

    def _scores(self, stats_tensor, steps, tau, ema=None):
        """The reference's per-tensor score (stquant_opt_simple.py:446-466) for all tensors at
        once: the same fp32 torch expressions, element for element, on ``[n]`` vectors.
        ``ema``: (n, r, v) EMAs to score against instead of the optimizer's."""
        n_ema, r_ema, v_ema = ema if ema is not None else (self.n_ema, self.r_ema, self.v_global_ema)
        n_l, r_l, v_l = stats_tensor[:, 0], stats_tensor[:, 1], stats_tensor[:, 2]
        t = torch.tensor([s / tau for s in steps], device=stats_tensor.device, dtype=torch.float32)
        s_t = 1.0 + (1.0 / torch.cosh(t))
        return (
            7.2
            + torch.log2(r_l / (r_ema + 1e-12))
            + torch.log2(n_l / (n_ema + 1e-12))
            + torch.log2(s_t)
            + torch.log2(v_l / (v_ema + 1e-12))
        )

    @staticmethod
    def _score_to_bits(score) -> int:
        """The widest width whose threshold the score reaches; 4 bits otherwise (NaN too)."""
        s = float(score.item()) if torch.is_tensor(score) and score.numel() == 1 else float(score)
        return next((bits for bits, lo in _WIDTH_THRESHOLDS if s >= lo), 4)

    def _folded_ema(self, mean: torch.Tensor):
        """The global EMAs ``(n, r, v)`` after folding in this decision's mean statistics
        ``[n, r, v]`` (the first decision assigns them); the same fp32 ops per component as the
        reference's :433-440."""
        if self.n_ema is None:
            return mean.unbind(0)
        a = self.param_groups[0]["alpha"]
        prev = torch.stack((self.n_ema, self.r_ema, self.v_global_ema))
        return (a * mean + (1 - a) * prev).unbind(0)

    def _fold_ema(self, mean: torch.Tensor) -> None:
        self.n_ema, self.r_ema, self.v_global_ema = self._folded_ema(mean)

    def _decide_bits(self, work) -> None:
        """Score every tensor with a grad against the global statistics and give the tensors of
        scored groups their width; fills the decision's timing keys."""
        dev = work[0][0].device
        lt = self.last_step_timings
        steps = [self.state[p]["step"] for p, _g in work]
        tau = self.param_groups[0]["tau"]
        self._settled = 0
        with _Stopwatch(dev) as sw:
            stats = self._all_grad_stats([p.grad for p, _g in work], steps, tau)
        lt["mdq_grad_stats_ms"] = sw.ms
        lt["mdq_grad_stats_settled"] = self._settled
        mean = stats.mean(dim=0)
        if dist.is_available() and dist.is_initialized():
            with _Stopwatch(dev) as sw:
                dist.all_reduce(mean, op=dist.ReduceOp.SUM)
                mean /= dist.get_world_size()
            lt["mdq_allreduce_ms"] = sw.ms
        with _Stopwatch(dev) as sw:
            self._fold_ema(mean)
            states = [self.state[p] for p, _g in work]
            scores = self._scores(stats, steps, tau)
            host = scores.cpu().tolist()                 # the step's one device -> host read
            for (_p, g), st, s, h in zip(work, states, scores.unbind(0), host):
                st["last_score"] = s
                if g.get("bits") is None:
                    st["current_bit"] = self._score_to_bits(h)
        lt["mdq_score_bits_ms"] = sw.ms

    # ------------------------------------------------------------------
    # state
    # ------------------------------------------------------------------
    @staticmethod
    def _fresh_state(p, block: int):
        """A tensor's state before its first step (stquant_opt_simple.py:212-225): 16-bit zero
        codes, zero scales and v_min = -20 per quant block, so v starts at e^-20 (quirk Q1)."""
        m, v = codes.zero_codes(p, codes.STORE_S16)
        nblk = -(-p.numel() // block)
        return {"step": 0, "exp_avg": m, "exp_avg_sq": v,
                "scale_m": torch.zeros(nblk, dtype=torch.float32, device=p.device),
                "scale_v": torch.zeros(nblk, dtype=torch.float32, device=p.device),
                "v_min": torch.full((nblk,), -20.0, dtype=torch.float32, device=p.device),
                "current_bit": 16, "last_score": torch.tensor(12.0, device=p.device)}

    @staticmethod
    def _layout(state) -> int:
        return codes.layout_of(state["exp_avg"], state["exp_avg_sq"])

    @classmethod
    def _storage_matches_bits(cls, state, bits: int) -> bool:
        """True when the codes already rest in the layout a ``bits``-wide step leaves, so the
        step needs no layout change (stquant_opt_fused_io.py:19-37).  As there, an empty tensor
        never counts as packed."""
        if "exp_avg" not in state:
            return False
        rest = codes.resting_layout(bits)
        try:
            lay = cls._layout(state)
        except RuntimeError:
            return False
        return lay == rest and not (rest == codes.STORE_P4 and state["exp_avg"].numel() == 0)

    def _begin_update(self, p, group) -> bool:
        """``step += 1`` for the tensor; True when its codes must change layout this step."""
        state = self.state[p]
        state["step"] += 1
        return not self._storage_matches_bits(state, int(state["current_bit"]))

    # ------------------------------------------------------------------
    # layout changes
    # ------------------------------------------------------------------
    def _move_codes(self, moves) -> None:
        """Re-store the codes of ``[(state, layout)]``: one device launch for the CUDA tensors
        (``_device_transitions``), the torch value map for the rest."""
        launch, news = [], []
        for state, kind in moves:
            ea, easq = state["exp_avg"], state["exp_avg_sq"]
            if ea.is_cuda and self._device_transitions and ea.numel() > 0:
                nm, nv = codes.empty_codes(ea, kind)
                launch.append((ea, easq, nm, nv))
            else:
                nm, nv = codes.restore(ea, easq, kind)
            news.append((state, nm, nv))
        if launch:
            mdq_hip.convert_codes(launch)
        for state, nm, nv in news:
            state["exp_avg"], state["exp_avg_sq"] = nm, nv

    def _split_moves(self, moved):
        """Of the tensors whose layout changes: ``{id(p): (p, group, state, new codes)}`` for
        the storage-changing step kernel, and ``[(p, group)]`` for separate conversions."""
        fused, separate = {}, []
        for p, group in moved:
            state = self.state[p]
            rest = codes.resting_layout(int(state["current_bit"]))
            ea = state["exp_avg"]
            if (self._fused_transitions and self._device_transitions and ea.is_cuda and ea.numel() > 0
                    and rest is not None and rest != self._layout(state)
                    and min(int(group["block_size"]), 1024) in mdq_hip.RESTORE_BLOCK_SIZES
                    and p.grad.dtype in self._RESTORE_GRAD_DTYPES):
                fused[id(p)] = (p, group, state, codes.empty_codes(ea, rest))
            else:
                separate.append((p, group))
        return fused, separate

    def _entries(self, rows):
        """``mdq_hip.TensorState`` of ``[(p, group, state, grad)]``."""
        ids = self._tensor_ids
        return [mdq_hip.TensorState(
            p=p, grad=gr, exp_avg=st["exp_avg"], exp_avg_sq=st["exp_avg_sq"], scale_m=st["scale_m"],
            scale_v=st["scale_v"], v_min=st["v_min"], step=st["step"], bits=int(st["current_bit"]),
            lr=g["lr"], beta1=g["betas"][0], beta2=g["betas"][1], eps=g["eps"],
            weight_decay=g["weight_decay"], tensor_id=ids.get(p, 0)) for p, g, st, gr in rows]

    def _run_restores(self, restores) -> None:
        """Storage-changing steps: one launch per (device, source layout, destination layout,
        grad dtype, block size, rounding, seed); the new codes then replace the old ones."""
        buckets = OrderedDict()
        for p, group, state, out in restores:
            grad = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
            key = (p.device, self._layout(state), codes.layout_of(*out), grad.dtype,
                   min(int(group["block_size"]), 1024), mdq_hip.rounding_code(group.get("rounding", "nearest")),
                   int(group.get("seed", 0) or 0))
            buckets.setdefault(key, []).append((p, group, state, out, grad))
        for (dev, _src, _dst, _gdt, block, rnd, seed), rows in buckets.items():
            entries = self._entries([(p, g, st, gr) for p, g, st, _o, gr in rows])
            prof = self._profile.active(dev) if self.sync_timing else None
            mdq_hip.multi_tensor_restore(entries, [o for _p, _g, _st, o, _gr in rows], block, rounding=rnd,
                                         seed=seed, profile_cycles=prof)
            for _p, _g, st, (nm, nv), _gr in rows:
                st["exp_avg"], st["exp_avg_sq"] = nm, nv

    # ------------------------------------------------------------------
    # the multi-tensor launches
    # ------------------------------------------------------------------
    def _run_kernels(self, items):
        """Group tensors by (device, code storage, grad dtype, block size,
        rounding, seed) and run one multi-tensor launch per group; returns
        ``[(plan, indices into items), ...]``.

        Each group's launch plan is cached and reused while its params and
        their state tensors are the same objects at the same addresses (a layout
        change replaces state tensors, ``p.data = ...`` moves a param; both
        rebuild the plan); per step only the grad pointers, steps, bit widths and
        hyper-parameters are refreshed.  Plans keep no reference to gradients.
        """
        buckets = OrderedDict()
        for i, (p, group) in enumerate(items):
            state = self.state[p]
            grad = p.grad
            if grad.is_sparse:
                raise RuntimeError("MDQAdamWSimple does not support sparse gradients")
            if not grad.is_contiguous():
                grad = grad.contiguous()
            ea, easq = state["exp_avg"], state["exp_avg_sq"]
            key = (p.device, ea.dtype, easq.dtype, easq.numel() == 0, grad.dtype,
                   min(int(group["block_size"]), 1024), mdq_hip.rounding_code(group.get("rounding", "nearest")),
                   int(group.get("seed", 0) or 0))
            buckets.setdefault(key, []).append((p, group, state, grad, i))
        cache = self.__dict__.setdefault("_plan_cache", {})
        runs = []
        for key, rows in buckets.items():
            idx = [r[4] for r in rows]
            rows = [r[:4] for r in rows]
            dev, block, rnd, seed = key[0], key[5], key[6], key[7]
            sig = tuple((id(p), p.data_ptr()) + tuple((id(st[k]), st[k].data_ptr()) for k in _STATE_TENSORS)
                        for p, _g, st, _gr in rows)
            plan = cache.get(key)
            if plan is None or plan.sig != sig:
                plan = self._plan_cls(self._entries(rows), block, rounding=rnd, seed=seed)
                plan.entries = None          # no references to grads
                # Strong references to the params and state tensors the plan points
                # at: while they are held no other object can reuse their id(), so
                # the id signature identifies exactly these tensors.
                plan.keep = [(p,) + tuple(st[k] for k in _STATE_TENSORS) for p, _g, st, _gr in rows]
                plan.sig = sig
                cache[key] = plan
            else:
                plan.set_grads([gr for _p, _g, _st, gr in rows])
                plan.set_steps([st["step"] for _p, _g, st, _gr in rows])
                plan.set_hparams(
                    lr=[g["lr"] for _p, g, _st, _gr in rows], beta1=[g["betas"][0] for _p, g, _st, _gr in rows],
                    beta2=[g["betas"][1] for _p, g, _st, _gr in rows], eps=[g["eps"] for _p, g, _st, _gr in rows],
                    weight_decay=[g["weight_decay"] for _p, g, _st, _gr in rows],
                    bits=[int(st["current_bit"]) for _p, _g, st, _gr in rows])
            plan.run(self._profile.active(dev) if self.sync_timing else None)
            runs.append((plan, idx))
        # plans of buckets that no longer exist keep pointers to dropped tensors
        for key in [k for k in cache if k not in buckets]:
            del cache[key]
        return runs

    @property
    def _tensor_ids(self):
        """Position of each param over all groups: the tensor id of its stochastic-rounding stream."""
        ids = getattr(self, "_tensor_id_cache", None)
        if ids is None or len(ids) != sum(len(g["params"]) for g in self.param_groups):
            ids = {p: k for k, p in enumerate(p for g in self.param_groups for p in g["params"])}
            self._tensor_id_cache = ids
        return ids

    def _batched_update(self, work):
        """One step of every tensor in ``work``:
        - tensors whose codes already rest in their width's layout go straight to the step
          launches;
        - tensors whose layout changes take the storage-changing step kernel where it exists,
          else a conversion to the kernel layout before the step and one to the resting layout
          after it.

        The timing keys are filled as the reference's per-tensor loop fills them (:501-502).
        """
        dev = work[0][0].device
        lt = self.last_step_timings
        t0 = time.perf_counter()
        flags = [self._begin_update(p, g) for p, g in work]
        moved = [w for w, f in zip(work, flags) if f]
        fused, separate = self._split_moves(moved)
        self._move_codes([(self.state[p], codes.kernel_layout(int(self.state[p]["current_bit"])))
                          for p, _g in separate])
        unpack_ms = (time.perf_counter() - t0) * 1000.0
        with _Stopwatch(dev, self.sync_timing) as sw:
            direct = [w for w in work if id(w[0]) not in fused]
            runs = self._run_kernels(direct) if direct else []
            if fused:
                self._run_restores(list(fused.values()))
        t1 = time.perf_counter()
        packs = []
        for p, _g in separate:
            st = self.state[p]
            rest = codes.resting_layout(int(st["current_bit"]))
            if rest is not None and rest != self._layout(st):
                packs.append((st, rest))
        self._move_codes(packs)
        pack_ms = (time.perf_counter() - t1) * 1000.0
        lt["quant_dequant_unpack_ms"] += unpack_ms
        lt["quant_dequant_kernel_ms"] += sw.ms
        lt["quant_dequant_pack_ms"] += pack_ms
        # No storage was replaced: the plans just launched describe the state as
        # it stands, so the next step can reuse them (``_steady_step``).
        self._steady = self._make_steady(work, runs) if runs and not moved else None

    # ------------------------------------------------------------------
    # step (stquant_opt_simple.py:383-508)
    # ------------------------------------------------------------------
    def _new_timings(self, decide: bool, update_freq) -> dict:
        lt = dict.fromkeys(_DECISION_KEYS, 0.0)
        lt.update(mdq_update_decision=decide, mdq_update_freq=update_freq)
        lt.update(dict.fromkeys(_KERNEL_WALL_KEYS, 0.0))
        lt.update(mdq_fused_io_fast_path_params=0, mdq_fused_io_fallback_params=0)
        return lt

    def _finalize_step_timings(self, profile_device):
        """Derived timing keys of the reference (:282-316): totals of the three kernel-side walls,
        and the kernel wall split into its five phases by their cycle shares (zeros and an empty
        cycle list when the params are not on a GPU)."""
        lt = self.last_step_timings
        unpack, kernel, pack = (lt.get(k, 0.0) for k in _KERNEL_WALL_KEYS)
        lt.update(mdq_unpack_ms=unpack, mdq_pack_ms=pack, mdq_fused_kernel_ms=kernel,
                  mdq_quant_dequant_ms=unpack + kernel + pack)
        if profile_device is None:
            lt.update(dict.fromkeys(_PHASE_KEYS, 0.0), mdq_kernel_phases_sum_ms=0.0, mdq_kernel_profile_cycles=[])
            return
        phases = self._profile.split(profile_device, kernel)
        lt.update(zip(_PHASE_KEYS, phases))
        lt["mdq_kernel_phases_sum_ms"] = sum(phases)
        lt["mdq_kernel_profile_cycles"] = self._profile.cycles(profile_device)

    def _profile_device(self, device):
        """The device whose phase profile this step fills (buffer zeroed), or None."""
        if not self.sync_timing or device.type != "cuda":
            return None
        self._profile.on(device).zero_()
        return device

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self.total_steps += 1
        update_freq = self.param_groups[0]["update_freq"]
        # steps 1-4 and every update_freq-th step re-decide the widths (:407)
        decide = self.total_steps < 5 or self.total_steps % update_freq == 0
        self.last_step_timings = self._new_timings(decide, update_freq)

        sc = self._steady_lookup(decide)
        if sc is not None:
            self.last_step_timings["mdq_extra_stats_ms"] = 0.0
            prof_dev = self._profile_device(sc["params"][0].device)
            if self._steady_step(sc):
                self._finalize_step_timings(prof_dev)
                return loss
        self._steady = None

        work = []
        for group in self.param_groups:
            block = min(int(group.get("block_size", 256)), 1024)
            for p in group["params"]:
                if p.grad is None:
                    continue
                work.append((p, group))
                if not self.state[p]:
                    self.state[p].update(self._fresh_state(p, block))
        # Fixed-width groups take their width; the other groups' tensors are scored against
        # global statistics over every tensor with a grad, as the reference computes them (it
        # has no fixed groups).
        for p, group in work:
            if group.get("bits") is not None:
                self.state[p]["current_bit"] = int(group["bits"])
        if decide and work and any(g.get("bits") is None for _p, g in work):
            self._decide_bits(work)
        lt = self.last_step_timings
        lt["mdq_stats_ms"] = lt["mdq_grad_stats_ms"]
        lt["mdq_bit_decision_ms"] = lt["mdq_allreduce_ms"] + lt["mdq_score_bits_ms"]
        lt["mdq_extra_stats_ms"] = lt["mdq_grad_stats_ms"] + lt["mdq_bit_decision_ms"]

        prof_dev = self._profile_device(work[0][0].device) if work else None
        if work:
            self._batched_update(work)
        self._finalize_step_timings(prof_dev)
        return loss

    # ------------------------------------------------------------------
    # metrics / checkpoint (stquant_opt_simple.py:321-378)
    # ------------------------------------------------------------------
    def _widths(self):
        """``(bits, numel)`` of every param that has a width."""
        for group in self.param_groups:
            for p in group["params"]:
                st = self.state.get(p)
                if st and "current_bit" in st:
                    yield int(st["current_bit"]), p.numel()

    @staticmethod
    def _percent(counts: Counter) -> dict:
        total = sum(counts.values())
        out = {b: 0.0 for b in _REPORTED_WIDTHS}
        if total:
            out.update({b: (c / total) * 100.0 for b, c in ({b: 0 for b in _REPORTED_WIDTHS} | counts).items()})
        return out

    def get_bit_distribution(self):
        """Percent of tensors at each width."""
        return self._percent(Counter(b for b, _n in self._widths()))

    def get_bit_distribution_param_weighted(self):
        """Percent of parameters at each width."""
        counts = Counter()
        for b, n in self._widths():
            counts[b] += n
        return self._percent(counts)

    def get_avg_bit_param_weighted(self):
        share = self.get_bit_distribution_param_weighted()
        return float(sum(b * (pc / 100.0) for b, pc in share.items()))

    def get_all_raw_scores(self):
        scores = [st["last_score"] for g in self.param_groups for p in g["params"]
                  for st in (self.state.get(p),) if st and "last_score" in st]
        if not scores:
            return []
        # one device read for all of them
        return torch.stack([s.reshape(()).to(scores[0].device, torch.float64) for s in scores]).cpu().tolist()

    def _global_stats(self) -> dict:
        return {"n_ema": self.n_ema, "r_ema": self.r_ema, "v_global_ema": self.v_global_ema,
                "total_steps": self.total_steps}

    def state_dict(self):
        return {**super().state_dict(), "mdq_global_stats": self._global_stats()}

    def load_state_dict(self, state_dict):
        """The reference's loader (stquant_opt_simple.py:371-378) with two repairs:
        - torch's ``Optimizer.load_state_dict`` casts every floating-point param's state tensors to
          the param dtype, which would turn the integer codes into float32 and lose the low bits of
          32-bit codes.  The code tensors are therefore held back from torch's loader and put back
          unchanged, on the param's device.
        - torch moves per-param state to the param's device but not the global EMA statistics;
          they are moved to the device of the first param (where the bit decision computes them),
          so a checkpoint written on one device resumes on another."""
        self._steady = None
        self.__dict__.pop("_plan_cache", None)
        sd = dict(state_dict)
        stats = sd.pop("mdq_global_stats", None)
        held = {}
        sd["state"] = {}
        for pid, st in state_dict.get("state", {}).items():
            st = dict(st)
            held[pid] = {k: st.pop(k) for k in _CODE_KEYS if k in st and torch.is_tensor(st[k])}
            sd["state"][pid] = st
        if stats is not None:
            self.n_ema, self.r_ema = stats["n_ema"], stats["r_ema"]
            self.v_global_ema, self.total_steps = stats["v_global_ema"], stats["total_steps"]
        super().load_state_dict(sd)
        params = [p for g in self.param_groups for p in g["params"]]
        saved_ids = [pid for g in sd["param_groups"] for pid in g["params"]]
        for pid, p in zip(saved_ids, params):
            for k, t in held.get(pid, {}).items():
                self.state[p][k] = t.to(p.device)
        if params:
            dev = params[0].device
            for k in ("n_ema", "r_ema", "v_global_ema"):
                v = getattr(self, k)
                if torch.is_tensor(v) and v.device != dev:
                    setattr(self, k, v.to(dev))

    # ------------------------------------------------------------------
    # steady state: same tensors, same storage, same bit widths as last step
    # ------------------------------------------------------------------
    def _group_cfg(self):
        return tuple((g.get("bits"), min(int(g.get("block_size", 256)), 1024), g.get("rounding", "nearest"),
                      g.get("seed", 0)) for g in self.param_groups)

    def _make_steady(self, params_with_grad, runs):
        gpos = {id(g): k for k, g in enumerate(self.param_groups)}
        states = [self.state[p] for p, _g in params_with_grad]
        with_grad = {id(p) for p, _g in params_with_grad}
        every = [p for g in self.param_groups for p in g["params"]]
        return {
            "all_ids": [id(p) for p in every],
            "nograd": [p for p in every if id(p) not in with_grad],
            "params": [p for p, _g in params_with_grad],
            "states": states,
            "state_obj": self.state,
            "cfg": self._group_cfg(),
            "runs": [(plan, idx, np.array([gpos[id(params_with_grad[i][1])] for i in idx], np.int64))
                     for plan, idx in runs],
        }

    def _steady_lookup(self, update_decision: bool):
        """The cached steady state if this step may reuse it, else None.

        Reuse needs: the same param objects in the groups in the same order, the
        same ``state`` dict, the same per-group bits / block size / rounding /
        seed, and no bit decision this step (scored groups re-decide bits on
        update steps).  Storage is only replaced by steps that re-pack, by
        ``load_state_dict`` and by ``add_param_group``, which all drop the cache;
        a param whose ``data`` moved, or whose grad appeared or went away, is
        caught by ``_steady_step``.
        """
        sc = self.__dict__.get("_steady")
        if sc is None or sc["state_obj"] is not self.state:
            return None
        if update_decision and any(g.get("bits") is None for g in self.param_groups):
            return None
        if sc["cfg"] != self._group_cfg():
            return None
        if list(map(id, [p for g in self.param_groups for p in g["params"]])) != sc["all_ids"]:
            return None
        return sc

    def _steady_step(self, sc) -> bool:
        """One step over the cached plans: ``step += 1`` per tensor, fresh param and grad
        pointers, steps and per-group hyper-parameters; False (nothing launched, nothing
        changed) if a param or grad no longer matches its plan."""
        params, states = sc["params"], sc["states"]
        t0 = time.perf_counter()
        grads = [p.grad for p in params]
        if any(p.grad is not None for p in sc["nograd"]):
            return False
        for plan, idx, _gidx in sc["runs"]:
            if len(sc["runs"]) == 1:
                ok = plan.try_refresh(params, grads)
            else:
                ok = plan.try_refresh([params[i] for i in idx], [grads[i] for i in idx])
            if not ok:
                return False
        steps = []
        for st in states:
            st["step"] += 1
            steps.append(st["step"])
        steps = np.asarray(steps, np.int32)
        groups = self.param_groups
        lr = np.array([g["lr"] for g in groups], np.float32)
        b1 = np.array([g["betas"][0] for g in groups], np.float32)
        b2 = np.array([g["betas"][1] for g in groups], np.float32)
        eps = np.array([g["eps"] for g in groups], np.float32)
        wd = np.array([g["weight_decay"] for g in groups], np.float32)
        unpack_ms = (time.perf_counter() - t0) * 1000.0
        dev = params[0].device
        prof = self._profile.active(dev) if self.sync_timing else None
        with _Stopwatch(dev, self.sync_timing) as sw:
            for plan, idx, gidx in sc["runs"]:
                a = plan.arr
                a["step"] = steps[idx]
                a["lr"] = lr[gidx]
                a["beta1"] = b1[gidx]
                a["beta2"] = b2[gidx]
                a["eps"] = eps[gidx]
                a["weight_decay"] = wd[gidx]
                plan.run(prof)
        lt = self.last_step_timings
        lt["quant_dequant_unpack_ms"] += unpack_ms
        lt["quant_dequant_kernel_ms"] += sw.ms
        self._count_steady_params(len(states))
        return True

    def _count_steady_params(self, n: int) -> None:
        """Per-tensor bookkeeping a steady step skips (FusedIO counts fast-path tensors)."""


_STATE_TENSORS = ("exp_avg", "exp_avg_sq", "scale_m", "scale_v", "v_min")
_CODE_KEYS = ("exp_avg", "exp_avg_sq")
