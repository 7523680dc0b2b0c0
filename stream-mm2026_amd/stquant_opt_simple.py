"""MDQAdamWSimple -- drop-in for /root/reference/CUDA/stquant_opt_simple.py on MI355X.

Same constructor, param groups, ``step()``, state layout (per param: ``step``,
``exp_avg`` / ``exp_avg_sq`` integer codes -- packed nibbles in ``exp_avg`` and an
empty ``exp_avg_sq`` at 4 bits --, ``scale_m``, ``scale_v``, ``v_min`` per quant
block, ``current_bit``, ``last_score``), ``state_dict`` extras, bit-distribution
getters and timing keys as the reference.

What differs is underneath: instead of one kernel launch per tensor bracketed by
two device synchronisations (:242-265), ``step()`` runs ONE multi-tensor HIP
launch per storage class through the C ABI of ``libstquant_hip.so``
(``mdq_hip.multi_tensor_step``).  Tensors whose bit width changed go through
one launch of the storage-changing step (``mdq_hip.multi_tensor_restore``: the
reference's align -> kernel -> pack of :140-280 in one pass, block sizes
64 / 128 / 256), or else through device conversions with exactly the
reference's storage rules (:140-210).  Results per element are those of the
reference kernel (:246-263 -> stquant_kernel.cu).

New optional param-group keys (defaults keep the reference behaviour):
``bits`` (fixed code width 4/8/16/32 instead of the score-based choice; such groups still
count in the global gradient statistics that score the other groups),
``rounding`` ('nearest' or 'stochastic') and ``seed`` (stochastic stream).
``sync_timing=False`` skips the device synchronisations that fill the timing
dict (and the kernel phase profile), so ``step()`` issues its work
asynchronously on the current stream.
"""
from __future__ import annotations

import math
import time
from collections import OrderedDict

import numpy as np
import torch
import torch.distributed as dist
from torch.optim import Optimizer

import mdq_hip


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
        # stquant_opt_simple.py:33-44
        tau_adaptive = 300 * math.log(layer_count) * math.sqrt(batch_size)
        if bits is not None and int(bits) not in (4, 8, 16, 32):
            raise ValueError(f"bits must be one of 4, 8, 16, 32 or None, got {bits}")
        mdq_hip.rounding_code(rounding)
        if grad_stats not in ("fused", "reference"):
            raise ValueError(f"grad_stats must be 'fused' or 'reference', got {grad_stats!r}")
        defaults = dict(
            lr=lr,
            betas=betas,
            eps=eps,
            weight_decay=weight_decay,
            alpha=alpha,
            tau=tau_adaptive,
            update_freq=update_freq,
            block_size=block_size,
            bits=bits,
            rounding=rounding,
            seed=seed,
        )
        super().__init__(params, defaults)

        self.n_ema = None
        self.r_ema = None
        self.v_global_ema = None
        self.total_steps = 0
        self.last_step_timings = {}
        self.sync_timing = sync_timing
        self.grad_stats = grad_stats
        self._kernel_profile_buf = None
        self._kernel_profile_device = None

    _KERNEL_PROF_SLOTS = 5
    # launch-plan class of ``_run_kernels`` (a test harness substitutes its own executor)
    _plan_cls = mdq_hip.MultiTensorPlan
    # storage changes of CUDA tensors in one conversion launch per step; False keeps the
    # reference's per-tensor torch passes (same results)
    _device_transitions = True
    # with device transitions: a tensor whose storage changes is stepped by a kernel that reads
    # the old storage and writes the new one (block sizes 64 / 128 / 256), instead of convert ->
    # step -> pack; False keeps the separate passes (same results)
    _fused_transitions = True

    def add_param_group(self, param_group):
        self.__dict__["_steady"] = None
        super().add_param_group(param_group)

    # ------------------------------------------------------------------
    # kernel phase profile (stquant_opt_simple.py:56-83)
    # ------------------------------------------------------------------
    def _kernel_profile_buf_for(self, device):
        if self._kernel_profile_buf is None or self._kernel_profile_device != device:
            self._kernel_profile_buf = torch.zeros(self._KERNEL_PROF_SLOTS, dtype=torch.int64, device=device)
            self._kernel_profile_device = device
        return self._kernel_profile_buf

    def _reset_kernel_profile(self, device):
        self._kernel_profile_buf_for(device).zero_()

    def _read_kernel_profile_cycles(self, device):
        buf = self._kernel_profile_buf_for(device)
        return buf.double().cpu().tolist()

    def _kernel_phases_ms_from_wall(self, device, kernel_wall_ms):
        if kernel_wall_ms <= 0:
            return [0.0] * self._KERNEL_PROF_SLOTS
        cycles = self._read_kernel_profile_cycles(device)
        total = sum(cycles)
        if total <= 0:
            return [0.0] * self._KERNEL_PROF_SLOTS
        return [kernel_wall_ms * (c / total) for c in cycles]

    @staticmethod
    def _sync_device(device):
        if device.type == "cuda":
            torch.cuda.synchronize(device)

    # ------------------------------------------------------------------
    # grad stats and bit choice (stquant_opt_simple.py:93-109)
    # ------------------------------------------------------------------
    @staticmethod
    def _compute_grad_stats(grad: torch.Tensor) -> torch.Tensor:
        n_l = torch.sqrt(torch.mean(grad * grad))
        r_l = torch.std(grad) / (grad.abs().mean() + 1e-12)
        v_l = torch.mean(grad * grad)
        return torch.stack([n_l, r_l, v_l])

    def _all_grad_stats(self, grads):
        """``[n, 3]`` stats of all grads: one fused launch per grad dtype, or the reference's
        per-tensor torch reductions (``grad_stats="reference"``, stquant_opt_simple.py:427-431)."""
        if self.grad_stats == "fused" and grads and grads[0].is_cuda:
            return mdq_hip.grad_stats(grads)
        return torch.stack([self._compute_grad_stats(g.float()) for g in grads])

    def _scores(self, stats_tensor, steps, tau):
        """The reference's per-tensor score (stquant_opt_simple.py:446-466) for all tensors at
        once: the same fp32 torch expressions, element for element, on ``[n]`` vectors."""
        n_l, r_l, v_l = stats_tensor[:, 0], stats_tensor[:, 1], stats_tensor[:, 2]
        t = torch.tensor([s / tau for s in steps], device=stats_tensor.device, dtype=torch.float32)
        s_t = 1.0 + (1.0 / torch.cosh(t))
        return (
            7.2
            + torch.log2(r_l / (self.r_ema + 1e-12))
            + torch.log2(n_l / (self.n_ema + 1e-12))
            + torch.log2(s_t)
            + torch.log2(v_l / (self.v_global_ema + 1e-12))
        )

    @staticmethod
    def _score_to_bits(score) -> int:
        s = float(score.item()) if torch.is_tensor(score) and score.numel() == 1 else float(score)
        if s >= 24:
            return 32
        if s >= 12:
            return 16
        if s >= 6.8:
            return 8
        return 4

    # ------------------------------------------------------------------
    # code storage pack / unpack / align (stquant_opt_simple.py:114-210)
    # ------------------------------------------------------------------
    @staticmethod
    def _is_momentum_packed4(state):
        if "exp_avg" not in state or "exp_avg_sq" not in state:
            return False
        ea, easq = state["exp_avg"], state["exp_avg_sq"]
        return ea.dtype == torch.uint8 and easq.numel() == 0 and ea.numel() > 0

    @classmethod
    def _storage_matches_bits(cls, state, bits: int) -> bool:
        """True when the code storage is already the one ``bits`` uses
        (stquant_opt_fused_io.py:19-37); aligning and re-packing are no-ops then."""
        if "exp_avg" not in state:
            return False
        ea, easq = state["exp_avg"], state.get("exp_avg_sq")
        if bits == 4:
            return cls._is_momentum_packed4(state)
        if bits == 8:
            return (
                ea.dtype == torch.int8
                and easq is not None
                and easq.dtype == torch.uint8
                and easq.numel() == ea.numel()
            )
        if bits == 16:
            return ea.dtype == torch.int16 and easq is not None and easq.dtype == torch.uint16
        if bits >= 32:
            return ea.dtype == torch.int32 and easq is not None and easq.dtype == torch.uint32
        return False

    @staticmethod
    def _unpack_packed4_momentum(state):
        packed = state["exp_avg"]
        m_u = (packed.to(torch.int32) & 0x0F).to(torch.int16)
        v_q = ((packed.to(torch.int32) >> 4) & 0x0F).to(torch.int32)
        state["exp_avg"] = (m_u - 8).to(torch.int8)
        state["exp_avg_sq"] = v_q.to(torch.uint8)

    @staticmethod
    def _pack_momentum_to_nibbles(state):
        ea, easq = state["exp_avg"], state["exp_avg_sq"]
        if ea.dtype != torch.int8 or easq.numel() != ea.numel():
            return
        dev = ea.device
        m_u = (ea.to(torch.int16) + 8).clamp(0, 15).to(torch.uint8)
        v_lo = easq.to(torch.int32).clamp(0, 15).to(torch.uint8)
        state["exp_avg"] = (m_u | (v_lo << 4)).to(dev)
        state["exp_avg_sq"] = torch.empty(0, dtype=torch.uint8, device=dev)

    @classmethod
    def _align_momentum_storage(cls, state, bits):
        if cls._is_momentum_packed4(state):
            cls._unpack_packed4_momentum(state)

        ea, easq = state["exp_avg"], state["exp_avg_sq"]

        if bits >= 32:
            if ea.dtype != torch.int32:
                state["exp_avg"] = ea.to(torch.int32)
            if easq.dtype != torch.uint32:
                state["exp_avg_sq"] = easq.to(torch.uint32)
            return

        if bits > 8:
            if ea.dtype == torch.int8:
                state["exp_avg"] = ea.to(torch.int16)
                state["exp_avg_sq"] = easq.to(torch.uint16)
            elif ea.dtype == torch.int32:
                state["exp_avg"] = ea.clamp(-32768, 32767).to(torch.int16)
                state["exp_avg_sq"] = easq.to(torch.int64).clamp(0, 65535).to(torch.uint16)
            elif ea.dtype != torch.int16:
                state["exp_avg"] = ea.to(torch.int16)
                state["exp_avg_sq"] = easq.to(torch.uint16)
            return

        if ea.dtype == torch.int16:
            state["exp_avg"] = ea.clamp(-128, 127).to(torch.int8)
            state["exp_avg_sq"] = easq.to(torch.int64).clamp(0, 255).to(torch.uint8)
        elif ea.dtype == torch.int32:
            state["exp_avg"] = ea.clamp(-128, 127).to(torch.int8)
            state["exp_avg_sq"] = easq.to(torch.int64).clamp(0, 255).to(torch.uint8)
        elif ea.dtype == torch.int8 and easq.numel() > 0 and easq.dtype != torch.uint8:
            state["exp_avg_sq"] = easq.to(torch.uint8)

    @classmethod
    def _pack_momentum_storage(cls, state, bits):
        ea, easq = state["exp_avg"], state["exp_avg_sq"]

        if bits <= 8:
            if ea.dtype == torch.int16:
                state["exp_avg"] = ea.clamp(-128, 127).to(torch.int8)
                state["exp_avg_sq"] = easq.to(torch.int64).clamp(0, 255).to(torch.uint8)
            elif ea.dtype == torch.int32:
                state["exp_avg"] = ea.clamp(-128, 127).to(torch.int8)
                state["exp_avg_sq"] = easq.to(torch.int64).clamp(0, 255).to(torch.uint8)
            elif ea.dtype == torch.int8 and easq.numel() > 0 and easq.dtype != torch.uint8:
                state["exp_avg_sq"] = easq.to(torch.uint8)

            if (
                bits == 4
                and state["exp_avg"].dtype == torch.int8
                and state["exp_avg_sq"].numel() == state["exp_avg"].numel()
            ):
                cls._pack_momentum_to_nibbles(state)
            return

        if bits == 16:
            if ea.dtype == torch.int32:
                state["exp_avg"] = ea.clamp(-32768, 32767).to(torch.int16)
                state["exp_avg_sq"] = easq.to(torch.int64).clamp(0, 65535).to(torch.uint16)
            elif ea.dtype == torch.int8:
                state["exp_avg"] = ea.to(torch.int16)
                state["exp_avg_sq"] = easq.to(torch.uint16)
            return

        if bits >= 32:
            if ea.dtype != torch.int32:
                state["exp_avg"] = ea.to(torch.int32)
            if easq.dtype != torch.uint32:
                state["exp_avg_sq"] = easq.to(torch.uint32)

    def _init_state_if_needed(self, p, state, block_size):
        # stquant_opt_simple.py:212-225
        if len(state) != 0:
            return
        state["step"] = 0
        state["exp_avg"] = torch.zeros_like(p, dtype=torch.int16, memory_format=torch.contiguous_format)
        state["exp_avg_sq"] = torch.zeros_like(p, dtype=torch.uint16, memory_format=torch.contiguous_format)
        num_blocks = (p.numel() + block_size - 1) // block_size
        state["scale_m"] = torch.zeros(num_blocks, dtype=torch.float32, device=p.device)
        state["scale_v"] = torch.zeros(num_blocks, dtype=torch.float32, device=p.device)
        state["v_min"] = torch.full((num_blocks,), -20.0, dtype=torch.float32, device=p.device)
        state["current_bit"] = 16
        state["last_score"] = torch.tensor(12.0, device=p.device)

    def get_last_step_timings(self):
        return dict(self.last_step_timings)

    # ------------------------------------------------------------------
    # per-tensor preparation around the batched kernel
    # ------------------------------------------------------------------
    def _prepare_update(self, p, group):
        """Per-tensor work before the kernel: ``step += 1`` and the storage
        alignment of stquant_opt_simple.py:231-239.  Returns True when the
        storage must be re-packed after the kernel (:269).

        A state whose storage already fits ``bits`` is handed to the kernel
        as it is: for packed nibbles at 4 bits, unpack -> int8/uint8 kernel ->
        re-pack (the reference's route) yields the same codes, scales and params
        byte for byte; for the other widths aligning and packing change nothing.
        """
        state = self.state[p]
        bits = int(state["current_bit"])
        state["step"] += 1
        if self._storage_matches_bits(state, bits):
            return False
        pending = self.__dict__.get("_pending_align")
        if pending is not None and state["exp_avg"].is_cuda:
            pending.append((p, group, state, bits))    # one launch for all (_flush_align)
        else:
            self._align_momentum_storage(state, bits)
        return True

    def _finish_update(self, p):
        state = self.state[p]
        bits = int(state["current_bit"])
        pending = self.__dict__.get("_pending_pack")
        if pending is not None and state["exp_avg"].is_cuda:
            pending.append((state, bits))
        else:
            self._pack_momentum_storage(state, bits)

    @staticmethod
    def _aligned_storage(bits: int) -> int:
        """The code storage _align_momentum_storage leaves for ``bits`` (:166-198)."""
        if bits >= 32:
            return mdq_hip.STORE_S32
        if bits > 8:
            return mdq_hip.STORE_S16
        return mdq_hip.STORE_S8

    @classmethod
    def _final_storage(cls, bits: int):
        """The code storage a step at ``bits`` leaves (align, kernel, pack: :140-219), or None
        for widths the storage cannot hold (17..31 bits go to int16 there)."""
        if bits == 4:
            return mdq_hip.STORE_P4
        if 1 <= bits <= 16 or bits == 32:
            return cls._aligned_storage(bits)
        return None

    _RESTORE_GRAD_DTYPES = (torch.float32, torch.bfloat16, torch.float16)

    @staticmethod
    def _convert_states(moves):
        """Re-store the codes of ``[(state, dst_storage)]`` with one conversion launch."""
        items, news = [], []
        for state, dst in moves:
            ea, easq = state["exp_avg"], state["exp_avg_sq"]
            nm, nv = mdq_hip.empty_codes(ea, dst)
            items.append((ea, easq, nm, nv))
            news.append((state, nm, nv))
        mdq_hip.convert_codes(items)
        for state, nm, nv in news:
            state["exp_avg"], state["exp_avg_sq"] = nm, nv

    def _flush_align(self):
        """Device version of _align_momentum_storage for all deferred tensors: the same value map
        (unpack nibbles, widen, or clamp to the narrower range; :140-198) in one launch.

        Tensors that a storage-changing kernel can step (``_fused_transitions``) are not
        converted: they get destination codes in their final storage and are collected in
        ``self._restores`` for ``_run_restores``."""
        pending, self._pending_align = self.__dict__.get("_pending_align") or [], None
        moves = []
        restores = {}
        for p, group, state, bits in pending:
            if state["exp_avg"].numel() == 0:          # the reference's dtype rules for empty tensors
                self._align_momentum_storage(state, bits)
                continue
            src = mdq_hip.storage_of(state["exp_avg"], state["exp_avg_sq"])
            fin = self._final_storage(bits)
            if (self._fused_transitions and fin is not None and fin != src
                    and min(int(group["block_size"]), 1024) in mdq_hip.RESTORE_BLOCK_SIZES
                    and p.grad.dtype in self._RESTORE_GRAD_DTYPES):
                restores[id(p)] = (p, group, state, mdq_hip.empty_codes(state["exp_avg"], fin))
                continue
            dst = self._aligned_storage(bits)
            if src != dst:
                moves.append((state, dst))
        if moves:
            self._convert_states(moves)
        self._restores = restores

    def _run_restores(self, restores):
        """Storage-changing steps: one launch per (device, source storage, destination storage,
        grad dtype, block size, rounding, seed), then the new codes replace the old ones."""
        buckets = OrderedDict()
        ids = self._tensor_ids
        for p, group, state, out in restores:
            grad = p.grad if p.grad.is_contiguous() else p.grad.contiguous()
            key = (p.device, mdq_hip.storage_of(state["exp_avg"], state["exp_avg_sq"]),
                   mdq_hip.storage_of(*out), grad.dtype, min(int(group["block_size"]), 1024),
                   mdq_hip.rounding_code(group.get("rounding", "nearest")), int(group.get("seed", 0) or 0))
            buckets.setdefault(key, []).append((p, group, state, out, grad))
        for key, lst in buckets.items():
            dev, bsz, rnd, seed = key[0], key[4], key[5], key[6]
            entries = [mdq_hip.TensorState(
                p=p, grad=gr, exp_avg=st["exp_avg"], exp_avg_sq=st["exp_avg_sq"], scale_m=st["scale_m"],
                scale_v=st["scale_v"], v_min=st["v_min"], step=st["step"], bits=int(st["current_bit"]),
                lr=g["lr"], beta1=g["betas"][0], beta2=g["betas"][1], eps=g["eps"],
                weight_decay=g["weight_decay"], tensor_id=ids.get(p, 0)) for p, g, st, _o, gr in lst]
            prof = None
            if self.sync_timing and self._kernel_profile_buf is not None and self._kernel_profile_device == dev:
                prof = self._kernel_profile_buf
            mdq_hip.multi_tensor_restore(entries, [o for _p, _g, _st, o, _gr in lst], bsz, rounding=rnd,
                                         seed=seed, profile_cycles=prof)
            for _p, _g, st, (nm, nv), _gr in lst:
                st["exp_avg"], st["exp_avg_sq"] = nm, nv

    def _flush_pack(self):
        """Device version of _pack_momentum_storage after the step: 4-bit tensors in int8/uint8
        storage go to nibbles (:214-219) in one launch; after alignment every other width
        is already in its final storage."""
        pending, self._pending_pack = self.__dict__.get("_pending_pack") or [], None
        moves = []
        for state, bits in pending:
            if (bits == 4 and state["exp_avg"].numel() > 0
                    and mdq_hip.storage_of(state["exp_avg"], state["exp_avg_sq"]) == mdq_hip.STORE_S8):
                moves.append((state, mdq_hip.STORE_P4))
            else:
                self._pack_momentum_storage(state, bits)
        if moves:
            self._convert_states(moves)

    def _launch_fused_update(self, p, group):
        """Single-tensor update with the reference's per-tensor timing (:231-280)."""
        t0 = time.perf_counter()
        repack = self._prepare_update(p, group)
        unpack_ms = (time.perf_counter() - t0) * 1000.0
        self._sync_device(p.device)
        tk0 = time.perf_counter()
        self._run_kernels([(p, group)])
        self._sync_device(p.device)
        kernel_ms = (time.perf_counter() - tk0) * 1000.0
        t1 = time.perf_counter()
        if repack:
            self._finish_update(p)
        pack_ms = (time.perf_counter() - t1) * 1000.0
        lt = self.last_step_timings
        lt["quant_dequant_unpack_ms"] = lt.get("quant_dequant_unpack_ms", 0.0) + unpack_ms
        lt["quant_dequant_kernel_ms"] = lt.get("quant_dequant_kernel_ms", 0.0) + kernel_ms
        lt["quant_dequant_pack_ms"] = lt.get("quant_dequant_pack_ms", 0.0) + pack_ms

    def _run_kernels(self, items):
        """Group tensors by (device, code storage, grad dtype, block size,
        rounding, seed) and run one multi-tensor launch per group; returns
        ``[(plan, indices into items), ...]``.

        Each group's launch plan is cached and reused while its tensors and
        their state tensors stay the same objects (bit-width transitions replace
        state tensors and so rebuild the plan); per step only the grad
        pointers, steps, bit widths and hyper-parameters are refreshed.  Plans
        keep no reference to gradients.
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
        ids = self._tensor_ids
        runs = []
        for key, lst in buckets.items():
            lst = [x[:4] for x in lst]
            idx = [x[4] for x in buckets[key]]
            dev, bsz, rnd, seed = key[0], key[5], key[6], key[7]
            sig = tuple((id(p), id(st["exp_avg"]), id(st["exp_avg_sq"]), id(st["scale_m"]),
                         id(st["scale_v"]), id(st["v_min"])) for p, _g, st, _gr in lst)
            plan = cache.get(key)
            if plan is None or plan.sig != sig:
                entries = [mdq_hip.TensorState(
                    p=p, grad=gr, exp_avg=st["exp_avg"], exp_avg_sq=st["exp_avg_sq"], scale_m=st["scale_m"],
                    scale_v=st["scale_v"], v_min=st["v_min"], step=st["step"], bits=int(st["current_bit"]),
                    lr=g["lr"], beta1=g["betas"][0], beta2=g["betas"][1], eps=g["eps"],
                    weight_decay=g["weight_decay"], tensor_id=ids.get(p, 0)) for p, g, st, gr in lst]
                plan = self._plan_cls(entries, bsz, rounding=rnd, seed=seed)
                plan.entries = None          # no references to grads
                # Strong references to the params and state tensors the plan points
                # at: while they are held no other object can reuse their id(), so
                # the id signature identifies exactly these tensors.
                plan.keep = [(p, st["exp_avg"], st["exp_avg_sq"], st["scale_m"], st["scale_v"], st["v_min"])
                             for p, _g, st, _gr in lst]
                plan.sig = sig
                cache[key] = plan
            else:
                plan.set_grads([gr for _p, _g, _st, gr in lst])
                plan.set_steps([st["step"] for _p, _g, st, _gr in lst])
                plan.set_hparams(
                    lr=[g["lr"] for _p, g, _st, _gr in lst], beta1=[g["betas"][0] for _p, g, _st, _gr in lst],
                    beta2=[g["betas"][1] for _p, g, _st, _gr in lst], eps=[g["eps"] for _p, g, _st, _gr in lst],
                    weight_decay=[g["weight_decay"] for _p, g, _st, _gr in lst],
                    bits=[int(st["current_bit"]) for _p, _g, st, _gr in lst])
            prof = None
            if self.sync_timing and self._kernel_profile_buf is not None and self._kernel_profile_device == dev:
                prof = self._kernel_profile_buf
            plan.run(prof)
            runs.append((plan, idx))
        # plans of buckets that no longer exist keep pointers to dropped tensors
        for key in [k for k in cache if k not in buckets]:
            del cache[key]
        return runs

    @property
    def _tensor_ids(self):
        ids = getattr(self, "_tensor_id_cache", None)
        if ids is None or len(ids) != sum(len(g["params"]) for g in self.param_groups):
            ids = {}
            k = 0
            for g in self.param_groups:
                for p in g["params"]:
                    ids[p] = k
                    k += 1
            self._tensor_id_cache = ids
        return ids

    def _finalize_step_timings(self, profile_device):
        # stquant_opt_simple.py:282-316
        unpack = self.last_step_timings.get("quant_dequant_unpack_ms", 0.0)
        pack = self.last_step_timings.get("quant_dequant_pack_ms", 0.0)
        kernel_wall = self.last_step_timings.get("quant_dequant_kernel_ms", 0.0)

        self.last_step_timings["mdq_unpack_ms"] = unpack
        self.last_step_timings["mdq_pack_ms"] = pack
        self.last_step_timings["mdq_fused_kernel_ms"] = kernel_wall
        self.last_step_timings["mdq_quant_dequant_ms"] = unpack + kernel_wall + pack

        if profile_device is not None:
            k_ms = self._kernel_phases_ms_from_wall(profile_device, kernel_wall)
            (
                self.last_step_timings["mdq_kernel_dequant_ms"],
                self.last_step_timings["mdq_kernel_adam_mv_ms"],
                self.last_step_timings["mdq_kernel_scale_reduce_ms"],
                self.last_step_timings["mdq_kernel_quant_ms"],
                self.last_step_timings["mdq_kernel_update_p_ms"],
            ) = k_ms
            self.last_step_timings["mdq_kernel_phases_sum_ms"] = sum(k_ms)
            self.last_step_timings["mdq_kernel_profile_cycles"] = self._read_kernel_profile_cycles(profile_device)
        else:
            for key in (
                "mdq_kernel_dequant_ms",
                "mdq_kernel_adam_mv_ms",
                "mdq_kernel_scale_reduce_ms",
                "mdq_kernel_quant_ms",
                "mdq_kernel_update_p_ms",
                "mdq_kernel_phases_sum_ms",
                "mdq_kernel_profile_cycles",
            ):
                self.last_step_timings[key] = 0.0 if key != "mdq_kernel_profile_cycles" else []

    # ------------------------------------------------------------------
    # metrics / checkpoint (stquant_opt_simple.py:321-378)
    # ------------------------------------------------------------------
    def get_bit_distribution(self):
        counts = {4: 0, 8: 0, 16: 0, 32: 0}
        num_tensors = 0
        for group in self.param_groups:
            for p in group["params"]:
                st = self.state.get(p)
                if st and "current_bit" in st:
                    b = int(st["current_bit"])
                    counts[b] = counts.get(b, 0) + 1
                    num_tensors += 1
        if num_tensors == 0:
            return {4: 0.0, 8: 0.0, 16: 0.0, 32: 0.0}
        return {b: (c / num_tensors) * 100.0 for b, c in counts.items()}

    def get_bit_distribution_param_weighted(self):
        counts_numel = {4: 0, 8: 0, 16: 0, 32: 0}
        for group in self.param_groups:
            for p in group["params"]:
                st = self.state.get(p)
                if st and "current_bit" in st:
                    b = int(st["current_bit"])
                    counts_numel[b] = counts_numel.get(b, 0) + p.numel()
        total = sum(counts_numel.values())
        if total == 0:
            return {4: 0.0, 8: 0.0, 16: 0.0, 32: 0.0}
        return {k: (v / total) * 100.0 for k, v in counts_numel.items()}

    def get_avg_bit_param_weighted(self):
        dist_bits = self.get_bit_distribution_param_weighted()
        return float(sum(b * (perc / 100.0) for b, perc in dist_bits.items()))

    def get_all_raw_scores(self):
        scores = []
        for group in self.param_groups:
            for p in group["params"]:
                st = self.state.get(p)
                if st and "last_score" in st:
                    scores.append(float(st["last_score"].item()))
        return scores

    def state_dict(self):
        out = super().state_dict()
        out["mdq_global_stats"] = {
            "n_ema": self.n_ema,
            "r_ema": self.r_ema,
            "v_global_ema": self.v_global_ema,
            "total_steps": self.total_steps,
        }
        return out

    _CODE_KEYS = ("exp_avg", "exp_avg_sq")

    def load_state_dict(self, state_dict):
        """As stquant_opt_simple.py:371-378, plus the repair the reference lacks:
        torch's ``Optimizer.load_state_dict`` casts every floating-point-param
        state tensor to the param dtype, turning integer codes into float32.
        The code values are small integers (exact in float32); each code tensor
        is cast back to the integer dtype it had in ``state_dict``.  torch also
        moves per-param state to the param's device, but not the global EMA
        statistics; they are moved to the device of the first param (where the
        bit decision computes them), so a checkpoint written on one device
        resumes on another."""
        self._steady = None
        self.__dict__.pop("_plan_cache", None)
        saved_dtypes = {}
        for pid, st in state_dict.get("state", {}).items():
            saved_dtypes[pid] = {k: st[k].dtype for k in self._CODE_KEYS
                                 if k in st and torch.is_tensor(st[k])}
        state_dict = dict(state_dict)
        if "mdq_global_stats" in state_dict:
            stats = state_dict.pop("mdq_global_stats")
            self.n_ema = stats["n_ema"]
            self.r_ema = stats["r_ema"]
            self.v_global_ema = stats["v_global_ema"]
            self.total_steps = stats["total_steps"]
        super().load_state_dict(state_dict)
        params = [p for g in self.param_groups for p in g["params"]]
        saved_ids = [pid for g in state_dict["param_groups"] for pid in g["params"]]
        for pid, p in zip(saved_ids, params):
            st = self.state.get(p)
            if not st:
                continue
            for k, dt in saved_dtypes.get(pid, {}).items():
                if st[k].dtype != dt:
                    st[k] = st[k].to(dt)
        if params:
            for k in ("n_ema", "r_ema", "v_global_ema"):
                v = getattr(self, k)
                if torch.is_tensor(v) and v.device != params[0].device:
                    setattr(self, k, v.to(params[0].device))

    # ------------------------------------------------------------------
    # step (stquant_opt_simple.py:383-508)
    # ------------------------------------------------------------------
    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()

        self.total_steps += 1
        self.last_step_timings = {
            "mdq_stats_ms": 0.0,
            "mdq_bit_decision_ms": 0.0,
            "mdq_grad_stats_ms": 0.0,
            "mdq_allreduce_ms": 0.0,
            "mdq_score_bits_ms": 0.0,
            "mdq_update_decision": False,
            "mdq_update_freq": 0,
            "quant_dequant_unpack_ms": 0.0,
            "quant_dequant_kernel_ms": 0.0,
            "quant_dequant_pack_ms": 0.0,
            "mdq_fused_io_fast_path_params": 0,
            "mdq_fused_io_fallback_params": 0,
        }

        update_freq = self.param_groups[0]["update_freq"]
        update_decision = (self.total_steps % update_freq == 0) or (self.total_steps < 5)
        self.last_step_timings["mdq_update_decision"] = update_decision
        self.last_step_timings["mdq_update_freq"] = update_freq

        sc = self._steady_lookup(update_decision)
        if sc is not None:
            for key in ("mdq_grad_stats_ms", "mdq_allreduce_ms", "mdq_score_bits_ms", "mdq_stats_ms",
                        "mdq_bit_decision_ms", "mdq_extra_stats_ms"):
                self.last_step_timings[key] = 0.0
            dev = sc["params"][0].device
            profile_device = dev if self.sync_timing and dev.type == "cuda" else None
            if profile_device is not None:
                self._reset_kernel_profile(profile_device)
            if self._steady_step(sc):
                self._finalize_step_timings(profile_device)
                return loss
        self._steady = None

        params_with_grad = []

        for group in self.param_groups:
            b_size = min(int(group.get("block_size", 256)), 1024)
            for p in group["params"]:
                if p.grad is None:
                    continue
                params_with_grad.append((p, group))
                state = self.state[p]
                self._init_state_if_needed(p, state, b_size)

        # Fixed-width groups (new ``bits`` option) take their width; tensors of the other groups
        # are scored against global statistics over every tensor with a grad, as the reference
        # computes them (it has no fixed groups).
        for p, group in params_with_grad:
            if group.get("bits") is not None:
                self.state[p]["current_bit"] = int(group["bits"])
        scored = any(g.get("bits") is None for _p, g in params_with_grad)

        grad_stats_ms = 0.0
        allreduce_ms = 0.0
        score_bits_ms = 0.0

        stats_tensor = None
        if update_decision and params_with_grad and scored:
            dev = params_with_grad[0][0].device
            self._sync_device(dev)
            t_grad = time.perf_counter()
            stats_tensor = self._all_grad_stats([p.grad for p, _g in params_with_grad])
            self._sync_device(dev)
            grad_stats_ms = (time.perf_counter() - t_grad) * 1000.0

        if stats_tensor is not None:
            dev = params_with_grad[0][0].device
            avg_stats = stats_tensor.mean(dim=0)

            if dist.is_available() and dist.is_initialized():
                self._sync_device(dev)
                t_ar = time.perf_counter()
                dist.all_reduce(avg_stats, op=dist.ReduceOp.SUM)
                avg_stats /= dist.get_world_size()
                self._sync_device(dev)
                allreduce_ms = (time.perf_counter() - t_ar) * 1000.0

            self._sync_device(dev)
            t_score = time.perf_counter()
            if self.n_ema is None:
                self.n_ema = avg_stats[0]
                self.r_ema = avg_stats[1]
                self.v_global_ema = avg_stats[2]
            else:
                alpha = self.param_groups[0]["alpha"]
                self.n_ema = alpha * avg_stats[0] + (1 - alpha) * self.n_ema
                self.r_ema = alpha * avg_stats[1] + (1 - alpha) * self.r_ema
                self.v_global_ema = alpha * avg_stats[2] + (1 - alpha) * self.v_global_ema

            tau = self.param_groups[0]["tau"]
            states = [self.state[p] for p, _g in params_with_grad]
            scores = self._scores(stats_tensor, [st["step"] for st in states], tau)
            host_scores = scores.cpu().tolist()          # the step's one device -> host read
            for (_p, g), st, sc, hs in zip(params_with_grad, states, scores.unbind(0), host_scores):
                st["last_score"] = sc
                if g.get("bits") is None:
                    st["current_bit"] = self._score_to_bits(hs)
            self._sync_device(dev)
            score_bits_ms = (time.perf_counter() - t_score) * 1000.0

        lt = self.last_step_timings
        lt["mdq_grad_stats_ms"] = grad_stats_ms
        lt["mdq_allreduce_ms"] = allreduce_ms
        lt["mdq_score_bits_ms"] = score_bits_ms
        lt["mdq_stats_ms"] = grad_stats_ms
        lt["mdq_bit_decision_ms"] = allreduce_ms + score_bits_ms
        lt["mdq_extra_stats_ms"] = grad_stats_ms + allreduce_ms + score_bits_ms

        # Phase profiling needs the cycle buffer read back (a device sync), so it
        # is on only with sync_timing, as the reference always has it.
        profile_device = None
        if params_with_grad and self.sync_timing:
            profile_device = params_with_grad[0][0].device
            if profile_device.type == "cuda":
                self._reset_kernel_profile(profile_device)

        if params_with_grad:
            self._batched_update(params_with_grad)

        self._finalize_step_timings(
            profile_device if profile_device is not None and profile_device.type == "cuda" else None
        )
        return loss

    def _batched_update(self, params_with_grad):
        """All tensors: prepare (align storage), one launch per storage class,
        re-pack; timing keys as the per-tensor loop of :501-502 fills them."""
        dev = params_with_grad[0][0].device
        t0 = time.perf_counter()
        self._pending_align = [] if self._device_transitions else None
        try:
            repack = [self._prepare_update(p, g) for p, g in params_with_grad]
        finally:
            self._flush_align()
        unpack_ms = (time.perf_counter() - t0) * 1000.0
        if self.sync_timing:
            self._sync_device(dev)
        tk0 = time.perf_counter()
        restores = self.__dict__.pop("_restores", None) or {}
        if restores:
            steady = [(p, g) for p, g in params_with_grad if id(p) not in restores]
            runs = self._run_kernels(steady) if steady else []
            self._run_restores(list(restores.values()))
        else:
            runs = self._run_kernels(params_with_grad)
        if self.sync_timing:
            self._sync_device(dev)
        kernel_ms = (time.perf_counter() - tk0) * 1000.0
        t1 = time.perf_counter()
        self._pending_pack = [] if self._device_transitions else None
        try:
            for (p, _g), rp in zip(params_with_grad, repack):
                if rp and id(p) not in restores:
                    self._finish_update(p)
        finally:
            self._flush_pack()
        pack_ms = (time.perf_counter() - t1) * 1000.0
        lt = self.last_step_timings
        lt["quant_dequant_unpack_ms"] += unpack_ms
        lt["quant_dequant_kernel_ms"] += kernel_ms
        lt["quant_dequant_pack_ms"] += pack_ms
        # No storage was replaced: the plans just launched describe the state as
        # it stands, so the next step can reuse them (``_steady_step``).
        self._steady = self._make_steady(params_with_grad, runs) if runs and not any(repack) else None

    # ------------------------------------------------------------------
    # steady state: same tensors, same storage, same bit widths as last step
    # ------------------------------------------------------------------
    def _group_cfg(self):
        return tuple((g.get("bits"), min(int(g.get("block_size", 256)), 1024), g.get("rounding", "nearest"),
                      g.get("seed", 0)) for g in self.param_groups)

    def _make_steady(self, params_with_grad, runs):
        gpos = {id(g): k for k, g in enumerate(self.param_groups)}
        states = [self.state[p] for p, _g in params_with_grad]
        return {
            "ids": [id(p) for p, _g in params_with_grad],
            "params": [p for p, _g in params_with_grad],
            "states": states,
            "state_obj": self.state,
            "cfg": self._group_cfg(),
            "runs": [(plan, idx, np.array([gpos[id(params_with_grad[i][1])] for i in idx], np.int64))
                     for plan, idx in runs],
        }

    def _steady_lookup(self, update_decision: bool):
        """The cached steady state if this step may reuse it, else None.

        Reuse needs: the same param objects with grads in the same order, the
        same ``state`` dict, the same per-group bits / block size / rounding /
        seed, and no bit decision this step (scored groups re-decide bits on
        update steps).  Storage is only replaced by steps that re-pack, by
        ``load_state_dict`` and by ``add_param_group``, which all drop the cache.
        """
        sc = self.__dict__.get("_steady")
        if sc is None or sc["state_obj"] is not self.state:
            return None
        if update_decision and any(g.get("bits") is None for g in self.param_groups):
            return None
        if sc["cfg"] != self._group_cfg():
            return None
        cur = [id(p) for g in self.param_groups for p in g["params"] if p.grad is not None]
        if cur != sc["ids"]:
            return None
        return sc

    def _steady_step(self, sc) -> bool:
        """One step over the cached plans: ``step += 1`` per tensor, fresh grad
        pointers, steps and per-group hyper-parameters; False (nothing launched,
        nothing changed) if a grad no longer matches its plan."""
        params, states = sc["params"], sc["states"]
        t0 = time.perf_counter()
        for plan, idx, _gidx in sc["runs"]:
            if not plan.try_set_grads([params[i].grad for i in idx]):
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
        prof = None
        if self.sync_timing and self._kernel_profile_buf is not None and self._kernel_profile_device == dev:
            prof = self._kernel_profile_buf
        if self.sync_timing:
            self._sync_device(dev)
        tk0 = time.perf_counter()
        for plan, idx, gidx in sc["runs"]:
            a = plan.arr
            a["step"] = steps[idx]
            a["lr"] = lr[gidx]
            a["beta1"] = b1[gidx]
            a["beta2"] = b2[gidx]
            a["eps"] = eps[gidx]
            a["weight_decay"] = wd[gidx]
            plan.run(prof)
        if self.sync_timing:
            self._sync_device(dev)
        kernel_ms = (time.perf_counter() - tk0) * 1000.0
        lt = self.last_step_timings
        lt["quant_dequant_unpack_ms"] += unpack_ms
        lt["quant_dequant_kernel_ms"] += kernel_ms
        self._count_steady_params(len(states))
        return True

    def _count_steady_params(self, n: int) -> None:
        """Per-tensor bookkeeping a steady step skips (FusedIO counts fast-path tensors)."""
