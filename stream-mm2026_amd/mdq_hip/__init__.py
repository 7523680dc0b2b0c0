"""MI355X-native fused dequant -> AdamW -> requant step (MDQ / STREAM optimizer).

Host side of the C-ABI library ``libstquant_hip.so``.  Torch tensors are used
only for device memory and streams; every call goes through the C ABI declared
in ``include/stquant_hip.h`` and runs hand-written HIP kernels for gfx950.
There is no CPU or eager-PyTorch fallback: a missing library raises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch

from . import _capi, storage
from ._capi import NOALLOC_MAX_TENSORS, ROUND_NEAREST, ROUND_STOCHASTIC, StqTensor, check, dtype_code, lib
from .storage import STORE_P4, STORE_S8, STORE_S16, STORE_S32, empty_codes
from .storage import layout_of as storage_of

__all__ = [
    "ROUND_NEAREST", "ROUND_STOCHASTIC", "STORE_P4", "STORE_S8", "STORE_S16", "STORE_S32",
    "TensorState", "MultiTensorPlan", "fused_step", "multi_tensor_step", "multi_tensor_restore",
    "RESTORE_BLOCK_SIZES", "grad_stats", "step_table_uploads", "convert_codes", "empty_codes", "storage_of",
    "block_aligned_ranges", "shard_states",
    "device_math", "device_math_digests", "device_log_approx_error", "device_hw_ulp_error", "host_math",
    "host_round_half_away",
    "host_div_code_range", "host_philox",
    "lib", "rounding_code", "storage",
]


def rounding_code(rounding) -> int:
    if rounding in (ROUND_NEAREST, "nearest", None):
        return ROUND_NEAREST
    if rounding in (ROUND_STOCHASTIC, "stochastic"):
        return ROUND_STOCHASTIC
    raise ValueError(f"rounding must be 'nearest' or 'stochastic', got {rounding!r}")


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _check_dense(name: str, t: torch.Tensor) -> None:
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _profile_args(profile_cycles: Optional[torch.Tensor]):
    # stquant_kernel.cu:403-412: undefined or empty -> off; else CUDA int64 with >= 5 slots.
    if profile_cycles is None or profile_cycles.numel() == 0:
        return None, 0
    if not profile_cycles.is_cuda or profile_cycles.dtype != torch.int64:
        raise RuntimeError("profile_cycles must be CUDA int64 tensor")
    if profile_cycles.numel() < 5:
        raise RuntimeError("profile_cycles needs >= 5 elements")
    return profile_cycles.data_ptr(), profile_cycles.numel()


def fused_step(p, grad, exp_avg, exp_avg_sq, scale_m, scale_v, v_min,
               beta1, beta2, lr, weight_decay, eps, step, bits, block_size,
               profile_cycles=None, *, rounding=ROUND_NEAREST, seed=0, tensor_id=0) -> None:
    """One fused step on one tensor (the reference's ``fused_mdq_adamw``).

    Checks and messages follow /root/reference/CUDA/stquant_kernel.cu:420-464.
    """
    if not (p.is_cuda and grad.is_cuda):
        raise RuntimeError("p/grad must be CUDA")
    if not exp_avg.is_cuda:
        raise RuntimeError("exp_avg must be CUDA")
    if p.dtype != torch.float32:
        raise RuntimeError(f"expected scalar type Float but found {p.dtype}")
    for name, t in (("scale_m", scale_m), ("scale_v", scale_v), ("v_min", v_min)):
        if t.dtype != torch.float32:
            raise RuntimeError(f"{name}: expected scalar type Float but found {t.dtype}")
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be CUDA")
        _check_dense(name, t)
    for name, t in (("p", p), ("grad", grad), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
        _check_dense(name, t)
    for name, t in (("grad", grad), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq), ("scale_m", scale_m),
                    ("scale_v", scale_v), ("v_min", v_min)):
        if t.device != p.device and (t.numel() or name != "exp_avg_sq"):
            raise RuntimeError(f"{name} must be on the params' device ({p.device}), got {t.device}")
    if exp_avg_sq.numel() and not exp_avg_sq.is_cuda:
        raise RuntimeError("exp_avg_sq must be CUDA")
    prof_ptr, prof_n = _profile_args(profile_cycles)
    L = lib()
    with torch.cuda.device(p.device):
        rc = L.stq_fused_mdq_adamw(
            _ptr(p), _ptr(grad), dtype_code(grad.dtype), grad.numel(), p.numel(),
            _ptr(exp_avg), dtype_code(exp_avg.dtype), exp_avg.numel(),
            _ptr(exp_avg_sq), dtype_code(exp_avg_sq.dtype), exp_avg_sq.numel(),
            _ptr(scale_m), scale_m.numel(), _ptr(scale_v), scale_v.numel(),
            _ptr(v_min), v_min.numel(),
            float(beta1), float(beta2), float(lr), float(weight_decay), float(eps),
            int(step), int(bits), int(block_size),
            prof_ptr, prof_n,
            rounding_code(rounding), int(seed) & 0xFFFFFFFFFFFFFFFF, int(tensor_id) & 0xFFFFFFFF,
            _capi.stream_handle(p.device))
    check(rc)


@dataclass
class TensorState:
    """One tensor of a multi-tensor step (state tensors as the optimizer keeps them)."""

    p: torch.Tensor
    grad: torch.Tensor
    exp_avg: torch.Tensor
    exp_avg_sq: torch.Tensor
    scale_m: torch.Tensor
    scale_v: torch.Tensor
    v_min: torch.Tensor
    step: int
    bits: int
    lr: float
    beta1: float
    beta2: float
    eps: float
    weight_decay: float
    tensor_id: int = 0
    elem_offset: int = 0        # element 0's index in tensor_id's stochastic-rounding stream


# numpy mirror of ``stq_tensor`` (152 bytes, no padding): a plan's descriptor list
# lives in one structured array whose columns are refreshed vectorised per step.
STQ_TENSOR_DTYPE = np.dtype([
    ("p", np.uint64), ("grad", np.uint64), ("exp_avg", np.uint64), ("exp_avg_sq", np.uint64),
    ("scale_m", np.uint64), ("scale_v", np.uint64), ("v_min", np.uint64),
    ("numel", np.int64), ("grad_numel", np.int64), ("exp_avg_numel", np.int64),
    ("exp_avg_sq_numel", np.int64), ("scale_m_numel", np.int64), ("scale_v_numel", np.int64),
    ("v_min_numel", np.int64),
    ("beta1", np.float32), ("beta2", np.float32), ("lr", np.float32), ("weight_decay", np.float32),
    ("eps", np.float32), ("step", np.int32), ("bits", np.int32), ("tensor_id", np.uint32),
    ("elem_offset", np.int64),
])
assert STQ_TENSOR_DTYPE.itemsize == ctypes.sizeof(StqTensor)


class MultiTensorPlan:
    """The ``stq_tensor`` list of a fixed set of tensors, ready to launch.

    Validation and pointer extraction happen once; per call only the columns
    that change between steps are refreshed (``set_steps``, ``set_grads``,
    ``set_hparams``).  The tensors must stay alive and keep their storage while
    the plan is used.
    """

    def __init__(self, entries: Sequence[TensorState], block_size: int, *,
                 rounding=ROUND_NEAREST, seed: int = 0):
        self.n = len(entries)
        self.block_size = int(block_size)
        self.rounding = rounding_code(rounding)
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        self.entries = list(entries)
        self.arr, self.codes = _pack_entries(self.entries)
        self.device = self.entries[0].p.device if self.entries else None
        self._grad_dtype = self.entries[0].grad.dtype if self.entries else None
        self._dev_index = self.entries[0].p.get_device() if self.entries else -1
        self._numel = self.arr["numel"].tolist()
        self._last_p = self.arr["p"].tolist()         # param pointers as Python ints (try_refresh)

    def set_steps(self, steps) -> None:
        self.arr["step"] = steps

    def set_grads(self, grads: Sequence[torch.Tensor]) -> None:
        """New grad tensors of the same dtype and size (autograd reallocates them)."""
        gdt = self.codes[0]
        if len(grads) != self.n:
            raise RuntimeError("set_grads: one grad per planned tensor")
        numel = self.arr["numel"]
        for i, g in enumerate(grads):
            if dtype_code(g.dtype) != gdt or g.numel() != numel[i] or not g.is_contiguous() \
                    or g.device != self.device:
                raise RuntimeError("set_grads: grad must match the planned dtype, size and device")
        self.arr["grad"] = [g.data_ptr() for g in grads]

    def try_set_grads(self, grads: Sequence[torch.Tensor]) -> bool:
        """``set_grads`` that returns False (and changes nothing) instead of raising."""
        if len(grads) != self.n:
            return False
        tdt, di = self._grad_dtype, self._dev_index
        ptrs = []
        for g, n in zip(grads, self._numel):
            if g is None or g.dtype is not tdt or g.get_device() != di or g.numel() != n \
                    or not g.is_contiguous():
                return False
            ptrs.append(g.data_ptr())
        self.arr["grad"] = ptrs
        return True

    def try_set_params(self, params: Sequence[torch.Tensor]) -> bool:
        """Refresh the param pointers (``p.data`` may have been replaced by a tensor elsewhere,
        as ``Module.to()`` does); False (nothing changed) when a param no longer fits its row:
        another dtype, size or device, or not contiguous."""
        if len(params) != self.n:
            return False
        di = self._dev_index
        ptrs = []
        for p, n in zip(params, self._numel):
            if p.dtype is not torch.float32 or p.get_device() != di or p.numel() != n or not p.is_contiguous():
                return False
            ptrs.append(p.data_ptr())
        self.arr["p"] = ptrs
        self._last_p = ptrs
        return True

    def try_refresh(self, params: Sequence[torch.Tensor], grads: Sequence[torch.Tensor]) -> bool:
        """``try_set_params`` and ``try_set_grads`` in one pass, for a steady optimizer step: a
        param whose data pointer is the one this plan last launched with is checked for its
        size only (its dtype, device and layout came with that storage), a param at a new
        address fully; a grad for its dtype and contiguity (torch ties a param's grad to the
        param's size and device).  False (nothing changed) when something no longer fits."""
        if len(params) != self.n or len(grads) != self.n:
            return False
        tdt, di, last = self._grad_dtype, self._dev_index, self._last_p
        pp, gp = [], []
        for k, (p, g, n) in enumerate(zip(params, grads, self._numel)):
            a = p.data_ptr()
            if a != last[k] and (p.dtype is not torch.float32 or p.get_device() != di or not p.is_contiguous()):
                return False
            if p.numel() != n or g is None or g.dtype is not tdt or not g.is_contiguous():
                return False
            pp.append(a)
            gp.append(g.data_ptr())
        self.arr["p"] = pp
        self.arr["grad"] = gp
        self._last_p = pp
        return True

    def set_hparams(self, lr=None, beta1=None, beta2=None, eps=None, weight_decay=None, bits=None) -> None:
        for name, v in (("lr", lr), ("beta1", beta1), ("beta2", beta2), ("eps", eps),
                        ("weight_decay", weight_decay), ("bits", bits)):
            if v is not None:
                self.arr[name] = v

    def run(self, profile_cycles: Optional[torch.Tensor] = None, *, noalloc: bool = False) -> None:
        """One launch over the plan's tensors on the current stream.  ``noalloc`` takes the
        library's allocation-free entry point (``stq_multi_tensor_mdq_adamw_noalloc``: at
        most NOALLOC_MAX_TENSORS tensors, one table per GPU shared by all its streams)."""
        if self.n == 0:
            return
        if self.device.type != "cuda":
            raise RuntimeError("p/grad must be CUDA")
        prof_ptr, prof_n = _profile_args(profile_cycles)
        gdt, eadt, easqdt = self.codes
        L = lib()
        fn = L.stq_multi_tensor_mdq_adamw_noalloc if noalloc else L.stq_multi_tensor_mdq_adamw
        with torch.cuda.device(self.device):
            rc = fn(self.arr.ctypes.data_as(ctypes.POINTER(StqTensor)), self.n, gdt, eadt, easqdt,
                    self.block_size, self.rounding, self.seed, prof_ptr, prof_n, _capi.stream_handle(self.device))
        check(rc)


def _pack_entries(entries: Sequence[TensorState]):
    n = len(entries)
    arr = np.zeros(n, dtype=STQ_TENSOR_DTYPE)
    if n == 0:
        return arr, (0, 0, 0)
    e0 = entries[0]
    dev = e0.p.device
    gdt, eadt, easqdt = e0.grad.dtype, e0.exp_avg.dtype, e0.exp_avg_sq.dtype
    rows = []
    for e in entries:
        if e.p.device != dev or e.grad.device != dev:
            raise RuntimeError("multi_tensor_step: all tensors must be on one device")
        for name, t in (("exp_avg", e.exp_avg), ("exp_avg_sq", e.exp_avg_sq), ("scale_m", e.scale_m),
                        ("scale_v", e.scale_v), ("v_min", e.v_min)):
            if t.device != dev and (t.numel() or name != "exp_avg_sq"):
                raise RuntimeError(f"{name} must be on the params' device ({dev}), got {t.device}")
        if e.grad.dtype != gdt or e.exp_avg.dtype != eadt or e.exp_avg_sq.dtype != easqdt:
            raise RuntimeError("multi_tensor_step: grad and code dtypes must match across tensors")
        if e.p.dtype != torch.float32:
            raise RuntimeError(f"expected scalar type Float but found {e.p.dtype}")
        for name, t in (("p", e.p), ("grad", e.grad), ("exp_avg", e.exp_avg),
                        ("exp_avg_sq", e.exp_avg_sq), ("scale_m", e.scale_m),
                        ("scale_v", e.scale_v), ("v_min", e.v_min)):
            if not t.is_contiguous():
                raise RuntimeError(f"{name} must be contiguous")
        rows.append((
            e.p.data_ptr(), e.grad.data_ptr(), e.exp_avg.data_ptr(),
            e.exp_avg_sq.data_ptr() if e.exp_avg_sq.numel() else 0,
            e.scale_m.data_ptr(), e.scale_v.data_ptr(), e.v_min.data_ptr(),
            e.p.numel(), e.grad.numel(), e.exp_avg.numel(), e.exp_avg_sq.numel(),
            e.scale_m.numel(), e.scale_v.numel(), e.v_min.numel(),
            e.beta1, e.beta2, e.lr, e.weight_decay, e.eps, int(e.step), int(e.bits),
            int(e.tensor_id) & 0xFFFFFFFF, int(e.elem_offset)))
    arr[:] = rows
    return arr, (dtype_code(gdt), dtype_code(eadt), dtype_code(easqdt))


def block_aligned_ranges(numel: int, block_size: int, world: int):
    """``[(start, end)] * world``: one tensor's elements cut into ``world`` contiguous pieces at
    quant-block boundaries of B = min(block_size, 1024), balanced by whole blocks (the first
    ``nblocks % world`` pieces hold one block more; the last non-empty piece ends at ``numel``).
    Blocks are independent, so stepping every piece gives exactly the whole tensor's step."""
    if world < 1:
        raise ValueError("world must be >= 1")
    B = min(int(block_size), 1024)
    nb = (numel + B - 1) // B
    q, r = divmod(nb, world)
    out, b = [], 0
    for k in range(world):
        nk = q + (1 if k < r else 0)
        out.append((min(b * B, numel), min((b + nk) * B, numel)))
        b += nk
    return out


def shard_states(entries: Sequence[TensorState], block_size: int, world: int, rank: int):
    """The TensorState views of piece ``rank`` of every tensor (block_aligned_ranges); tensors
    whose piece is empty are left out.  Each piece's ``elem_offset`` is its start in the tensor,
    so stochastic rounding draws the whole tensor's random numbers too."""
    B = min(int(block_size), 1024)
    out = []
    for e in entries:
        s, t = block_aligned_ranges(e.p.numel(), block_size, world)[rank]
        if s == t:
            continue
        b0, b1 = s // B, (t + B - 1) // B
        vsq = e.exp_avg_sq if e.exp_avg_sq.numel() == 0 else e.exp_avg_sq.view(-1)[s:t]
        out.append(TensorState(e.p.view(-1)[s:t], e.grad.view(-1)[s:t], e.exp_avg.view(-1)[s:t], vsq,
                               e.scale_m[b0:b1], e.scale_v[b0:b1], e.v_min[b0:b1], e.step, e.bits, e.lr,
                               e.beta1, e.beta2, e.eps, e.weight_decay, e.tensor_id, e.elem_offset + s))
    return out


def multi_tensor_step(entries: Sequence[TensorState], block_size: int, *,
                      rounding=ROUND_NEAREST, seed: int = 0,
                      profile_cycles: Optional[torch.Tensor] = None) -> None:
    """One launch over all ``entries`` (same device, code storage, grad dtype)."""
    if len(entries) == 0:
        return
    MultiTensorPlan(entries, block_size, rounding=rounding, seed=seed).run(profile_cycles)


# stq_code_out: destination code pointers and sizes of one tensor of a storage-changing step
STQ_CODE_OUT_DTYPE = np.dtype([("exp_avg", np.uint64), ("exp_avg_sq", np.uint64), ("exp_avg_numel", np.int64),
                               ("exp_avg_sq_numel", np.int64)])
# block sizes with storage-changing step kernels (stq_multi_tensor_mdq_adamw_restore)
RESTORE_BLOCK_SIZES = (64, 128, 256)


def multi_tensor_restore(entries: Sequence[TensorState], outs, block_size: int, *,
                         rounding=ROUND_NEAREST, seed: int = 0,
                         profile_cycles: Optional[torch.Tensor] = None) -> None:
    """One launch of a step that changes the code storage: each entry's codes are read from
    ``exp_avg`` / ``exp_avg_sq`` (one source storage for all entries) and its new codes written
    to ``outs[i] = (exp_avg, exp_avg_sq)`` (one destination storage), as MDQAdamWSimple's
    align -> kernel -> pack route for a changed bit width (stquant_opt_simple.py:231-280)."""
    entries, outs = list(entries), list(outs)
    if len(entries) != len(outs):
        raise RuntimeError("multi_tensor_restore: one destination per tensor")
    if not entries:
        return
    src = storage_of(entries[0].exp_avg, entries[0].exp_avg_sq)
    dst = storage_of(*outs[0])
    out = np.zeros(len(entries), dtype=STQ_CODE_OUT_DTYPE)
    dev = entries[0].p.device
    if dev.type != "cuda":
        raise RuntimeError("p/grad must be CUDA")
    for k, (e, (m, v)) in enumerate(zip(entries, outs)):
        if storage_of(e.exp_avg, e.exp_avg_sq) != src or storage_of(m, v) != dst:
            raise RuntimeError("multi_tensor_restore: one source and one destination storage per call")
        for t in (e.exp_avg, e.exp_avg_sq, m, v):
            if t.numel() and (t.device != dev or not t.is_contiguous()):
                raise RuntimeError("multi_tensor_restore: code tensors must be contiguous and on the params' device")
        out[k] = (m.data_ptr() if m.numel() else 0, v.data_ptr() if v.numel() else 0, m.numel(), v.numel())
    arr, (gdt, _eadt, _easqdt) = _pack_entries(entries)
    prof_ptr, prof_n = _profile_args(profile_cycles)
    with torch.cuda.device(dev):
        rc = lib().stq_multi_tensor_mdq_adamw_restore(
            arr.ctypes.data_as(ctypes.POINTER(StqTensor)), out.ctypes.data, len(entries), gdt, src, dst,
            int(block_size), rounding_code(rounding), int(seed) & 0xFFFFFFFFFFFFFFFF, prof_ptr, prof_n,
            _capi.stream_handle(dev))
    check(rc)


def step_table_uploads(device=None) -> int:
    """Descriptor tables the step entry points have uploaded on ``device`` (default: the current
    CUDA device) since the library was loaded.  Steps over a fixed tensor set whose tensors share
    their step count and AdamW constants launch from the device copy of an identical table left
    by an earlier call on the same stream, without an upload."""
    count = ctypes.c_int64(0)
    with torch.cuda.device(device if device is not None else torch.cuda.current_device()):
        check(lib().stq_step_table_uploads(ctypes.byref(count)))
    return int(count.value)


def grad_stats(grads: Sequence[torch.Tensor], out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Per-tensor ``(sqrt(mean g^2), std(g) / (mean|g| + 1e-12), mean g^2)`` as a float32
    ``[len(grads), 3]`` device tensor, from one multi-tensor launch per grad dtype (fp64 sums,
    fixed order).  The reference computes the same three values per tensor with fp32 torch
    reductions (stquant_opt_simple.py:93-98)."""
    n = len(grads)
    if n == 0:
        return torch.empty(0, 3, dtype=torch.float32)
    dev = grads[0].device
    if dev.type != "cuda":
        raise RuntimeError("grad_stats: grads must be CUDA tensors")
    if out is None:
        out = torch.empty(n, 3, dtype=torch.float32, device=dev)
    elif out.shape != (n, 3) or out.dtype != torch.float32 or out.device != dev or not out.is_contiguous():
        raise RuntimeError("grad_stats: out must be a contiguous float32 [n, 3] tensor on the grads' device")
    by_dtype = {}
    for i, g in enumerate(grads):
        if g.device != dev:
            raise RuntimeError("grad_stats: all grads must be on one device")
        by_dtype.setdefault(g.dtype, []).append(i)
    keep = []
    with torch.cuda.device(dev):
        stream = _capi.stream_handle(dev)
        for dt, idx in by_dtype.items():
            gs = [grads[i] if grads[i].is_contiguous() else grads[i].contiguous() for i in idx]
            keep.extend(gs)
            ptrs = np.array([g.data_ptr() if g.numel() else 0 for g in gs], dtype=np.uint64)
            numels = np.array([g.numel() for g in gs], dtype=np.int64)
            dst = out if len(idx) == n else torch.empty(len(idx), 3, dtype=torch.float32, device=dev)
            check(lib().stq_multi_tensor_grad_stats(ptrs.ctypes.data, numels.ctypes.data, len(idx),
                                                    dtype_code(dt), dst.data_ptr(), stream))
            if dst is not out:
                out[torch.as_tensor(idx, device=dev)] = dst
    return out


# stq_code_convert: 4 pointers, int64 numel, two int32 storages (48 bytes)
STQ_CONVERT_DTYPE = np.dtype([("src_m", np.uint64), ("src_v", np.uint64), ("dst_m", np.uint64),
                              ("dst_v", np.uint64), ("numel", np.int64), ("src", np.int32), ("dst", np.int32)])


def convert_codes(items) -> None:
    """Re-store codes for a list of ``(src_exp_avg, src_exp_avg_sq, dst_exp_avg, dst_exp_avg_sq)``
    in one launch (storage classes inferred from the dtypes): decode the source, clamp to the
    destination's range, encode -- every storage change of stquant_opt_simple.py:140-210."""
    items = list(items)
    if not items:
        return
    arr = np.zeros(len(items), dtype=STQ_CONVERT_DTYPE)
    dev = items[0][0].device
    for k, (sm, sv, dm, dv) in enumerate(items):
        for t in (sm, sv, dm, dv):
            if t.numel() and (t.device != dev or not t.is_contiguous()):
                raise RuntimeError("convert_codes: code tensors must be contiguous and on one CUDA device")
        if dm.numel() != sm.numel():
            raise RuntimeError("convert_codes: source and destination sizes differ")
        arr[k] = (sm.data_ptr() if sm.numel() else 0, sv.data_ptr() if sv.numel() else 0,
                  dm.data_ptr() if dm.numel() else 0, dv.data_ptr() if dv.numel() else 0, sm.numel(),
                  storage_of(sm, sv), storage_of(dm, dv))
    if dev.type != "cuda":
        raise RuntimeError("convert_codes: code tensors must be CUDA tensors")
    with torch.cuda.device(dev):
        check(lib().stq_multi_tensor_convert_codes(arr.ctypes.data, len(items), _capi.stream_handle(dev)))


def device_log_approx_error(first: int, count: int, slope: float = 0.0, device="cuda:0") -> float:
    """max(0, max |v_log_f32(x) ln 2 - log x| - slope |log x|) over the floats with bit patterns
    first .. first+count-1, computed on the device in fp64 (the bound behind the step kernel's
    fast v-code path)."""
    dev = torch.device(device)
    out = torch.zeros(1, dtype=torch.int64, device=dev)
    with torch.cuda.device(dev):
        check(lib().stq_device_log_approx_error(int(first), int(count), float(slope), out.data_ptr(),
                                                _capi.stream_handle(dev)))
    return float(out.cpu().view(torch.float64).item())


def device_hw_ulp_error(which: str, first: int, count: int, device="cuda:0") -> int:
    """Largest ulp distance between the hardware sqrt (``which='sqrt'``) or reciprocal
    (``'rcp'``) of the step's parameter update and the correctly rounded result, over the
    floats with bit patterns first .. first+count-1."""
    dev = torch.device(device)
    out = torch.zeros(1, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        check(lib().stq_device_hw_ulp_error({"sqrt": 0, "rcp": 1}[which], int(first), int(count), out.data_ptr(),
                                            _capi.stream_handle(dev)))
    return int(out.cpu().item())


def device_math(which: str, x: torch.Tensor) -> torch.Tensor:
    """Device e^x (``which='exp'``), log x (``'log'``) or the stochastic requant's reciprocal
    (``'rcp'``) with the kernels' own fp32 code; or ``'vcode_map'``: x holds (dv, vmin) pairs,
    the result the fast v-code path's (ln 2 / dv, -vmin / dv) pairs; or ``'sr_vfast'``: x holds
    (x, kv, dv, vmin, lmax, QV) 6-tuples, the result (Zh, ep, 0, 0, 0, 0): the stochastic fast
    v-code path's estimate of T - 1/2 and its error bound."""
    assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()
    y = torch.empty_like(x)
    code = {"exp": 0, "log": 1, "vcode_map": 2, "rcp": 3, "sr_vfast": 4}[which]
    with torch.cuda.device(x.device):
        check(lib().stq_device_math(code, _ptr(x), _ptr(y), x.numel(), _capi.stream_handle(x.device)))
    return y


def device_math_digests(which: str, first: int, count: int, chunk: int, device=None) -> torch.Tensor:
    device = torch.device(device or "cuda")
    nchunks = (count + chunk - 1) // chunk
    dig = torch.zeros(nchunks, dtype=torch.int64, device=device)
    with torch.cuda.device(device):
        check(lib().stq_device_math_digests({"exp": 0, "log": 1, "rcp": 3}[which], first, count, chunk,
                                            dig.data_ptr(), _capi.stream_handle(device)))
    return dig


def host_math(which: str, x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().stq_host_math(0 if which == "exp" else 1, x.ctypes.data, y.ctypes.data, x.size)
    return y


def host_round_half_away(u, d, inv_ulps: int = 0):
    u = np.ascontiguousarray(u, dtype=np.float32)
    d = np.ascontiguousarray(d, dtype=np.float32)
    out = np.empty_like(u)
    lib().stq_host_round_half_away(u.ctypes.data, d.ctypes.data, out.ctypes.data, u.size, int(inv_ulps))
    return out


def host_div_code_range(x, bits: int):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().stq_host_div_code_range(x.ctypes.data, out.ctypes.data, x.size, int(bits))
    return out


def host_philox(ctr, key):
    c = np.ascontiguousarray(np.asarray(ctr, dtype=np.uint32).reshape(4))
    k = np.ascontiguousarray(np.asarray(key, dtype=np.uint32).reshape(2))
    out = np.zeros(4, dtype=np.uint32)
    lib().stq_host_philox4x32_10(c.ctypes.data, k.ctypes.data, out.ctypes.data)
    return out
