"""Code layouts of the optimizer state and the one value map between them.

A tensor's Adam moments are integer codes in one of four layouts:

========  =================  ======================  ===========  ========
layout    ``exp_avg``        ``exp_avg_sq``          m range      v range
========  =================  ======================  ===========  ========
P4        uint8 bytes        empty uint8             [-8, 7]      [0, 15]
S8        int8               uint8                   int8         uint8
S16       int16              uint16                  int16        uint16
S32       int32              uint32                  int32        uint32
========  =================  ======================  ===========  ========

A P4 byte holds ``(v << 4) | (m + 8)``.  The reference keeps exactly these tensors in the
optimizer state (/root/reference/CUDA/stquant_opt_simple.py:114-225); checkpoints must carry
them unchanged.

The reference moves codes between layouts with a chain of casts and clamps per width change
(:121-210).  Every one of those moves is the same map, which this module states once:
decode the codes to integers, clamp them to the destination's ranges, and encode them.
Scales are not touched, so a narrower width clamps codes and keeps the scales (quirk Q4).
The device conversion kernel (``stq_multi_tensor_convert_codes``) applies the same map.
``restore`` is its torch form, for CPU tensors and for the optimizer's torch route.

Which layout a width uses:

* the kernel runs on ``kernel_layout(bits)`` (:140-173): S8 up to 8 bits, S16 up to 16,
  S32 above;
* the state rests in ``resting_layout(bits)`` after a step (:175-210): P4 at 4 bits,
  otherwise the kernel layout.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

STORE_P4, STORE_S8, STORE_S16, STORE_S32 = 0, 1, 2, 3


@dataclass(frozen=True)
class Layout:
    kind: int
    name: str
    m_dtype: torch.dtype
    v_dtype: torch.dtype
    m_lo: int
    m_hi: int
    v_hi: int

    @property
    def packed(self) -> bool:
        return self.kind == STORE_P4


LAYOUTS = (
    Layout(STORE_P4, "packed nibbles", torch.uint8, torch.uint8, -8, 7, 15),
    Layout(STORE_S8, "int8/uint8", torch.int8, torch.uint8, -(1 << 7), (1 << 7) - 1, (1 << 8) - 1),
    Layout(STORE_S16, "int16/uint16", torch.int16, torch.uint16, -(1 << 15), (1 << 15) - 1, (1 << 16) - 1),
    Layout(STORE_S32, "int32/uint32", torch.int32, torch.uint32, -(1 << 31), (1 << 31) - 1, (1 << 32) - 1),
)


def kernel_layout(bits: int) -> int:
    """The layout the step kernel works on for a code width."""
    if bits >= 32:
        return STORE_S32
    return STORE_S16 if bits > 8 else STORE_S8


def resting_layout(bits: int) -> Optional[int]:
    """The layout a tensor stepped at ``bits`` is left in, or None for 17..31 bits.  The
    reference has no layout for those widths: it steps them in int16 codes, which cannot
    hold them."""
    if bits == 4:
        return STORE_P4
    if 1 <= bits <= 16 or bits == 32:
        return kernel_layout(bits)
    return None


def layout_of(exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor) -> int:
    """The layout of a state's ``(exp_avg, exp_avg_sq)`` pair."""
    if exp_avg.dtype == torch.uint8 and exp_avg_sq.numel() == 0:
        return STORE_P4
    for lay in LAYOUTS[1:]:
        if (exp_avg.dtype, exp_avg_sq.dtype) == (lay.m_dtype, lay.v_dtype) \
                and exp_avg_sq.numel() == exp_avg.numel():
            return lay.kind
    raise RuntimeError(f"no code storage class for exp_avg {exp_avg.dtype} / exp_avg_sq {exp_avg_sq.dtype}"
                       f"[{exp_avg_sq.numel()}]")


def empty_codes(like: torch.Tensor, kind: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Uninitialised codes of ``like``'s shape and device in layout ``kind``."""
    lay = LAYOUTS[kind]
    m = torch.empty_like(like, dtype=lay.m_dtype, memory_format=torch.contiguous_format)
    if lay.packed:
        return m, torch.empty(0, dtype=torch.uint8, device=like.device)
    return m, torch.empty_like(like, dtype=lay.v_dtype, memory_format=torch.contiguous_format)


def zero_codes(like: torch.Tensor, kind: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """All-zero codes of ``like``'s shape and device in layout ``kind``; a P4 zero byte
    decodes to m = -8, so P4 is not a layout a fresh state starts in."""
    m, v = empty_codes(like, kind)
    return m.zero_(), v.zero_()


# The narrowest signed integer type holding every code value of a layout (uint16 v needs
# int32, uint32 v int64).
_VALUE_DTYPE = {STORE_P4: torch.int16, STORE_S8: torch.int16, STORE_S16: torch.int32, STORE_S32: torch.int64}
_WIDTH = {torch.int16: 0, torch.int32: 1, torch.int64: 2}


def value_dtype(*kinds: int) -> torch.dtype:
    """The narrowest signed integer type holding the code values of all ``kinds``."""
    return max((_VALUE_DTYPE[k] for k in kinds), key=_WIDTH.__getitem__)


def decode(exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor,
           dtype: torch.dtype = torch.int64) -> Tuple[torch.Tensor, torch.Tensor]:
    """The integer code values ``(m, v)`` as ``dtype`` tensors of ``exp_avg``'s shape
    (``dtype`` must hold the layout's values: ``value_dtype(layout)`` or wider)."""
    if layout_of(exp_avg, exp_avg_sq) == STORE_P4:
        byte = exp_avg.to(dtype)
        return (byte & 15) - 8, byte >> 4
    return exp_avg.to(dtype), exp_avg_sq.to(dtype)


def encode(m: torch.Tensor, v: torch.Tensor, kind: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """int64 code values clamped to layout ``kind``'s ranges, stored in that layout."""
    lay = LAYOUTS[kind]
    m = m.clamp(lay.m_lo, lay.m_hi)
    v = v.clamp(0, lay.v_hi)
    if lay.packed:
        return ((v << 4) | (m + 8)).to(torch.uint8), torch.empty(0, dtype=torch.uint8, device=m.device)
    return m.to(lay.m_dtype), v.to(lay.v_dtype)


def restore(exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor, kind: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """The codes re-stored in layout ``kind``: ``encode(decode(codes), kind)``.  Empty
    tensors have no values, so only their dtypes change."""
    if exp_avg.numel() == 0:
        return empty_codes(exp_avg, kind)
    src, dst = LAYOUTS[layout_of(exp_avg, exp_avg_sq)], LAYOUTS[kind]
    if not src.packed and not dst.packed and dst.m_lo <= src.m_lo and src.m_hi <= dst.m_hi \
            and src.v_hi <= dst.v_hi:
        # every value fits the destination: the map is a plain cast
        return exp_avg.to(dst.m_dtype, copy=True), exp_avg_sq.to(dst.v_dtype, copy=True)
    # values in the narrowest type that holds both layouts' ranges: the passes move
    # 2 or 4 bytes per value rather than 8
    m, v = decode(exp_avg, exp_avg_sq, value_dtype(src.kind, kind))
    return encode(m, v, kind)
