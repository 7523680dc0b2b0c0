"""CPU oracle for the fused dequant -> AdamW -> requant step (ctypes over libmdq_oracle.so).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` import this module, and only as the checker
or the CPU baseline.  The shipped library never imports, links or calls it.

The C code (``mdq_oracle.c``) restates ``/root/reference/CUDA/stquant_kernel.cu``
(kernels :53-401, dispatch :414-465) element by element.  How each part is
pinned (independently of the oracle's own formulas):

=====================  ==============================================================
part                   pinned by
=====================  ==============================================================
expf / logf            every fp32 input vs float64 exp/log, <1 ulp
                       (tests/test_oracle_math.py)
FP64 divide + round    C ``round`` == numpy half-away rounding of the float64 quotient
                       on random and constructed-tie inputs (test_oracle_math.py)
Philox4x32            10 rounds: Random123 known-answer vectors + rocRAND's philox4x32_10;
                       7 rounds (the stochastic-rounding stream): rocRAND's own round and
                       key-bump functions applied 7 times (tests/test_oracle_philox.py)
nibble pack / unpack   all 256 bytes, closed form of stquant_kernel.cu:72-74,130
m codes / scale_m      max-|m| element -> +7 or -8 (asymmetric clamp), exact
                       ties (k+1/2)*d, codes vs a float64 closed form
v codes / scale_v      min-log element -> 0, max-log element -> 2^bits-1, tail lanes
                       force Lmax >= 0 (tests/test_oracle_step.py)
AdamW update           bits=32: matches a float64 textbook AdamW with v0 = e^-20 to
                       1e-6; lr=0 leaves p; g=0 state=0 gives p*(1-lr*wd) exactly
stochastic rounding    unbiasedness and code histogram; pieces stepped with their element
                       offsets reproduce the whole tensor (tests/test_oracle_step.py)
NaN / inf grads        the reference's fmaxf / fminf reductions ignore NaN and its (int)
                       conversion maps NaN to 0: a NaN element leaves its block's scales
                       and other codes as a finite stand-in does, codes 0, p NaN; an inf
                       element gives inf scales and all-zero codes; an all-NaN block NaN
                       scales (tests/test_oracle_nonfinite.py)
grad statistics        the reference's own torch expression (stquant_opt_simple.py:93-98)
                       on CPU tensors, closed forms for constant / two-valued grads,
                       numel 0 / 1 NaN cases, NaN / inf grads and overflowing squares
                       (tests/test_oracle_grad_stats.py)
=====================  ==============================================================

Parity with the CUDA binary itself is unpinned at one boundary only: the ulp-level
results of CUDA's ``expf``/``logf`` and nvcc's fma contraction choices, which no
file of the reference fixes (no golden vectors, no tests upstream); the oracle
fixes them as documented in ``mdq_oracle.h``.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# MDQ_ORACLE_LIB points the tests at another build of mdq_oracle.c (the mutation tests load
# builds with one planted mistake each, to show that the pinning tests catch it).
_LIB_PATH = os.environ.get("MDQ_ORACLE_LIB") or os.path.join(_HERE, "libmdq_oracle.so")

STORE_P4, STORE_S8, STORE_S16, STORE_S32 = 0, 1, 2, 3
GRAD_F32, GRAD_BF16, GRAD_F16 = 0, 1, 2
ROUND_NEAREST, ROUND_STOCHASTIC = 0, 1

STORAGE_DTYPES = {
    STORE_P4: (np.uint8, None),
    STORE_S8: (np.int8, np.uint8),
    STORE_S16: (np.int16, np.uint16),
    STORE_S32: (np.int32, np.uint32),
}


class _Tensor(ctypes.Structure):
    _fields_ = [
        ("p", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("code_m", ctypes.c_void_p),
        ("code_v", ctypes.c_void_p),
        ("scale_m", ctypes.c_void_p),
        ("scale_v", ctypes.c_void_p),
        ("v_min", ctypes.c_void_p),
        ("numel", ctypes.c_int64),
        ("storage", ctypes.c_int32),
        ("grad_dtype", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("bits", ctypes.c_int32),
        ("step", ctypes.c_int32),
        ("tensor_id", ctypes.c_uint32),
        ("elem_offset", ctypes.c_int64),
    ]


class _HParams(ctypes.Structure):
    _fields_ = [
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("lr", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("rounding", ctypes.c_int32),
        ("seed", ctypes.c_uint64),
        ("threads", ctypes.c_int32),
    ]


_lib = None


def lib():
    """Load (once) the compiled oracle; build it with ``make -C oracle`` first."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle not built: {_LIB_PATH} missing (run `make -C oracle`)")
        L = ctypes.CDLL(_LIB_PATH)
        L.mdq_oracle_step.argtypes = [ctypes.POINTER(_Tensor), ctypes.POINTER(_HParams)]
        L.mdq_oracle_step.restype = ctypes.c_int
        L.mdq_oracle_expf.argtypes = [ctypes.c_float]
        L.mdq_oracle_expf.restype = ctypes.c_float
        L.mdq_oracle_logf.argtypes = [ctypes.c_float]
        L.mdq_oracle_logf.restype = ctypes.c_float
        for name in ("mdq_oracle_expf_n", "mdq_oracle_logf_n"):
            fn = getattr(L, name)
            fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
            fn.restype = None
        L.mdq_oracle_max_ulp_err.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32]
        L.mdq_oracle_max_ulp_err.restype = ctypes.c_double
        L.mdq_oracle_round_div.argtypes = [ctypes.c_float, ctypes.c_float]
        L.mdq_oracle_round_div.restype = ctypes.c_double
        L.mdq_oracle_philox4x32_10.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.mdq_oracle_philox4x32_10.restype = None
        L.mdq_oracle_philox4x32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        L.mdq_oracle_philox4x32.restype = None
        L.mdq_oracle_math_chunk_digests.argtypes = [
            ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
        L.mdq_oracle_math_chunk_digests.restype = None
        _lib = L
    return _lib


def _ptr(a: Optional[np.ndarray]) -> Optional[int]:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def max_ulp_err(which: str, first: int, count: int) -> float:
    """Largest error in float ulps of the oracle's exp (``which='exp'``) or log over the float bit
    patterns ``first .. first+count-1``, against double-precision libm (all host threads)."""
    return float(lib().mdq_oracle_max_ulp_err(0 if which == "exp" else 1, int(first), int(count)))


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().mdq_oracle_expf_n(_ptr(x), _ptr(y), x.size)
    return y


def logf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().mdq_oracle_logf_n(_ptr(x), _ptr(y), x.size)
    return y


def round_div(num: float, den: float) -> float:
    return lib().mdq_oracle_round_div(float(num), float(den))


def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.ascontiguousarray(np.asarray(ctr, dtype=np.uint32).reshape(4))
    k = np.ascontiguousarray(np.asarray(key, dtype=np.uint32).reshape(2))
    out = np.zeros(4, dtype=np.uint32)
    lib().mdq_oracle_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return out


def philox4x32(ctr, key, rounds: int) -> np.ndarray:
    c = np.ascontiguousarray(np.asarray(ctr, dtype=np.uint32).reshape(4))
    k = np.ascontiguousarray(np.asarray(key, dtype=np.uint32).reshape(2))
    out = np.zeros(4, dtype=np.uint32)
    lib().mdq_oracle_philox4x32(_ptr(c), _ptr(k), int(rounds), _ptr(out))
    return out


SR_ROUNDS = 7   # MDQO_SR_ROUNDS: Philox4x32 rounds of the stochastic-rounding stream


def math_chunk_digests(which: str, first: int, count: int, chunk: int) -> np.ndarray:
    """Per-chunk digests of exp (``which='exp'``), log, or IEEE 1 / x (``'rcp'``) over bit patterns."""
    nchunks = (count + chunk - 1) // chunk
    out = np.zeros(nchunks, dtype=np.uint64)
    lib().mdq_oracle_math_chunk_digests({"exp": 0, "log": 1, "rcp": 3}[which], first, count, chunk, _ptr(out))
    return out


def step(p: np.ndarray, grad: np.ndarray, code_m: np.ndarray, code_v: Optional[np.ndarray],
         scale_m: np.ndarray, scale_v: np.ndarray, v_min: np.ndarray, *,
         beta1: float, beta2: float, lr: float, weight_decay: float, eps: float,
         step: int, bits: int, block_size: int, storage: int,
         rounding: int = ROUND_NEAREST, seed: int = 0, tensor_id: int = 0,
         threads: int = 0, elem_offset: int = 0) -> None:
    """One fused step on numpy arrays, in place (p, codes, scales).

    ``grad`` may be float32, or a uint16 array holding bf16 (``grad_dtype``
    inferred: float32 -> F32, uint16 -> BF16, float16 -> F16).  ``elem_offset``:
    the index of element 0 in the tensor's stochastic-rounding stream (a piece of
    a larger tensor starting there draws that tensor's random numbers).
    """
    n = p.size
    assert p.dtype == np.float32
    if grad.dtype == np.float32:
        gdt = GRAD_F32
    elif grad.dtype == np.uint16:
        gdt = GRAD_BF16
    elif grad.dtype == np.float16:
        gdt = GRAD_F16
    else:
        raise TypeError(f"unsupported grad dtype {grad.dtype}")
    assert grad.size == n and code_m.size == n
    nb = (n + block_size - 1) // block_size if n else 0
    for s in (scale_m, scale_v, v_min):
        assert s.dtype == np.float32 and s.size >= nb
    t = _Tensor(_ptr(p), _ptr(grad), _ptr(code_m), _ptr(code_v), _ptr(scale_m), _ptr(scale_v),
                _ptr(v_min), n, storage, gdt, block_size, bits, step, tensor_id, elem_offset)
    h = _HParams(beta1, beta2, lr, weight_decay, eps, rounding, seed, threads)
    rc = lib().mdq_oracle_step(ctypes.byref(t), ctypes.byref(h))
    if rc != 0:
        raise ValueError("mdq_oracle_step rejected its arguments")


def init_state(n: int, block_size: int, storage: int):
    """Fresh state as stquant_opt_simple.py:216-223 creates it, stored for ``storage``.

    Codes zero, scales zero, v_min = -20 (reference quirk: v starts at e^-20).
    A packed-4 zero state is byte 0x08 (m code 0 -> nibble 8, v code 0).
    """
    nb = (n + block_size - 1) // block_size
    dm, dv = STORAGE_DTYPES[storage]
    if storage == STORE_P4:
        code_m = np.full(n, 0x08, dtype=np.uint8)
        code_v = None
    else:
        code_m = np.zeros(n, dtype=dm)
        code_v = np.zeros(n, dtype=dv)
    return (code_m, code_v, np.zeros(nb, np.float32), np.zeros(nb, np.float32),
            np.full(nb, -20.0, np.float32))


def grad_stats(g: np.ndarray) -> np.ndarray:
    """``stquant_opt_simple.py:93-98`` restated for one gradient: float32
    ``[sqrt(mean(g^2)), std(g) / (mean(|g|) + 1e-12), mean(g^2)]`` with the
    unbiased std.  Each square is rounded to fp32 (the reference's ``grad * grad``);
    the sums are float64, the variance two-pass; then the reference's final fp32
    operations (sqrt of the fp32 mean, fp32 divide and add).  The reference sums in
    fp32 on the GPU (torch's mean, and its Welford std), so a sum of squares, of
    absolute values or of squared deviations whose exact value exceeds FLT_MAX gives
    inf.  numel 0 gives NaN means; numel 0 or 1 a NaN std, as torch does."""
    x32 = np.asarray(g, dtype=np.float32).ravel()
    x = x32.astype(np.float64)
    n = x.size
    nan = np.float32(np.nan)
    big = float(np.finfo(np.float32).max)

    def f32_mean(total, count):
        # the fp32 accumulator overflows once the exact sum exceeds FLT_MAX
        return np.float32(np.inf) if total > big else np.float32(total / count)

    with np.errstate(all="ignore"):
        if n:
            mean_sq = f32_mean(float(np.sum((x32 * x32).astype(np.float64))), n)
            mean_abs = f32_mean(float(np.sum(np.abs(x))), n)
        else:
            mean_sq = mean_abs = nan
        if n > 1:
            m2 = float(np.sum((x - np.sum(x) / n) ** 2))
            sd = np.float32(np.inf) if m2 > big else np.float32(np.sqrt(m2 / (n - 1)))
        else:
            sd = nan
        n_l = np.sqrt(mean_sq, dtype=np.float32)
        r_l = np.float32(sd / np.float32(mean_abs + np.float32(1e-12)))
    return np.array([n_l, r_l, mean_sq], dtype=np.float32)
