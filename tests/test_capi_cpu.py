"""The C-ABI library loads, exports every symbol include/stquant_hip.h declares,
and rejects bad arguments with the reference's messages before touching a GPU
(no device work is issued by any call in this file)."""
import ctypes
import os
import re

import pytest
import torch

import mdq_hip
from mdq_hip import _capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "stquant_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|void|const char \*)\s*(stq_\w+)\s*\(", text, re.M)))


def test_exports_every_declared_symbol():
    L = mdq_hip.lib()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(L, name), name
    assert set(names) == set(_capi.EXPORTED_SYMBOLS)
    assert L.stq_abi_version() == _capi.ABI_VERSION == 4


FAKE = 0x1000  # never dereferenced: every call below fails argument checks first


def call_single(numel=256, grad_dtype=0, grad_numel=None, ea_dt=3, ea_n=None, easq_dt=3, easq_n=0,
                scales=2, step=1, bits=4, block=128, prof_n=0, rounding=0):
    L = mdq_hip.lib()
    grad_numel = numel if grad_numel is None else grad_numel
    ea_n = numel if ea_n is None else ea_n
    return L.stq_fused_mdq_adamw(
        FAKE, FAKE, grad_dtype, grad_numel, numel, FAKE, ea_dt, ea_n, FAKE, easq_dt, easq_n,
        FAKE, scales, FAKE, scales, FAKE, scales, 0.9, 0.999, 1e-3, 0.01, 1e-8, step, bits, block,
        FAKE if prof_n else None, prof_n, rounding, 0, 0, None)


def err():
    return mdq_hip.lib().stq_last_error().decode()


@pytest.mark.parametrize("kw,msg", [
    (dict(ea_dt=5, easq_dt=3, easq_n=256), "MDQ: state must be packed4 (uint8+empty), (int8,uint8), (int16,uint16) or (int32,uint32), got Short / Byte bits=4"),
    (dict(ea_n=255), "packed4: exp_avg numel must match parameters"),
    (dict(prof_n=3), "profile_cycles needs >= 5 elements"),
    (dict(block=96), "block_size must be a power of two"),
    (dict(block=0), "block_size must be >= 1"),
    (dict(scales=1), "scale_m / scale_v / v_min need ceil(numel / 128) = 2 elements"),
    (dict(step=0), "step must be >= 1"),
    (dict(ea_dt=4, easq_dt=3, easq_n=256, bits=9), "bits=9 does not fit the 8-bit code storage"),
    (dict(grad_numel=255), "grad numel (255) must match parameters (256)"),
    (dict(grad_dtype=7), "grad must be Float, BFloat16 or Half, got Int"),
    (dict(rounding=2), "rounding must be 0 (nearest) or 1 (stochastic)"),
    (dict(ea_dt=4, easq_dt=3, easq_n=10), "exp_avg / exp_avg_sq must hold numel (256) codes"),
])
def test_argument_errors(kw, msg):
    assert call_single(**kw) == _capi.STQ_ERR_INVALID
    assert msg in err()


@pytest.mark.parametrize("which", ["p", "grad", "exp_avg", "exp_avg_sq", "scale_m"])
def test_pointers_off_their_element_size_are_rejected(which):
    # int16 / uint16 codes and bf16 grads: p and the scales need 4 bytes, the rest 2
    L = mdq_hip.lib()
    ptr = {k: FAKE for k in ("p", "grad", "exp_avg", "exp_avg_sq", "scale_m")}
    ptr[which] = FAKE + (2 if which in ("p", "scale_m") else 1)
    rc = L.stq_fused_mdq_adamw(
        ptr["p"], ptr["grad"], 1, 256, 256, ptr["exp_avg"], 5, 256, ptr["exp_avg_sq"], 6, 256,
        ptr["scale_m"], 2, FAKE, 2, FAKE, 2, 0.9, 0.999, 1e-3, 0.01, 1e-8, 1, 16, 128,
        None, 0, 0, 0, 0, None)
    assert rc == _capi.STQ_ERR_INVALID
    assert "aligned to their element size" in err()


def test_block_size_above_1024_is_clamped_like_the_reference():
    # min(block_size, 1024) (stquant_kernel.cu:421): 4096 -> 1024, so 1 scale suffices for 256
    assert call_single(block=4096, scales=0) == _capi.STQ_ERR_INVALID
    assert "ceil(numel / 1024) = 1" in err()


def test_empty_calls_are_no_ops():
    L = mdq_hip.lib()
    assert call_single(numel=0, scales=0) == _capi.STQ_OK
    assert L.stq_multi_tensor_mdq_adamw(None, 0, 0, 3, 3, 128, 0, 0, None, 0, None) == _capi.STQ_OK


def test_multi_tensor_rejects_mixed_storage():
    L = mdq_hip.lib()
    arr = (_capi.StqTensor * 2)()
    for i, s in enumerate(arr):
        s.p = s.grad = s.exp_avg = s.scale_m = s.scale_v = s.v_min = FAKE
        s.exp_avg_sq = FAKE if i else None
        s.numel = s.grad_numel = s.exp_avg_numel = 256
        s.exp_avg_sq_numel = 256 if i else 0
        s.scale_m_numel = s.scale_v_numel = s.v_min_numel = 2
        s.beta1, s.beta2, s.lr, s.weight_decay, s.eps = 0.9, 0.999, 1e-3, 0.0, 1e-8
        s.step, s.bits = 1, 4
    # tensor 0 is packed4 (empty v codes), tensor 1 would be uint8+uint8: not a valid pair
    rc = L.stq_multi_tensor_mdq_adamw(arr, 2, 0, 3, 3, 128, 0, 0, None, 0, None)
    assert rc == _capi.STQ_ERR_INVALID and "MDQ: state must be packed4" in err()


@pytest.mark.parametrize("off,block", [(-128, 128), (64, 128), (1, 2), (1000, 4096)])
def test_multi_tensor_rejects_bad_elem_offset(off, block):
    """elem_offset (a piece's start in its tensor's stochastic-rounding stream) must be >= 0 and a
    multiple of min(block_size, 1024)."""
    arr = (_capi.StqTensor * 1)()
    s = arr[0]
    s.p = s.grad = s.exp_avg = s.scale_m = s.scale_v = s.v_min = FAKE
    s.numel = s.grad_numel = s.exp_avg_numel = 256
    s.scale_m_numel = s.scale_v_numel = s.v_min_numel = 256
    s.beta1, s.beta2, s.lr, s.weight_decay, s.eps = 0.9, 0.999, 1e-3, 0.0, 1e-8
    s.step, s.bits, s.elem_offset = 1, 4, off
    rc = mdq_hip.lib().stq_multi_tensor_mdq_adamw(arr, 1, 0, 3, 3, block, 1, 0, None, 0, None)
    B = min(block, 1024)
    assert rc == _capi.STQ_ERR_INVALID
    assert f"elem_offset ({off}) must be >= 0 and a multiple of the block size {B}" in err()


def test_shard_states_set_elem_offsets():
    n, B, world = 1000, 64, 3
    t = torch.zeros(n)
    e = mdq_hip.TensorState(t, t, t.to(torch.uint8), torch.empty(0, dtype=torch.uint8), t[:16], t[:16], t[:16],
                            1, 4, 1e-3, 0.9, 0.999, 1e-8, 0.0, 7, elem_offset=640)
    got = [mdq_hip.shard_states([e], B, world, r)[0].elem_offset for r in range(world)]
    assert got == [640 + s for s, _ in mdq_hip.block_aligned_ranges(n, B, world)] == [640, 640 + 384, 640 + 704]


class StqCodeOut(ctypes.Structure):
    _fields_ = [("exp_avg", ctypes.c_void_p), ("exp_avg_sq", ctypes.c_void_p),
                ("exp_avg_numel", ctypes.c_int64), ("exp_avg_sq_numel", ctypes.c_int64)]


def call_restore(src=2, dst=0, bits=4, block=128, numel=256, src_m=FAKE, src_v=FAKE + 4096, dst_m=FAKE + 8192,
                 dst_v=None, src_n=None, dst_n=None):
    """stq_multi_tensor_mdq_adamw_restore on one tensor of fake (never dereferenced) pointers."""
    t = (_capi.StqTensor * 1)()
    s = t[0]
    s.p, s.grad, s.scale_m, s.scale_v, s.v_min = FAKE, FAKE, FAKE, FAKE, FAKE
    s.exp_avg, s.exp_avg_sq = src_m, (None if src == 0 else src_v)
    s.numel = s.grad_numel = numel
    s.exp_avg_numel = numel if src_n is None else src_n
    s.exp_avg_sq_numel = 0 if src == 0 else (numel if src_n is None else src_n)
    s.scale_m_numel = s.scale_v_numel = s.v_min_numel = (numel + block - 1) // block
    s.beta1, s.beta2, s.lr, s.weight_decay, s.eps = 0.9, 0.999, 1e-3, 0.0, 1e-8
    s.step, s.bits = 1, bits
    o = (StqCodeOut * 1)()
    o[0].exp_avg, o[0].exp_avg_sq = dst_m, dst_v
    o[0].exp_avg_numel = numel if dst_n is None else dst_n
    o[0].exp_avg_sq_numel = 0 if dst == 0 else (numel if dst_n is None else dst_n)
    return mdq_hip.lib().stq_multi_tensor_mdq_adamw_restore(t, o, 1, 0, src, dst, block, 0, 0, None, 0, None)


@pytest.mark.parametrize("kw,msg", [
    (dict(src=0, dst=0), "source and destination storage are the same"),
    (dict(block=512), "block size must be 64, 128 or 256, got 512"),
    (dict(block=32), "block size must be 64, 128 or 256, got 32"),
    (dict(src=1, dst=2, bits=4, dst_v=FAKE + 65536), "bits=4 is not stored in destination storage 2"),
    (dict(dst=1, bits=16, dst_v=FAKE + 65536), "bits=16 is not stored in destination storage 1"),
    (dict(dst=3, src=1, bits=24, dst_v=FAKE + 65536), "bits=24 is not stored in destination storage 3"),
    (dict(src_n=100), "source codes must hold numel (256) codes"),
    (dict(dst_n=100), "packed4: exp_avg numel must match parameters"),
    (dict(dst_m=FAKE + 4096 + 100), "source and destination codes overlap"),
    (dict(src=5), "storage must be STQ_STORE_P4 .. STQ_STORE_S32"),
    # int16 / int32 source codes are read with element-sized loads
    (dict(src=2, src_m=FAKE + 1), "data pointers must be aligned to their element size"),
    (dict(src=2, src_v=FAKE + 4096 + 1), "data pointers must be aligned to their element size"),
    (dict(src=3, src_m=FAKE + 2), "data pointers must be aligned to their element size"),
])
def test_restore_argument_errors(kw, msg):
    assert call_restore(**kw) == _capi.STQ_ERR_INVALID
    assert msg in err()


def test_restore_empty_list_is_a_no_op():
    L = mdq_hip.lib()
    assert L.stq_multi_tensor_mdq_adamw_restore(None, None, 0, 0, 2, 0, 128, 0, 0, None, 0, None) == _capi.STQ_OK
    assert call_restore(numel=0) == _capi.STQ_OK


def _state(n=300, B=128, dev="cpu"):
    nb = (n + B - 1) // B
    import torch
    return mdq_hip.TensorState(torch.zeros(n), torch.zeros(n), torch.full((n,), 8, dtype=torch.uint8),
                               torch.empty(0, dtype=torch.uint8), torch.zeros(nb, device=dev),
                               torch.zeros(nb), torch.full((nb,), -20.0), 1, 4, 1e-3, 0.9, 0.999, 1e-8, 0.01)


def test_host_tensors_are_rejected_before_any_launch():
    """The reference raises for non-CUDA tensors (stquant_kernel.cu:424-425); nothing reaches the
    C ABI (which would hand host pointers to a kernel)."""
    plan = mdq_hip.MultiTensorPlan([_state()], 128)
    with pytest.raises(RuntimeError, match="p/grad must be CUDA"):
        plan.run()
    import torch
    e = _state()
    with pytest.raises(RuntimeError, match="p/grad must be CUDA"):
        mdq_hip.multi_tensor_restore([e], [(torch.zeros(300, dtype=torch.int8), torch.zeros(300, dtype=torch.uint8))],
                                     128)


def test_state_tensors_on_another_device_are_rejected():
    with pytest.raises(RuntimeError, match="scale_m must be on the params' device"):
        mdq_hip.MultiTensorPlan([_state(dev="meta")], 128)
