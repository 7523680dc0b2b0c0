"""Code-storage conversion on the GPU (stq_multi_tensor_convert_codes) against the reference's own
torch restatement of the storage changes (MDQAdamWSimple._align_momentum_storage /
_pack_momentum_storage, stquant_opt_simple.py:140-219) run on CPU copies: every source storage x
every target bit width, codes spanning each source type's full range (so every clamp is hit),
sizes around the 4096-element tile, several tensors per launch.  Bit-exact."""
import numpy as np
import pytest
import torch

import mdq_hip
from stquant_opt_simple import MDQAdamWSimple

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SIZES = [1, 7, 4095, 4096, 4097, 100_003]
SRC = {"p4": (torch.uint8, None), "s8": (torch.int8, torch.uint8), "s16": (torch.int16, torch.uint16),
       "s32": (torch.int32, torch.uint32)}


def rand_codes(kind, n, seed):
    rng = np.random.default_rng(seed)
    dm, dv = SRC[kind]
    if kind == "p4":
        return torch.from_numpy(rng.integers(0, 256, n, dtype=np.uint8)), torch.empty(0, dtype=torch.uint8)
    info_m, info_v = torch.iinfo(dm), torch.iinfo(dv)
    # half the values near zero (in range of every narrower type), half over the full range
    m = np.where(rng.random(n) < 0.5, rng.integers(-20, 20, n), rng.integers(info_m.min, info_m.max, n, endpoint=True))
    v = np.where(rng.random(n) < 0.5, rng.integers(0, 20, n), rng.integers(0, info_v.max, n, endpoint=True))
    return torch.from_numpy(m).to(dm), torch.from_numpy(v.astype(np.int64)).to(dv)


def as_i64(t):
    if t.dtype == torch.uint16:
        return t.view(torch.int16).to(torch.int64) & 0xFFFF
    if t.dtype == torch.uint32:
        return t.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    return t.to(torch.int64)


@pytest.mark.parametrize("src", list(SRC))
@pytest.mark.parametrize("bits", [4, 8, 16, 32])
def test_align_matches_reference(src, bits):
    print(f"case: convert align {src} -> bits {bits}", flush=True)
    states, items, want = [], [], []
    for k, n in enumerate(SIZES):
        cm, cv = rand_codes(src, n, 100 * bits + k)
        ref = {"exp_avg": cm.clone(), "exp_avg_sq": cv.clone()}
        MDQAdamWSimple._align_momentum_storage(ref, bits)
        want.append(ref)
        gm, gv = cm.to(DEV), cv.to(DEV)
        dst = MDQAdamWSimple._aligned_storage(bits)
        nm, nv = mdq_hip.empty_codes(gm, dst)
        items.append((gm, gv, nm, nv))
        states.append((nm, nv))
    mdq_hip.convert_codes(items)
    torch.cuda.synchronize()
    for (nm, nv), ref, n in zip(states, want, SIZES):
        assert nm.dtype == ref["exp_avg"].dtype and nv.dtype == ref["exp_avg_sq"].dtype, (n, nm.dtype, nv.dtype)
        assert torch.equal(as_i64(nm.cpu()), as_i64(ref["exp_avg"])), f"m codes, n={n}"
        assert torch.equal(as_i64(nv.cpu()), as_i64(ref["exp_avg_sq"])), f"v codes, n={n}"


def test_pack_to_nibbles_matches_reference():
    items, want, outs = [], [], []
    for k, n in enumerate(SIZES):
        cm, cv = rand_codes("s8", n, 7 + k)
        ref = {"exp_avg": cm.clone(), "exp_avg_sq": cv.clone()}
        MDQAdamWSimple._pack_momentum_storage(ref, 4)
        want.append(ref["exp_avg"])
        gm, gv = cm.to(DEV), cv.to(DEV)
        nm, nv = mdq_hip.empty_codes(gm, mdq_hip.STORE_P4)
        items.append((gm, gv, nm, nv))
        outs.append((nm, nv))
    mdq_hip.convert_codes(items)
    torch.cuda.synchronize()
    for (nm, nv), w, n in zip(outs, want, SIZES):
        assert nm.dtype == torch.uint8 and nv.numel() == 0
        assert torch.equal(nm.cpu(), w), f"n={n}"


def test_empty_tensors_are_a_no_op():
    # (the optimizer keeps the reference's torch path for empty tensors, whose dtype rules differ)
    e8, e16 = torch.empty(0, dtype=torch.int8, device=DEV), torch.empty(0, dtype=torch.int16, device=DEV)
    out = mdq_hip.empty_codes(e16, mdq_hip.STORE_S8)
    mdq_hip.convert_codes([(e16, torch.empty(0, dtype=torch.uint16, device=DEV), *out),
                           (e8, torch.empty(0, dtype=torch.uint8, device=DEV), *mdq_hip.empty_codes(e8, mdq_hip.STORE_S32))])
    torch.cuda.synchronize()
    assert out[0].numel() == 0 and out[0].dtype == torch.int8


def test_rejects_bad_arguments():
    a = torch.zeros(8, dtype=torch.int16, device=DEV)
    with pytest.raises(RuntimeError):
        mdq_hip.convert_codes([(a, a.to(torch.uint16), torch.zeros(9, dtype=torch.int8, device=DEV),
                                torch.zeros(9, dtype=torch.uint8, device=DEV))])       # size mismatch
    with pytest.raises(RuntimeError):
        mdq_hip.convert_codes([(a, torch.zeros(8, dtype=torch.int32, device=DEV), a, a)])  # no storage class
