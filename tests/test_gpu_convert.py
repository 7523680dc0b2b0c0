"""Code-storage conversion on the GPU (stq_multi_tensor_convert_codes) against the element-wise
model of the reference's storage rules on a bit-width change (tests/storage_model.py,
stquant_opt_simple.py:140-219): every source storage x every target bit width, codes spanning
each source type's full range (so every clamp is hit), sizes around the 4096-element tile,
several tensors per launch.  Bit-exact."""
import numpy as np
import pytest
import torch

import mdq_hip
from mdq_hip import storage
from storage_model import after_kernel, before_kernel, model_arrays

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


def _model(fn, src, cm, cv, bits):
    """The storage model applied to CPU codes of layout ``src`` (a storage constant or a SRC key)."""
    src = _STORE.get(src, src)
    m = as_i64(cm).numpy()
    v = np.zeros_like(m) if src == storage.STORE_P4 else as_i64(cv).numpy()
    return model_arrays(fn, src, m, v, bits)


@pytest.mark.parametrize("src", list(SRC))
@pytest.mark.parametrize("bits", [4, 8, 16, 32])
def test_align_matches_reference(src, bits):
    print(f"case: convert align {src} -> bits {bits}", flush=True)
    states, items, want = [], [], []
    for k, n in enumerate(SIZES):
        cm, cv = rand_codes(src, n, 100 * bits + k)
        want.append(_model(before_kernel, src, cm, cv, bits))
        gm, gv = cm.to(DEV), cv.to(DEV)
        dst = storage.kernel_layout(bits)
        nm, nv = mdq_hip.empty_codes(gm, dst)
        items.append((gm, gv, nm, nv))
        states.append((nm, nv))
    mdq_hip.convert_codes(items)
    torch.cuda.synchronize()
    for (nm, nv), (lay, m, v), n in zip(states, want, SIZES):
        assert storage.layout_of(nm, nv) == lay, (n, nm.dtype, nv.dtype)
        assert np.array_equal(as_i64(nm.cpu()).numpy(), m), f"m codes, n={n}"
        assert np.array_equal(as_i64(nv.cpu()).numpy(), v), f"v codes, n={n}"


@pytest.mark.parametrize("src,bits", [("s16", 4), ("p4", 8), ("s8", 16)])
def test_thousands_of_small_tensors_one_launch(src, bits):
    """2000 tensors of 1 to 3000 elements (log-uniform) aligned in one launch, the usual
    transitions of the MDQ schedule: every tensor against the storage model."""
    print(f"case: convert 2000 tensors {src} -> bits {bits}", flush=True)
    rng = np.random.default_rng(2000 + bits)
    sizes = [int(x) for x in np.floor(np.exp(rng.uniform(0, np.log(3000), 2000)))]
    items, states, want = [], [], []
    for k, n in enumerate(sizes):
        cm, cv = rand_codes(src, n, 9000 + k)
        want.append(_model(before_kernel, src, cm, cv, bits))
        gm, gv = cm.to(DEV), cv.to(DEV)
        nm, nv = mdq_hip.empty_codes(gm, storage.kernel_layout(bits))
        items.append((gm, gv, nm, nv))
        states.append((nm, nv))
    mdq_hip.convert_codes(items)
    torch.cuda.synchronize()
    for k, ((nm, nv), (lay, m, v)) in enumerate(zip(states, want)):
        assert storage.layout_of(nm, nv) == lay, (k, nm.dtype, nv.dtype)
        assert np.array_equal(as_i64(nm.cpu()).numpy(), m), f"m codes, tensor {k}"
        assert np.array_equal(as_i64(nv.cpu()).numpy(), v), f"v codes, tensor {k}"


def test_pack_to_nibbles_matches_reference():
    items, want, outs = [], [], []
    for k, n in enumerate(SIZES):
        cm, cv = rand_codes("s8", n, 7 + k)
        want.append(_model(after_kernel, storage.STORE_S8, cm, cv, 4)[1])
        gm, gv = cm.to(DEV), cv.to(DEV)
        nm, nv = mdq_hip.empty_codes(gm, mdq_hip.STORE_P4)
        items.append((gm, gv, nm, nv))
        outs.append((nm, nv))
    mdq_hip.convert_codes(items)
    torch.cuda.synchronize()
    for (nm, nv), w, n in zip(outs, want, SIZES):
        assert nm.dtype == torch.uint8 and nv.numel() == 0
        assert np.array_equal(nm.cpu().numpy().astype(np.int64), w), f"n={n}"


def test_empty_tensors_are_a_no_op():
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


_RANGE = {"p4": ((-8, 7), (0, 15)), "s8": ((-128, 127), (0, 255)), "s16": ((-32768, 32767), (0, 65535)),
          "s32": ((-2 ** 31, 2 ** 31 - 1), (0, 2 ** 32 - 1))}
_STORE = {"p4": mdq_hip.STORE_P4, "s8": mdq_hip.STORE_S8, "s16": mdq_hip.STORE_S16, "s32": mdq_hip.STORE_S32}


def _decode(kind, cm, cv):
    """(m, v) as int64 numpy arrays: P4 bytes give m = (b & 15) - 8, v = b >> 4."""
    if kind == "p4":
        b = cm.numpy().astype(np.int64)
        return (b & 15) - 8, b >> 4
    return as_i64(cm).numpy(), as_i64(cv).numpy()


@pytest.mark.parametrize("src", list(SRC))
@pytest.mark.parametrize("dst", list(SRC))
def test_every_storage_pair_matches_the_value_map(src, dst):
    """All 16 (src, dst) pairs the C ABI accepts, in one launch per pair: two whole-tile tensors
    (vector path), a ragged one, and an unaligned view (storage offset 1: element path).  Every
    code is decode(src) clamped to dst's range; P4 stores clamp(m + 8, 0, 15) | clamp(v, 0, 15) << 4."""
    print(f"case: convert pair {src} -> {dst}", flush=True)
    sizes = [4096 * 3, 8192, 4096 * 2 + 777, 5000]
    items, want, outs = [], [], []
    for k, n in enumerate(sizes):
        unaligned = k == len(sizes) - 1
        cm, cv = rand_codes(src, n + (1 if unaligned else 0), 1000 + 31 * k + 7 * len(src) + len(dst))
        gm, gv = cm.to(DEV), cv.to(DEV)
        if unaligned:
            cm, gm = cm[1:], gm[1:]
            if src != "p4":
                cv, gv = cv[1:], gv[1:]
        m, v = _decode(src, cm, cv)
        (mlo, mhi), (vlo, vhi) = _RANGE[dst]
        m, v = np.clip(m, mlo, mhi), np.clip(v, vlo, vhi)
        want.append((m + 8) | (v << 4) if dst == "p4" else (m, v))
        nm, nv = mdq_hip.empty_codes(gm, _STORE[dst])
        if unaligned and dst != "p4":
            # destination views at an odd element offset too
            bm, bv = mdq_hip.empty_codes(torch.empty(n + 1, device=DEV), _STORE[dst])
            nm, nv = bm[1:], bv[1:]
        elif unaligned:
            nm = torch.empty(n + 1, dtype=torch.uint8, device=DEV)[1:]
        items.append((gm, gv, nm, nv))
        outs.append((nm, nv))
    mdq_hip.convert_codes(items)
    torch.cuda.synchronize()
    for (nm, nv), w, n in zip(outs, want, sizes):
        if dst == "p4":
            assert np.array_equal(nm.cpu().numpy().astype(np.int64), w), f"n={n}"
        else:
            assert np.array_equal(as_i64(nm.cpu()).numpy(), w[0]), f"m codes, n={n}"
            assert np.array_equal(as_i64(nv.cpu()).numpy(), w[1]), f"v codes, n={n}"
