"""The code layouts and their value map (``mdq_hip.storage``) against the element-wise model of
the reference's storage rules (tests/storage_model.py, /root/reference/CUDA/stquant_opt_simple.py:
140-210) on CPU tensors: every source layout x width, codes over each type's full range."""
import numpy as np
import pytest
import torch

from mdq_hip import storage as S
from storage_model import after_kernel, before_kernel, model_arrays

DT = {S.STORE_S8: (torch.int8, torch.uint8), S.STORE_S16: (torch.int16, torch.uint16),
      S.STORE_S32: (torch.int32, torch.uint32)}


def i64(t):
    return t.to(torch.int64).numpy()


def rand_codes(src, n, seed):
    """Codes of layout ``src``: half near zero, half over the whole range of the type, plus
    both ends of it."""
    rng = np.random.default_rng(seed)
    if src == S.STORE_P4:
        b = rng.integers(0, 256, n)
        b[:2] = (0, 255)
        return torch.from_numpy(b.astype(np.uint8)), torch.empty(0, dtype=torch.uint8)
    lay = S.LAYOUTS[src]
    m = np.where(rng.random(n) < 0.5, rng.integers(-20, 20, n), rng.integers(lay.m_lo, lay.m_hi, n, endpoint=True))
    v = np.where(rng.random(n) < 0.5, rng.integers(0, 20, n), rng.integers(0, lay.v_hi, n, endpoint=True))
    m[:2], v[:2] = (lay.m_lo, lay.m_hi), (0, lay.v_hi)
    dm, dv = DT[src]
    return torch.from_numpy(m).to(dm), torch.from_numpy(v).to(dv)


def model_inputs(src, cm, cv):
    if src == S.STORE_P4:
        return i64(cm), np.zeros(cm.numel(), np.int64)
    return i64(cm), i64(cv)


@pytest.mark.parametrize("src", [S.STORE_P4, S.STORE_S8, S.STORE_S16, S.STORE_S32])
@pytest.mark.parametrize("bits", [4, 8, 16, 32])
def test_kernel_and_resting_layouts_follow_the_reference_rules(src, bits):
    cm, cv = rand_codes(src, 3000, 10 * src + bits)
    m, v = model_inputs(src, cm, cv)
    # before the kernel: the width's kernel layout
    lay, mm, vv = model_arrays(before_kernel, src, m, v, bits)
    assert S.kernel_layout(bits) == lay
    km, kv = S.restore(cm, cv, S.kernel_layout(bits))
    assert S.layout_of(km, kv) == lay
    assert np.array_equal(i64(km), mm) and np.array_equal(i64(kv), vv)
    # after the kernel: the width's resting layout
    lay2, pm, pv = model_arrays(after_kernel, lay, mm, vv, bits)
    assert S.resting_layout(bits) == lay2
    rm, rv = S.restore(km, kv, S.resting_layout(bits))
    assert S.layout_of(rm, rv) == lay2
    assert np.array_equal(i64(rm), pm)
    assert (pv is None and rv.numel() == 0) or np.array_equal(i64(rv), pv)


def test_narrowing_clamps_codes():
    # int16 codes -> int8 by clamping (the reference keeps the scales: quirk Q4), then nibbles
    m, v = torch.tensor([300, -300, 5], dtype=torch.int16), torch.tensor([1000, 3, 255], dtype=torch.uint16)
    a, b = S.restore(m, v, S.STORE_S8)
    assert a.tolist() == [127, -128, 5] and a.dtype == torch.int8
    assert b.tolist() == [255, 3, 255] and b.dtype == torch.uint8
    a, b = S.restore(a, b, S.STORE_P4)
    assert a.tolist() == [15 | (15 << 4), 0 | (3 << 4), 13 | (15 << 4)] and b.numel() == 0
    a, b = S.restore(a, b, S.STORE_S8)
    assert a.tolist() == [7, -8, 5] and b.tolist() == [15, 3, 15]


def test_every_packed_byte_round_trips():
    byte = torch.arange(256, dtype=torch.int64).to(torch.uint8)
    m, v = S.decode(byte, torch.empty(0, dtype=torch.uint8))
    assert m.tolist() == [(b & 15) - 8 for b in range(256)] and v.tolist() == [b >> 4 for b in range(256)]
    for kind in (S.STORE_S8, S.STORE_S16, S.STORE_S32):
        wide = S.encode(m, v, kind)
        assert torch.equal(S.restore(*wide, S.STORE_P4)[0], byte)


def test_layout_of_and_empty_tensors():
    e8 = torch.empty(0, dtype=torch.uint8)
    assert S.layout_of(torch.zeros(3, dtype=torch.uint8), e8) == S.STORE_P4
    assert S.layout_of(e8, e8) == S.STORE_P4
    with pytest.raises(RuntimeError):
        S.layout_of(torch.zeros(3, dtype=torch.int16), torch.zeros(3, dtype=torch.uint8))
    for kind in range(4):
        m, v = S.restore(torch.empty(0, dtype=torch.int16), torch.empty(0, dtype=torch.uint16), kind)
        assert S.layout_of(m, v) == kind and m.numel() == 0
    assert S.resting_layout(20) is None and S.kernel_layout(20) == S.STORE_S16
