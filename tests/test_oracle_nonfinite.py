"""Pins the oracle on NaN and infinite grads to the reference's arithmetic (stquant_kernel.cu).
Its block reductions are fmaxf / fminf trees (:26-50), which ignore NaN unless every lane is NaN.
A NaN quotient passes its clamps (:113-127) into an (int) conversion, which gives 0 on the
reference's target (PTX cvt maps NaN to 0).  Hence, checked here without the oracle's formulas:

* a NaN grad at element i leaves its block's scales, every other code and every other param
  exactly as they are when element i is a copy of another element j of the block (same grad and
  codes, so its |m| and log v move no max or min); element i gets codes 0 (packed byte 0x08) and
  a NaN param;
* a +-inf grad makes |m| and log v infinite: scale_m = scale_v = inf, v_min as in the stand-in
  run, every code of the block 0 (finite / inf = 0, inf / inf = NaN -> 0), p NaN at that element
  and the other params as in the stand-in run;
* a block of NaN grads only: NaN scales, codes 0, NaN params; other blocks untouched;
* the step after a NaN grad runs on finite state again (codes 0 decode to m = 0, v = e^vmin).
"""
import numpy as np
import pytest

from oracle import mdq_oracle as orc

HP = dict(beta1=0.9, beta2=0.999, lr=1e-3, weight_decay=0.01, eps=1e-8)
WIDTH = {orc.STORE_P4: 4, orc.STORE_S8: 8, orc.STORE_S16: 16, orc.STORE_S32: 32}
CASES = [(s, B, r) for s in WIDTH for B in (64, 128) for r in (orc.ROUND_NEAREST, orc.ROUND_STOCHASTIC)
         if not (s == orc.STORE_S32 and r == orc.ROUND_STOCHASTIC)]


def warm_state(n, B, storage, rng):
    """p and a state after two ordinary steps (non-trivial codes and scales)."""
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    st = list(orc.init_state(n, B, storage))
    for t in (1, 2):
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        orc.step(p, g, *st, step=t, bits=WIDTH[storage], block_size=B, storage=storage, **HP)
    return p, st


def clone(p, st):
    return p.copy(), [None if a is None else a.copy() for a in st]


def run(p, st, g, storage, B, rounding):
    orc.step(p, g, *st, step=3, bits=WIDTH[storage], block_size=B, storage=storage, rounding=rounding, seed=9,
             tensor_id=2, **HP)


def codes_at(st, storage, idx):
    """(m code, v code) at the given indices."""
    cm, cv = st[0], st[1]
    if storage == orc.STORE_P4:
        b = cm[idx].astype(np.int64)
        return (b & 15) - 8, b >> 4
    return cm[idx].astype(np.int64), cv[idx].astype(np.int64)


def copy_element(st, storage, i, j):
    st[0][i] = st[0][j]
    if storage != orc.STORE_P4:
        st[1][i] = st[1][j]


@pytest.mark.parametrize("storage,B,rounding", CASES)
def test_nan_grad_is_ignored_by_its_block(storage, B, rounding):
    rng = np.random.default_rng(storage * 10 + B + rounding)
    n = 3 * B + 37
    p, st = warm_state(n, B, storage, rng)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    others = np.ones(n, bool)
    nan_at = [B, B + 5, 3 * B + 11]              # a block's first lane, another lane, the ragged tail
    pa, sa = clone(p, st)
    pb, sb = clone(p, st)
    ga, gb = g.copy(), g.copy()
    for i in nan_at:
        j = i + 1
        ga[i] = np.nan
        gb[i] = g[j]
        copy_element(sb, storage, i, j)
        copy_element(sa, storage, i, j)          # same codes before the step: only the grad differs
        others[i] = False
    run(pa, sa, ga, storage, B, rounding)
    run(pb, sb, gb, storage, B, rounding)
    for k in (2, 3, 4):
        assert np.array_equal(sa[k].view(np.uint32), sb[k].view(np.uint32)), k
    ma, va = codes_at(sa, storage, np.arange(n))
    mb, vb = codes_at(sb, storage, np.arange(n))
    assert np.array_equal(ma[others], mb[others]) and np.array_equal(va[others], vb[others])
    assert np.all(ma[nan_at] == 0) and np.all(va[nan_at] == 0)
    if storage == orc.STORE_P4:
        assert np.all(sa[0][nan_at] == 0x08)
    assert np.array_equal(pa[others].view(np.uint32), pb[others].view(np.uint32))
    assert np.all(np.isnan(pa[nan_at]))
    # the next step decodes codes 0 to m = 0, v = e^vmin: finite state again
    g2 = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    orc.step(pa, g2, *sa, step=4, bits=WIDTH[storage], block_size=B, storage=storage, **HP)
    assert np.all(np.isfinite(sa[2])) and np.all(np.isfinite(sa[3])) and np.all(np.isfinite(sa[4]))
    assert np.all(np.isfinite(pa[others])) and np.all(np.isnan(pa[nan_at]))


@pytest.mark.parametrize("sign", [1.0, -1.0])
@pytest.mark.parametrize("storage,B,rounding", CASES)
def test_infinite_grad_saturates_its_block(storage, B, rounding, sign):
    rng = np.random.default_rng(100 + storage * 10 + B + rounding)
    n = 3 * B + 37
    p, st = warm_state(n, B, storage, rng)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    i, j = 2 * B + 7, 2 * B + 9
    blk = i // B
    pa, sa = clone(p, st)
    pb, sb = clone(p, st)
    ga, gb = g.copy(), g.copy()
    ga[i] = sign * np.inf
    gb[i] = g[j]
    copy_element(sa, storage, i, j)
    copy_element(sb, storage, i, j)
    run(pa, sa, ga, storage, B, rounding)
    run(pb, sb, gb, storage, B, rounding)
    assert sa[2][blk] == np.inf and sa[3][blk] == np.inf
    assert sa[4][blk] == sb[4][blk]
    rest = np.ones(len(sa[2]), bool)
    rest[blk] = False
    for k in (2, 3, 4):
        assert np.array_equal(sa[k][rest].view(np.uint32), sb[k][rest].view(np.uint32)), k
    inb = np.zeros(n, bool)
    inb[blk * B:(blk + 1) * B] = True
    ma, va = codes_at(sa, storage, np.arange(n))
    mb, vb = codes_at(sb, storage, np.arange(n))
    assert np.all(ma[inb] == 0) and np.all(va[inb] == 0)
    assert np.array_equal(ma[~inb], mb[~inb]) and np.array_equal(va[~inb], vb[~inb])
    others = np.ones(n, bool)
    others[i] = False
    assert np.isnan(pa[i])
    assert np.array_equal(pa[others].view(np.uint32), pb[others].view(np.uint32))


@pytest.mark.parametrize("storage", list(WIDTH))
def test_all_nan_block_gets_nan_scales(storage):
    rng = np.random.default_rng(7 + storage)
    B = 64
    n = 4 * B
    p, st = warm_state(n, B, storage, rng)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    pa, sa = clone(p, st)
    pb, sb = clone(p, st)
    ga = g.copy()
    ga[B:2 * B] = np.nan
    run(pa, sa, ga, storage, B, orc.ROUND_NEAREST)
    run(pb, sb, g, storage, B, orc.ROUND_NEAREST)
    assert np.isnan(sa[2][1]) and np.isnan(sa[3][1]) and np.isnan(sa[4][1])
    for k in (2, 3, 4):
        assert np.array_equal(np.delete(sa[k], 1).view(np.uint32), np.delete(sb[k], 1).view(np.uint32))
    ma, va = codes_at(sa, storage, np.arange(B, 2 * B))
    assert np.all(ma == 0) and np.all(va == 0)
    assert np.all(np.isnan(pa[B:2 * B]))
    keep = np.r_[0:B, 2 * B:n]
    assert np.array_equal(pa[keep].view(np.uint32), pb[keep].view(np.uint32))
