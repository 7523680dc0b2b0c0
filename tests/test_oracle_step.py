"""Pins the oracle's fused step (restating stquant_kernel.cu:53-401) through
closed forms, invariants and special cases that do not re-derive its formulas:

* step 1 from a fresh state is float64 textbook AdamW with v0 = e^-20 (quirks
  Q1, Q2) to 1e-6, at every code width; 16-bit codes track it over 8 steps;
* the requant divisor's + 1e-12 shrinks codes whose scale nears 1e-12;
* lr=0 leaves p bit-identical; g=0 from a zero state gives p*(1-lr*wd) exactly;
* the max-|m| element gets code +7 (positive: +8 clamps, quirk Q6) or -8;
* the min-log-v element gets v code 0 and the max-log-v element 2^bits-1;
* exact ties (k+1/2)*d round away from zero (quirk Q7);
* all 256 packed bytes survive a decode -> encode round trip with b1=b2=1, lr=0;
* tail lanes feed 0 to the reductions (quirk Q3);
* packed-4 storage == int8/uint8 storage at bits=4 (the Simple optimizer's route);
* stochastic rounding is unbiased and only picks the two neighbouring codes.
"""
import numpy as np
import pytest

from oracle import mdq_oracle as orc

HP = dict(beta1=0.9, beta2=0.999, lr=1e-3, weight_decay=0.01, eps=1e-8)


def fresh(n, B, storage):
    return orc.init_state(n, B, storage)


def run(p, g, state, *, step, bits, B, storage, **kw):
    cm, cv, sm, sv, vm = state
    hp = dict(HP)
    hp.update(kw)
    orc.step(p, g, cm, cv, sm, sv, vm, step=step, bits=bits, block_size=B, storage=storage, **hp)


def adamw_f64(p0, grads, lr, b1, b2, eps, wd, v0):
    # hyper-parameters enter the reference kernel as C floats (stquant_core.cpp:6)
    lr, b1, b2, eps, wd = (float(np.float32(x)) for x in (lr, b1, b2, eps, wd))
    p = p0.astype(np.float64)
    m = np.zeros_like(p)
    v = np.full_like(p, v0)
    for t, g in enumerate(grads, start=1):
        g = g.astype(np.float64)
        m = b1 * m + (1 - b1) * g
        v = b2 * v + (1 - b2) * g * g
        mh = m / (1 - b1 ** t)
        p = p * (1 - lr * wd) - lr * mh / (np.sqrt(v) / np.sqrt(1 - b2 ** t) + eps)
    return p


@pytest.mark.parametrize("bits,storage", [(4, orc.STORE_P4), (8, orc.STORE_S8), (32, orc.STORE_S32)])
def test_step1_is_textbook_adamw(bits, storage):
    # The update uses the unquantised m, v of this step (quirk Q2), so from a
    # fresh state step 1 is exactly AdamW with m0 = 0 and v0 = e^-20 (Q1).
    rng = np.random.default_rng(0)
    n, B = 3000, 128
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    p = p0.copy()
    run(p, g, fresh(n, B, storage), step=1, bits=bits, B=B, storage=storage)
    ref = adamw_f64(p0, [g], 1e-3, 0.9, 0.999, 1e-8, 0.01, np.exp(-20.0))
    upd = np.abs(ref - p0.astype(np.float64) * (1 - 1e-5))
    assert np.all(np.abs(p - ref) <= 1e-6 * np.abs(ref) + 1e-6 * upd + 1e-12)
    # and v0 = e^-20 matters: with v0 = 0 the reference would differ measurably
    ref0 = adamw_f64(p0, [g], 1e-3, 0.9, 0.999, 1e-8, 0.01, 0.0)
    assert np.max(np.abs(ref0 - ref)) > 100 * np.max(np.abs(p - ref))


def test_bits16_tracks_textbook_adamw_over_steps():
    # 16-bit codes with O(1) gradients: scales >> 1e-12, so the dequantised state
    # carries m and v across steps to ~1e-4 relative; p tracks float64 AdamW.
    rng = np.random.default_rng(10)
    n, B = 4096, 128
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    grads = [rng.standard_normal(n).astype(np.float32) for _ in range(8)]
    p = p0.copy()
    st = fresh(n, B, orc.STORE_S16)
    for t, g in enumerate(grads, start=1):
        run(p, g, st, step=t, bits=16, B=B, storage=orc.STORE_S16)
    ref = adamw_f64(p0, grads, 1e-3, 0.9, 0.999, 1e-8, 0.01, np.exp(-20.0))
    scale = np.max(np.abs(ref - p0.astype(np.float64)))     # largest total update
    assert np.max(np.abs(p - ref)) < 1e-3 * scale
    # a broken carry (e.g. m not dequantised) would be off by O(1) of the update
    p_nocarry = p0.copy()
    for t, g in enumerate(grads, start=1):
        run(p_nocarry, g, fresh(n, B, orc.STORE_S16), step=t, bits=16, B=B, storage=orc.STORE_S16)
    assert np.max(np.abs(p_nocarry - ref)) > 0.1 * scale


def test_requant_divisor_epsilon_shrinks_tiny_scales():
    # stquant_kernel.cu:113 divides by (scale + 1e-12) while :74,168 multiply the
    # code by scale: once scale_m ~ 1e-12 the stored m shrinks by scale/(scale+1e-12).
    n, B = 128, 128
    g = np.full(n, 1e-3, np.float32)
    g[0] = 2e-3
    st = fresh(n, B, orc.STORE_S32)
    run(np.zeros(n, np.float32), g, st, step=1, bits=32, B=B, storage=orc.STORE_S32)
    sm = float(st[2][0])
    m = float(np.float32(0.1) * np.float32(2e-3))
    deq = float(st[0][0]) * sm
    assert sm < 2e-13                                         # (2e-4 + 1e-12) / 2^31
    assert abs(deq / m - sm / (sm + 1e-12)) < 1e-6            # ~0.085: the quirk, reproduced


def test_lr_zero_keeps_params_and_zero_grad_is_pure_decay():
    rng = np.random.default_rng(1)
    n, B = 1000, 64
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    p = p0.copy()
    run(p, g, fresh(n, B, orc.STORE_P4), step=1, bits=4, B=B, storage=orc.STORE_P4, lr=0.0)
    assert np.array_equal(p.view(np.uint32), p0.view(np.uint32))
    p = p0.copy()
    run(p, np.zeros(n, np.float32), fresh(n, B, orc.STORE_P4), step=1, bits=4, B=B, storage=orc.STORE_P4)
    decay = np.float32(1.0) - np.float32(1e-3) * np.float32(0.01)
    assert np.array_equal(p, p0 * decay)


@pytest.mark.parametrize("bits,storage", [(4, orc.STORE_P4), (4, orc.STORE_S8), (8, orc.STORE_S8),
                                          (16, orc.STORE_S16)])
def test_code_extremes(bits, storage):
    rng = np.random.default_rng(2)
    n, B = 128 * 40, 128
    # O(1) grads at 16 bits keep scale_m >> 1e-12 (see the divisor-epsilon test)
    g = (rng.standard_normal(n) * (1.0 if bits == 16 else 1e-3)).astype(np.float32)
    st = fresh(n, B, storage)
    run(np.zeros(n, np.float32), g, st, step=1, bits=bits, B=B, storage=storage)
    cm, cv, sm, sv, vm = st
    if storage == orc.STORE_P4:
        mcode = (cm & 15).astype(np.int64) - 8
        vcode = (cm >> 4).astype(np.int64)
    else:
        mcode, vcode = cm.astype(np.int64), cv.astype(np.int64)
    qm = 2 ** (bits - 1)
    m = np.float32(0.1) * g                                   # step 1 from a zero state
    for b in range(n // B):
        s = slice(b * B, (b + 1) * B)
        i = int(np.argmax(np.abs(m[s])))
        assert mcode[s][i] == (qm - 1 if m[s][i] > 0 else -qm)
        # max|m| -> scale_m, within fp32 rounding of (M + 1e-12) / qm
        assert abs(sm[b] - (abs(float(m[s][i])) + 1e-12) / qm) <= 1e-6 * sm[b]
        # v: log v is monotone in g^2 at step 1
        g2 = g[s].astype(np.float64) ** 2
        assert vcode[s][int(np.argmin(g2))] == 0
        assert vcode[s][int(np.argmax(g2))] == 2 ** bits - 1
    assert mcode.min() >= -qm and mcode.max() <= qm - 1


def test_exact_ties_round_away_from_zero():
    # beta1 = 0.5 makes m = 0.5 * g exact at step 1; place m on (k + 1/2) * d.
    n, B = 64, 64
    M = np.float32(0.75)
    sm = (M + np.float32(1e-12)) / np.float32(8.0)
    d = sm + np.float32(1e-12)
    ks = np.array([0, 1, 2, 3, 4, 5, 6], np.float64)
    m = np.zeros(n, np.float32)
    m[0] = M
    m[1:8] = ((ks + 0.5) * float(d)).astype(np.float32)
    m[8:15] = -m[1:8]
    exact = np.array_equal(m[1:8].astype(np.float64), (ks + 0.5) * float(d))
    g = (m * np.float32(2.0)).astype(np.float32)
    st = fresh(n, B, orc.STORE_S8)
    run(np.zeros(n, np.float32), g, st, step=1, bits=4, B=B, storage=orc.STORE_S8, beta1=0.5)
    mc = st[0].astype(np.int64)
    assert st[2][0] == sm and exact
    assert list(mc[1:8]) == [1, 2, 3, 4, 5, 6, 7]           # k + 1/2 -> k + 1 (7 after the +7 clamp)
    assert list(mc[8:15]) == [-1, -2, -3, -4, -5, -6, -7]   # -(k + 1/2) -> -(k + 1)


def test_all_packed_bytes_round_trip():
    # Each block holds all 256 bytes under scales that make decode -> encode the identity.
    n, B = 256 * 4, 256
    cm = np.tile(np.arange(256, dtype=np.uint8), 4)
    sm = np.full(4, np.float32(1e-3))
    sv = np.full(4, np.float32(0.4))
    vm = np.full(4, np.float32(-14.0))
    before = cm.copy()
    orc.step(np.zeros(n, np.float32), np.zeros(n, np.float32), cm, None, sm, sv, vm,
             beta1=1.0, beta2=1.0, lr=0.0, weight_decay=0.0, eps=1e-8, step=1, bits=4,
             block_size=B, storage=orc.STORE_P4)
    assert np.array_equal(cm, before)
    assert np.allclose(sm, 1e-3, rtol=1e-6) and np.allclose(sv, 0.4, rtol=1e-5) and np.allclose(vm, -14.0)


def test_tail_lanes_feed_zero():
    rng = np.random.default_rng(4)
    n, B = 128 * 3 + 37, 128
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    st = fresh(n, B, orc.STORE_P4)
    run(np.zeros(n, np.float32), g, st, step=1, bits=4, B=B, storage=orc.STORE_P4)
    _, _, sm, sv, vm = st
    # the ragged last block's Lmax is 0 (padding lanes), so sv = (0 - Lmin + 1e-12) / 15
    assert sv[-1] == (np.float32(0.0) - vm[-1] + np.float32(1e-12)) / np.float32(15.0)
    assert vm[-1] < -10
    assert all(sv[b] < sv[-1] / 2 for b in range(3))


def test_packed4_equals_int8_storage_at_4_bits():
    rng = np.random.default_rng(5)
    n, B = 128 * 17 + 5, 128
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    pa, pb = p0.copy(), p0.copy()
    sa, sb = fresh(n, B, orc.STORE_P4), fresh(n, B, orc.STORE_S8)
    for t in range(1, 6):
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        run(pa, g, sa, step=t, bits=4, B=B, storage=orc.STORE_P4)
        run(pb, g, sb, step=t, bits=4, B=B, storage=orc.STORE_S8)
        packed = ((sb[0].astype(np.int16) + 8).clip(0, 15) | (sb[1].astype(np.int16).clip(0, 15) << 4))
        assert np.array_equal(sa[0], packed.astype(np.uint8))
        for i in (2, 3, 4):
            assert np.array_equal(sa[i], sb[i])
        assert np.array_equal(pa, pb)


def test_stochastic_rounding_unbiased_and_two_valued():
    rng = np.random.default_rng(6)
    n, B = 128 * 8, 128
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    m = np.float32(0.5) * g                                   # exact with beta1 = 0.5
    acc = np.zeros(n)
    seeds = 400
    lo_hi_ok = True
    for seed in range(seeds):
        st = fresh(n, B, orc.STORE_S8)
        run(np.zeros(n, np.float32), g, st, step=1, bits=4, B=B, storage=orc.STORE_S8, beta1=0.5,
            rounding=orc.ROUND_STOCHASTIC, seed=seed)
        d = np.repeat(st[2] + np.float32(1e-12), B).astype(np.float64)
        y = m.astype(np.float64) / d
        c = st[0].astype(np.float64)
        inside = (y > -8) & (y < 7)
        lo_hi_ok &= bool(np.all((c[inside] == np.floor(y[inside])) | (c[inside] == np.floor(y[inside]) + 1)))
        acc += c * d
    assert lo_hi_ok
    mean = acc / seeds
    d = np.repeat(st[2] + np.float32(1e-12), B).astype(np.float64)
    y = m.astype(np.float64) / d
    inside = (y > -7.9) & (y < 6.9)
    # per-element standard error <= d / (2 sqrt(seeds)); allow 5 sigma
    z = np.abs(mean[inside] - m[inside]) / (d[inside] / (2 * np.sqrt(seeds)))
    assert np.mean(z) < 1.0 and np.max(z) < 6.0


def test_stochastic_stream_depends_on_step_tensor_and_seed():
    """The random numbers are a function of (element, tensor id, step, seed): the same state and
    grads stepped with another step number, tensor id or seed round differently somewhere, and
    about half of the elements (each code is an independent coin flip where the quotient sits
    between two codes) change; the same four values reproduce the codes exactly."""
    rng = np.random.default_rng(12)
    n, B = 128 * 16, 128
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)

    def codes(step, tensor_id, seed):
        st = fresh(n, B, orc.STORE_S8)
        run(np.zeros(n, np.float32), g, st, step=step, bits=4, B=B, storage=orc.STORE_S8,
            rounding=orc.ROUND_STOCHASTIC, seed=seed, tensor_id=tensor_id)
        return np.concatenate([st[0].astype(np.int64), st[1].astype(np.int64)])

    base = codes(3, 5, 99)
    assert np.array_equal(base, codes(3, 5, 99))
    for other in (codes(4, 5, 99), codes(3, 6, 99), codes(3, 5, 100)):
        frac = np.mean(base != other)
        assert 0.2 < frac < 0.8, frac


@pytest.mark.parametrize("bad", [dict(block_size=96), dict(bits=5, storage=orc.STORE_P4),
                                 dict(bits=9, storage=orc.STORE_S8), dict(step=0)])
def test_rejects_invalid(bad):
    n = 256
    args = dict(step=1, bits=4, block_size=128, storage=orc.STORE_P4)
    args.update(bad)
    st = fresh(n, 1, orc.STORE_P4 if args["storage"] == orc.STORE_P4 else orc.STORE_S8)
    with pytest.raises(ValueError):
        orc.step(np.zeros(n, np.float32), np.zeros(n, np.float32), st[0], st[1], st[2], st[3], st[4],
                 **HP, **args)


@pytest.mark.parametrize("B,storage,bits", [(2, orc.STORE_S8, 8), (64, orc.STORE_P4, 4), (128, orc.STORE_S16, 16)])
def test_pieces_with_elem_offset_reproduce_the_whole_tensor(B, storage, bits):
    """Stochastic rounding of block-aligned pieces: a piece stepped with elem_offset = its start
    draws the whole tensor's random numbers, so the pieces together give the whole tensor's step
    bit for bit; with offset 0 they do not (each piece would restart the stream)."""
    rng = np.random.default_rng(3)
    n = 50 * B + 7
    p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    kw = dict(beta1=0.9, beta2=0.999, lr=1e-3, weight_decay=0.01, eps=1e-8, step=3, bits=bits, block_size=B,
              storage=storage, rounding=orc.ROUND_STOCHASTIC, seed=5, tensor_id=9)
    whole_p, whole = p0.copy(), list(orc.init_state(n, B, storage))
    orc.step(whole_p, g, *whole, **kw)
    cuts = [0, 13 * B, 31 * B, n]
    for use_offset in (True, False):
        pp, st = p0.copy(), list(orc.init_state(n, B, storage))
        for s, e in zip(cuts[:-1], cuts[1:]):
            b0, b1 = s // B, (e + B - 1) // B
            orc.step(pp[s:e], g[s:e], st[0][s:e], None if st[1] is None else st[1][s:e],
                     st[2][b0:b1], st[3][b0:b1], st[4][b0:b1], elem_offset=s if use_offset else 0, **kw)
        same = np.array_equal(pp.view(np.uint32), whole_p.view(np.uint32)) and all(
            np.array_equal(a, b) for a, b in zip(st, whole) if a is not None)
        assert same == use_offset, use_offset
