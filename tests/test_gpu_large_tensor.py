"""One tensor of more than 2^31 elements through every kernel, checked on block-aligned slices.

The reference counts elements in a 32-bit ``int`` (stquant_kernel.cu:420), so a tensor of
2^31 elements or more is outside what it can run; this build indexes in 64 bits.  Quant blocks are
independent (per-block scales, elementwise update), so the oracle can judge any block-aligned
slice of the tensor on its own: here the head, the blocks around element 2^31, and the ragged tail.

- step 1 from a fresh state through the single-tensor entry point (``fused_mdq_adamw``), step 2
  through the multi-tensor entry point with a small tensor after the big one: packed 4-bit codes
  and block scales bit-exact, params within the parity bar (bf16 grads, B = 128, nearest);
- the grad statistics of the big tensor against float64 sums taken chunk by chunk on the device;
- the packed -> int8/uint8 code conversion against the nibble decode on the same slices.

About 21 GB of device memory.
"""
import numpy as np
import pytest
import torch

import mdq_hip
from oracle import mdq_oracle as orc
from param_bar import assert_param_bar

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
HP = dict(beta1=0.9, beta2=0.999, lr=1e-3, weight_decay=0.01, eps=1e-8)
B = 128
N = (1 << 31) + 3 * 4096 + 77                      # ragged last block (77 elements)
SLICES = [(0, 1 << 16),
          ((1 << 31) - (1 << 15), (1 << 31) + (1 << 15)),
          ((N - 5000) // B * B, N)]
CHUNK = 1 << 28


def host(t):
    """Host copy of a device slice (bf16 as its uint16 bit pattern, as the oracle takes it)."""
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16).copy()
    return t.cpu().numpy().copy()


def fill_grads(g, gen):
    for o in range(0, N, CHUNK):
        k = min(CHUNK, N - o)
        g[o:o + k].copy_(torch.randn(k, device=DEV, generator=gen).mul_(1e-3))


def snapshot(p, g, codes, sm, sv, vm):
    out = []
    for s, e in SLICES:
        b0, b1 = s // B, (e + B - 1) // B
        out.append([host(p[s:e]), host(g[s:e]), host(codes[s:e]), host(sm[b0:b1]), host(sv[b0:b1]),
                    host(vm[b0:b1])])
    return out


def check_against_oracle(snap, step, p, codes, sm, sv, vm):
    for (s, e), (hp, hg, hc, hsm, hsv, hvm) in zip(SLICES, snap):
        p_prev = hp.copy()
        orc.step(hp, hg, hc, None, hsm, hsv, hvm, step=step, bits=4, block_size=B, storage=orc.STORE_P4, **HP)
        b0, b1 = s // B, (e + B - 1) // B
        where = f"step {step}, elements [{s}, {e})"
        assert np.array_equal(host(codes[s:e]), hc), f"packed codes differ, {where}"
        for name, t, a in (("scale_m", sm, hsm), ("scale_v", sv, hsv), ("v_min", vm, hvm)):
            assert np.array_equal(host(t[b0:b1]).view(np.uint32), a.view(np.uint32)), f"{name} differs, {where}"
        assert_param_bar(host(p[s:e]), hp, p_prev, label=f"2^31+ tensor, {where}")


def test_tensor_beyond_2_31_elements():
    print(f"case: one tensor of {N} elements (bf16 grads, packed 4-bit, B={B})", flush=True)
    nb = (N + B - 1) // B
    gen = torch.Generator(device=DEV).manual_seed(0)
    p = torch.empty(N, dtype=torch.float32, device=DEV)
    for o in range(0, N, CHUNK):
        p[o:o + min(CHUNK, N - o)].normal_(0.0, 0.02, generator=gen)
    g = torch.empty(N, dtype=torch.bfloat16, device=DEV)
    fill_grads(g, gen)
    codes = torch.full((N,), 0x08, dtype=torch.uint8, device=DEV)
    sm = torch.zeros(nb, dtype=torch.float32, device=DEV)
    sv = torch.zeros(nb, dtype=torch.float32, device=DEV)
    vm = torch.full((nb,), -20.0, dtype=torch.float32, device=DEV)
    empty = torch.empty(0, dtype=torch.uint8, device=DEV)

    # step 1: the single-tensor entry point
    snap = snapshot(p, g, codes, sm, sv, vm)
    mdq_hip.fused_step(p, g, codes, empty, sm, sv, vm, HP["beta1"], HP["beta2"], HP["lr"],
                       HP["weight_decay"], HP["eps"], 1, 4, B)
    torch.cuda.synchronize()
    check_against_oracle(snap, 1, p, codes, sm, sv, vm)

    # step 2: the multi-tensor entry point, big tensor first, then a small one
    fill_grads(g, gen)
    rng = np.random.default_rng(1)
    n2 = 1000
    p2 = (rng.standard_normal(n2) * 0.02).astype(np.float32)
    g2 = (rng.standard_normal(n2) * 1e-3).astype(np.float32)
    st2 = list(orc.init_state(n2, B, orc.STORE_P4))
    tp2, tg2 = torch.from_numpy(p2.copy()).to(DEV), torch.from_numpy(g2.astype(np.float32)).to(DEV)
    tg2 = tg2.to(torch.bfloat16)
    g2_bits = host(tg2)
    tc2 = torch.from_numpy(st2[0].copy()).to(DEV)
    ts2 = [torch.from_numpy(a.copy()).to(DEV) for a in st2[2:]]
    snap = snapshot(p, g, codes, sm, sv, vm)
    mdq_hip.multi_tensor_step([
        mdq_hip.TensorState(p, g, codes, empty, sm, sv, vm, 2, 4, HP["lr"], HP["beta1"], HP["beta2"],
                            HP["eps"], HP["weight_decay"], 0),
        mdq_hip.TensorState(tp2, tg2, tc2, empty, *ts2, 1, 4, HP["lr"], HP["beta1"], HP["beta2"],
                            HP["eps"], HP["weight_decay"], 1),
    ], B)
    torch.cuda.synchronize()
    check_against_oracle(snap, 2, p, codes, sm, sv, vm)
    orc.step(p2, g2_bits, st2[0], None, *st2[2:], step=1, bits=4, block_size=B, storage=orc.STORE_P4, **HP)
    assert np.array_equal(host(tc2), st2[0]), "small tensor after the big one: codes differ"
    for t, a in zip(ts2, st2[2:]):
        assert np.array_equal(host(t).view(np.uint32), a.view(np.uint32)), "small tensor: scales differ"
    assert np.max(np.abs(host(tp2).astype(np.float64) - p2)) <= 1e-6 * np.abs(p2).max()

    # grad statistics of the big tensor: float64 sums, chunk by chunk on the device
    s1 = s2 = sa = 0.0
    for o in range(0, N, CHUNK):
        x = g[o:o + CHUNK].double()
        s1 += float(x.sum())
        s2 += float((x * x).sum())
        sa += float(x.abs().sum())
        del x
    mean_sq, mean_abs = s2 / N, sa / N
    sd = np.sqrt((s2 - s1 * (s1 / N)) / (N - 1))
    want = np.array([np.sqrt(mean_sq), sd / (mean_abs + 1e-12), mean_sq])
    got = mdq_hip.grad_stats([g]).cpu().numpy()[0].astype(np.float64)
    assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want)), (got, want)

    # packed -> int8 / uint8 conversion of the big tensor
    del p, sm, sv, vm
    torch.cuda.empty_cache()
    dm, dv = mdq_hip.empty_codes(codes, mdq_hip.STORE_S8)
    mdq_hip.convert_codes([(codes, empty, dm, dv)])
    torch.cuda.synchronize()
    for s, e in SLICES:
        b = host(codes[s:e]).astype(np.int64)
        assert np.array_equal(host(dm[s:e]).astype(np.int64), (b & 15) - 8), f"m codes [{s}, {e})"
        assert np.array_equal(host(dv[s:e]).astype(np.int64), b >> 4), f"v codes [{s}, {e})"
