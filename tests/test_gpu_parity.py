"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bar: packed codes, int codes and the three block-scale arrays bit-exact; params per element
within |dp| <= 2^-20 |update| + 2^-22 |p'| of the oracle's (the error bound of the device
update, which uses the hardware sqrt / reciprocal where the oracle uses IEEE sqrtf and division;
derived in tests/param_bar.py).  Every comparison records its per-element error distribution
(share bit-identical, quantiles of |dp|/|p'|, the share above 1e-6 relative), which the session
prints at its end.
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
STORE_TORCH = {
    orc.STORE_P4: (torch.uint8, None),
    orc.STORE_S8: (torch.int8, torch.uint8),
    orc.STORE_S16: (torch.int16, torch.uint16),
    orc.STORE_S32: (torch.int32, torch.uint32),
}


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def assert_bits_equal(name, t, a):
    got = t.cpu().numpy()
    if got.dtype == np.float32:
        ok = np.array_equal(got.view(np.uint32), a.view(np.uint32))
    else:
        ok = np.array_equal(got, a)
    if not ok:
        bad = np.nonzero(got.view(np.uint8 if got.dtype.itemsize == 1 else got.dtype) != a.view(got.dtype))[0]
        raise AssertionError(f"{name}: {bad.size} mismatches, first at {bad[:5]} got {got[bad[:5]]} want {a[bad[:5]]}")


def assert_params_close(p_gpu, p_ref, p_prev, label=""):
    """One step from identical inputs: |dp| <= 2^-20 |update| + 2^-22 |p'| per element (the
    device update's error bound, tests/param_bar.py), and over the tensor max|dp| <= 1e-6 times
    its params' magnitude, the larger of max|p'| and max|p| before the step (a tensor of one or
    a few elements whose step carries them next to zero has a tiny max|p'|)."""
    got = p_gpu.cpu().numpy() if isinstance(p_gpu, torch.Tensor) else np.asarray(p_gpu)
    assert_param_bar(got, p_ref, p_prev, label=label)
    err = np.abs(got.astype(np.float64) - p_ref.astype(np.float64))
    scale = max(np.abs(p_ref.astype(np.float64)).max(), np.abs(np.asarray(p_prev, dtype=np.float64)).max())
    assert err.max() <= 1e-6 * scale, (err.max(), scale)


def resync_params(tp, p):
    """Start the next step from the oracle's params so each step is judged alone."""
    tp.copy_(torch.from_numpy(p))


class Case:
    """One tensor's numpy state (oracle side) and torch state (device side)."""

    def __init__(self, n, B, storage, rng, grad_dtype=np.float32, offset=0, codes_aligned=False, tail=0):
        self.n, self.B, self.storage = n, B, storage
        self.p = (rng.standard_normal(n) * 0.02).astype(np.float32)
        self.state = list(orc.init_state(n, B, storage))
        self.offset, self.tail = offset, tail
        # device copies; `offset` elements of padding in front make the views unaligned (the code
        # arrays too unless `codes_aligned`, as when only params and grads are views of one buffer)
        self.tp = self._dev_view(self.p)
        cm, cv = self.state[0], self.state[1]
        cview = (lambda a: to_dev(a.copy())) if codes_aligned else self._dev_view
        self.tcm = cview(cm)
        self.tcv = cview(cv) if cv is not None else torch.empty(0, dtype=torch.uint8, device=DEV)
        self.tsm, self.tsv, self.tvm = (to_dev(a.copy()) for a in self.state[2:])
        self.grad_dtype = grad_dtype

    def _dev_view(self, a):
        if self.offset == 0 and self.tail == 0:
            return to_dev(a.copy())
        # padding of 7s around the view (the sentinel that padding_intact checks)
        buf = np.full(a.size + self.offset + self.tail, 7, dtype=a.dtype)
        buf[self.offset:self.offset + a.size] = a
        return to_dev(buf)[self.offset:self.offset + a.size]

    def padding_intact(self):
        base = self.tp._base
        assert base is not None
        torch.cuda.synchronize()
        pad = torch.cat([base[:self.offset], base[self.offset + self.n:]]).cpu()
        assert pad.numel() == self.offset + self.tail
        assert torch.equal(pad, torch.full_like(pad, 7.0)), "a store left the params' view"

    def grads(self, rng):
        g = (rng.standard_normal(self.n) * 1e-3).astype(np.float32)
        if self.grad_dtype == "bf16":
            tg = torch.from_numpy(g).to(torch.bfloat16)
            g_np = tg.view(torch.int16).numpy().view(np.uint16).copy()
            return g_np, self._dev_view_t(tg)
        if self.grad_dtype == np.float16:
            g16 = g.astype(np.float16)
            return g16, self._dev_view(g16)
        return g, self._dev_view(g)

    def _dev_view_t(self, t):
        if self.offset == 0:
            return t.to(DEV)
        buf = torch.zeros(t.numel() + self.offset, dtype=t.dtype)
        buf[self.offset:] = t
        return buf.to(DEV)[self.offset:]

    def oracle_step(self, g, step, bits, **kw):
        hp = dict(HP)
        hp.update(kw)
        cm, cv, sm, sv, vm = self.state
        orc.step(self.p, g, cm, cv, sm, sv, vm, step=step, bits=bits, block_size=self.B,
                 storage=self.storage, **hp)

    def entry(self, tg, step, bits, tensor_id=0, **kw):
        hp = dict(HP)
        hp.update(kw)
        return mdq_hip.TensorState(self.tp, tg, self.tcm, self.tcv, self.tsm, self.tsv, self.tvm, step, bits,
                                   hp["lr"], hp["beta1"], hp["beta2"], hp["eps"], hp["weight_decay"],
                                   tensor_id)

    def check(self, p_prev):
        torch.cuda.synchronize()
        cm, cv, sm, sv, vm = self.state
        assert_bits_equal("exp_avg", self.tcm, cm)
        if cv is not None:
            assert_bits_equal("exp_avg_sq", self.tcv, cv)
        assert_bits_equal("scale_m", self.tsm, sm)
        assert_bits_equal("scale_v", self.tsv, sv)
        assert_bits_equal("v_min", self.tvm, vm)
        assert_params_close(self.tp, self.p, p_prev)
        resync_params(self.tp, self.p)


def test_config1_flat_4m_packed4_ten_steps():
    """4,194,304 fp32 params ~N(0,0.02), fp32 grads ~N(0,1e-3)
    redrawn each step from seed 0; 4-bit, B=128, nearest; 10 steps, compared after each."""
    print("case: config1 n=4194304 B=128 packed4 nearest", flush=True)
    n, B = 4_194_304, 128
    gen = torch.Generator().manual_seed(0)
    p0 = (torch.randn(n, generator=gen) * 0.02).numpy()
    st = list(orc.init_state(n, B, orc.STORE_P4))
    p = p0.copy()
    tp = to_dev(p0.copy())
    tcm = to_dev(st[0].copy())
    tsm, tsv, tvm = (to_dev(a.copy()) for a in st[2:])
    empty = torch.empty(0, dtype=torch.uint8, device=DEV)
    for step in range(1, 11):
        g = (torch.randn(n, generator=gen) * 1e-3).numpy()
        p_prev = p.copy()
        orc.step(p, g, st[0], None, st[2], st[3], st[4], step=step, bits=4, block_size=B,
                 storage=orc.STORE_P4, **HP)
        mdq_hip.fused_step(tp, to_dev(g), tcm, empty, tsm, tsv, tvm, HP["beta1"], HP["beta2"], HP["lr"],
                           HP["weight_decay"], HP["eps"], step, 4, B)
        torch.cuda.synchronize()
        assert_bits_equal(f"step {step} codes", tcm, st[0])
        assert_bits_equal(f"step {step} scale_m", tsm, st[2])
        assert_bits_equal(f"step {step} scale_v", tsv, st[3])
        assert_bits_equal(f"step {step} v_min", tvm, st[4])
        assert_params_close(tp, p, p_prev, label=f"config 1 step {step}")
        resync_params(tp, p)


def test_config1_accumulated_param_drift():
    """Without re-syncing, 10 steps of independent roundoff stay within 1e-6 of max|p|."""
    n, B = 1 << 20, 128
    gen = torch.Generator().manual_seed(0)
    p = (torch.randn(n, generator=gen) * 0.02).numpy()
    st = list(orc.init_state(n, B, orc.STORE_P4))
    tp = to_dev(p.copy())
    tcm = to_dev(st[0].copy())
    tsm, tsv, tvm = (to_dev(a.copy()) for a in st[2:])
    empty = torch.empty(0, dtype=torch.uint8, device=DEV)
    for step in range(1, 11):
        g = (torch.randn(n, generator=gen) * 1e-3).numpy()
        orc.step(p, g, st[0], None, st[2], st[3], st[4], step=step, bits=4, block_size=B,
                 storage=orc.STORE_P4, **HP)
        mdq_hip.fused_step(tp, to_dev(g), tcm, empty, tsm, tsv, tvm, HP["beta1"], HP["beta2"], HP["lr"],
                           HP["weight_decay"], HP["eps"], step, 4, B)
    torch.cuda.synchronize()
    assert_bits_equal("codes", tcm, st[0])
    err = np.abs(tp.cpu().numpy().astype(np.float64) - p)
    assert err.max() <= 1e-6 * np.abs(p).max()


STORAGE_BITS = [(orc.STORE_P4, 4), (orc.STORE_S8, 4), (orc.STORE_S8, 8), (orc.STORE_S16, 16),
                (orc.STORE_S16, 8), (orc.STORE_S32, 32), (orc.STORE_S32, 16)]


@pytest.mark.parametrize("storage,bits", STORAGE_BITS)
@pytest.mark.parametrize("B", [64, 128, 256])
def test_storage_and_block_sizes(storage, bits, B):
    print(f"case: storage={storage} bits={bits} B={B}", flush=True)
    rng = np.random.default_rng(1000 * storage + 10 * bits + B)
    c = Case(B * 37 + 19, B, storage, rng)
    for step in (1, 2, 3):
        g, tg = c.grads(rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits)
        mdq_hip.multi_tensor_step([c.entry(tg, step, bits)], B)
        c.check(p_prev)


@pytest.mark.parametrize("B", [1, 2, 4, 8, 16, 32, 512, 1024])
def test_all_block_sizes(B):
    print(f"case: block size {B}", flush=True)
    rng = np.random.default_rng(B)
    for storage, bits in ((orc.STORE_P4, 4), (orc.STORE_S8, 8)):
        c = Case(B * 23 + max(1, B // 3), B, storage, rng)
        for step in (1, 2):
            g, tg = c.grads(rng)
            p_prev = c.p.copy()
            c.oracle_step(g, step, bits)
            mdq_hip.multi_tensor_step([c.entry(tg, step, bits)], B)
            c.check(p_prev)


@pytest.mark.parametrize("gdt", ["bf16", np.float16])
def test_low_precision_grads(gdt):
    print(f"case: grad dtype {gdt}", flush=True)
    rng = np.random.default_rng(5)
    c = Case(128 * 100 + 3, 128, orc.STORE_P4, rng, grad_dtype=gdt)
    for step in (1, 2, 3):
        g, tg = c.grads(rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, 4)
        mdq_hip.multi_tensor_step([c.entry(tg, step, 4)], 128)
        c.check(p_prev)


def test_unaligned_views_take_the_guarded_path():
    print("case: unaligned views", flush=True)
    rng = np.random.default_rng(6)
    c = Case(128 * 50, 128, orc.STORE_S8, rng, offset=1)
    for step in (1, 2):
        g, tg = c.grads(rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, 8)
        mdq_hip.multi_tensor_step([c.entry(tg, step, 8)], 128)
        c.check(p_prev)


@pytest.mark.parametrize("storage,bits", STORAGE_BITS)
@pytest.mark.parametrize("B,offset,gdt", [(128, 1, np.float32), (64, 3, "bf16"), (256, 2, np.float16),
                                          (1024, 1, "bf16"), (4, 5, np.float32)])
def test_param_and_grad_views_at_odd_offsets(storage, bits, B, offset, gdt):
    """Params and grads as views at odd element offsets of one buffer, codes allocated on their own
    (the optimizer's layout when a model's params are views of a flat buffer): whole tiles take the
    element-wise p / grad accesses with vector code accesses, the tail tile the guarded path."""
    print(f"case: p/g views offset={offset} storage={storage} bits={bits} B={B} grad={gdt}", flush=True)
    rng = np.random.default_rng(40_000 + 10 * offset + B + storage)
    c = Case(B * 29 + 3 * B // 4 + 1, B, storage, rng, grad_dtype=gdt, offset=offset, codes_aligned=True)
    for step in (1, 2):
        g, tg = c.grads(rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits)
        mdq_hip.multi_tensor_step([c.entry(tg, step, bits)], B)
        c.check(p_prev)


@pytest.mark.parametrize("storage,bits", [(orc.STORE_P4, 4), (orc.STORE_S8, 8), (orc.STORE_S16, 16)])
@pytest.mark.parametrize("B,offset,gdt,full", [(8, 4, np.float32, True), (16, 31, "bf16", False),
                                               (64, 8, np.float32, True), (128, 16, np.float16, False),
                                               (256, 28, np.float32, True), (512, 33, "bf16", True),
                                               (1024, 12, "bf16", True), (1024, 1, np.float32, False),
                                               (4, 20, np.float32, True)])
def test_param_views_inside_a_cache_line(storage, bits, B, offset, gdt, full):
    """Params that start inside a 128-byte line (offset mod 32 elements != 0; offsets that are
    multiples of 4 keep 16-byte alignment and the vector mode): whole tiles store p line by line
    through LDS.  Padding before and after the view stays untouched, with the tensor ending on a
    whole tile (`full`: the last tile is staged too) or on a ragged one."""
    print(f"case: p line offset={offset} storage={storage} bits={bits} B={B} grad={gdt} full={full}",
          flush=True)
    tile = 256 if B == 4 else (1024 if B == 1024 else 512)
    n = 5 * tile if full else 5 * tile + B // 2 + 3
    rng = np.random.default_rng(41_000 + 10 * offset + B + storage)
    c = Case(n, B, storage, rng, grad_dtype=gdt, offset=offset, codes_aligned=True, tail=45)
    for step in (1, 2):
        g, tg = c.grads(rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits)
        mdq_hip.multi_tensor_step([c.entry(tg, step, bits)], B)
        c.padding_intact()
        c.check(p_prev)


@pytest.mark.parametrize("storage,bits", [(orc.STORE_P4, 4), (orc.STORE_S8, 8), (orc.STORE_S16, 16),
                                          (orc.STORE_S32, 16)], ids=["p4", "s8", "s16", "s32"])
@pytest.mark.parametrize("B,offset,gdt", [(32, 5, np.float32), (64, 31, "bf16"), (64, 4, np.float16),
                                          (128, 3, np.float32), (128, 30, "bf16"), (256, 17, "bf16"),
                                          (512, 12, np.float32), (1024, 9, np.float32)])
def test_stochastic_rounding_on_param_views(storage, bits, B, offset, gdt):
    """Stochastic rounding on params and grads that start inside a 128-byte line (staged lines,
    except for 32-bit storage from B = 256 on: the lanes' element-aligned vectors there): codes
    bit-exact, padding untouched."""
    print(f"case: stochastic p/g views offset={offset} storage={storage} bits={bits} B={B} grad={gdt}",
          flush=True)
    rng = np.random.default_rng(42_000 + 10 * offset + B + storage)
    c = Case(512 * 6 + B + 5, B, storage, rng, grad_dtype=gdt, offset=offset, codes_aligned=True, tail=37)
    for step in (1, 2):
        g, tg = c.grads(rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits, rounding=orc.ROUND_STOCHASTIC, seed=99, tensor_id=3)
        mdq_hip.multi_tensor_step([c.entry(tg, step, bits, tensor_id=3)], B, rounding="stochastic", seed=99)
        c.padding_intact()
        c.check(p_prev)


@pytest.mark.parametrize("storage,bits", [(orc.STORE_P4, 4), (orc.STORE_S8, 8), (orc.STORE_S16, 16)])
def test_stochastic_rounding_bit_exact(storage, bits):
    print(f"case: stochastic storage={storage} bits={bits}", flush=True)
    rng = np.random.default_rng(7)
    c = Case(128 * 64 + 77, 128, storage, rng)
    for step in (1, 2, 3):
        g, tg = c.grads(rng)
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits, rounding=orc.ROUND_STOCHASTIC, seed=1234, tensor_id=9)
        mdq_hip.multi_tensor_step([c.entry(tg, step, bits, tensor_id=9)], 128,
                                  rounding="stochastic", seed=1234)
        c.check(p_prev)


@pytest.mark.parametrize("storage,bits", [(orc.STORE_P4, 4), (orc.STORE_S8, 8)], ids=["p4", "s8"])
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
def test_flat_blocks_beside_ordinary_ones(storage, bits, rounding):
    """Blocks whose v + 1e-12 is the same float in every element (zero grads every step, or one
    grad value for the whole block) next to ordinary blocks in the same waves, 8 steps from a fresh
    state.  Their v codes are 0 (log x - vmin = 0 exactly), which the fast path sets without the
    per-element logs; codes, scales and params against the oracle after every step."""
    print(f"case: flat blocks storage={storage} bits={bits} {rounding}", flush=True)
    rng = np.random.default_rng(31 + bits)
    B = 128
    n = B * 4 * 256
    nb = n // B
    c = Case(n, B, storage, rng)
    kind = rng.integers(0, 4, nb)            # 0: zero grads, 1: one value per block, 2-3: ordinary
    assert (kind == 0).any() and (kind == 1).any()
    rmode = orc.ROUND_STOCHASTIC if rounding == "stochastic" else orc.ROUND_NEAREST
    for step in range(1, 9):
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        gb = g.reshape(nb, B)
        gb[kind == 0] = 0.0
        gb[kind == 1] = np.float32(1e-3 * (1 + step % 3))
        p_prev = c.p.copy()
        c.oracle_step(g, step, bits, rounding=rmode, seed=77, tensor_id=5)
        mdq_hip.multi_tensor_step([c.entry(to_dev(g), step, bits, tensor_id=5)], B, rounding=rounding, seed=77)
        c.check(p_prev)
    # the flat blocks did end at code 0 with v_min at their common log
    cm, cv = c.state[0], c.state[1]
    vcodes = (cm >> 4) if cv is None else cv
    assert np.all(vcodes.reshape(nb, B)[kind == 0] == 0)


def test_multi_tensor_ragged_heavy_tail():
    """Config-5-style: many tensors with log-uniform sizes (mostly not multiples of B),
    Student-t grads with all-zero blocks and x1000 outliers, per-tensor steps and
    hyper-parameters, one launch."""
    print("case: ragged multi-tensor", flush=True)
    rng = np.random.default_rng(0)
    sizes = np.clip(np.floor(np.exp(rng.uniform(0, np.log(2 ** 17), 41))), 1, 2 ** 17).astype(int)
    B = 128
    cases = [Case(int(s), B, orc.STORE_P4, rng) for s in sizes]
    for step in (1, 2):
        entries, prevs = [], []
        for i, c in enumerate(cases):
            g = (rng.standard_t(3, c.n) * 1e-3).astype(np.float32)
            nb = (c.n + B - 1) // B
            zero_blocks = rng.random(nb) < 0.05
            g[np.repeat(zero_blocks, B)[: c.n]] = 0.0
            out = rng.random(c.n) < 0.001
            g[out] *= 1000.0
            lr = 1e-3 * (1 + i % 3)
            prevs.append(c.p.copy())
            c.oracle_step(g, step + i % 2, 4, lr=lr)
            entries.append(c.entry(to_dev(g), step + i % 2, 4, tensor_id=i, lr=lr))
        mdq_hip.multi_tensor_step(entries, B)
        for c, pp in zip(cases, prevs):
            c.check(pp)


@pytest.mark.parametrize("storage,bits,rounding", [(orc.STORE_P4, 4, "nearest"), (orc.STORE_S8, 8, "stochastic")],
                         ids=["p4-nearest", "s8-stochastic"])
def test_thousands_of_small_tensors_one_launch(storage, bits, rounding):
    """2000 tensors of 1 to 4096 elements (log-uniform: most have a ragged last block, many are
    a single tile or less) in one launch: a descriptor table of 2000 entries, found per tile by
    the kernel's binary search, with per-tensor steps and learning rates; two steps."""
    print(f"case: 2000 small tensors storage={storage} bits={bits} {rounding}", flush=True)
    rng = np.random.default_rng(2000 + bits)
    sizes = np.clip(np.floor(np.exp(rng.uniform(0, np.log(4096), 2000))), 1, 4096).astype(int)
    B = 128
    rmode = orc.ROUND_STOCHASTIC if rounding == "stochastic" else orc.ROUND_NEAREST
    cases = [Case(int(s), B, storage, rng) for s in sizes]
    for step in (1, 2):
        entries, prevs = [], []
        for i, c in enumerate(cases):
            g, tg = c.grads(rng)
            lr = 1e-3 * (1 + i % 3)
            prevs.append(c.p.copy())
            c.oracle_step(g, step + i % 2, bits, lr=lr, rounding=rmode, seed=21, tensor_id=i)
            entries.append(c.entry(tg, step + i % 2, bits, tensor_id=i, lr=lr))
        mdq_hip.multi_tensor_step(entries, B, rounding=rounding, seed=21)
        for c, pp in zip(cases, prevs):
            c.check(pp)


def test_determinism_across_calls():
    rng = np.random.default_rng(8)
    n, B = 128 * 300 + 5, 128
    p = torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)).to(DEV)
    g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(DEV)
    outs = []
    for _ in range(2):
        cm, _cv, sm, sv, vm = orc.init_state(n, B, orc.STORE_P4)
        t = [p.clone(), to_dev(cm), to_dev(sm), to_dev(sv), to_dev(vm)]
        mdq_hip.fused_step(t[0], g, t[1], torch.empty(0, dtype=torch.uint8, device=DEV), t[2], t[3], t[4],
                           0.9, 0.999, 1e-3, 0.01, 1e-8, 1, 4, B)
        outs.append([x.cpu() for x in t])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("tensors", [1, 2], ids=["one-tensor kernel", "descriptor-table kernel"])
def test_profile_cycles_accumulate(tensors):
    """All five phase sums grow, in the one-tensor launch (descriptor as a kernel argument) and in
    a launch over a descriptor table; the steps stay exact."""
    rng = np.random.default_rng(9)
    n, B = 128 * 1000, 128
    cases = [Case(n + 384 * k, B, orc.STORE_P4, rng) for k in range(tensors)]
    grads = [c.grads(rng) for c in cases]
    prof = torch.zeros(5, dtype=torch.int64, device=DEV)
    mdq_hip.multi_tensor_step([c.entry(tg, 1, 4, tensor_id=k) for k, (c, (_g, tg)) in enumerate(zip(cases, grads))],
                              B, profile_cycles=prof)
    for k, (c, (g, _tg)) in enumerate(zip(cases, grads)):
        p_prev = c.p.copy()
        c.oracle_step(g, 1, 4, tensor_id=k)
        c.check(p_prev)
    cyc = prof.cpu().numpy()
    assert np.all(cyc > 0), cyc


def test_errors_follow_the_reference_messages():
    p = torch.zeros(256, device=DEV)
    g = torch.zeros(256, device=DEV)
    sm = torch.zeros(2, device=DEV)
    bad_ea = torch.zeros(256, dtype=torch.int16, device=DEV)
    bad_easq = torch.zeros(256, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError, match="MDQ: state must be packed4"):
        mdq_hip.fused_step(p, g, bad_ea, bad_easq, sm, sm.clone(), sm.clone(), 0.9, 0.999, 1e-3, 0.0, 1e-8, 1, 4, 128)
    with pytest.raises(RuntimeError, match="packed4: exp_avg numel must match parameters"):
        mdq_hip.fused_step(p, g, torch.zeros(255, dtype=torch.uint8, device=DEV),
                           torch.empty(0, dtype=torch.uint8, device=DEV), sm, sm.clone(), sm.clone(),
                           0.9, 0.999, 1e-3, 0.0, 1e-8, 1, 4, 128)
    with pytest.raises(RuntimeError, match="p/grad must be CUDA"):
        mdq_hip.fused_step(p.cpu(), g, bad_ea, bad_easq, sm, sm, sm, 0.9, 0.999, 1e-3, 0.0, 1e-8, 1, 4, 128)
    with pytest.raises(RuntimeError, match="profile_cycles needs >= 5 elements"):
        mdq_hip.fused_step(p, g, torch.full((256,), 8, dtype=torch.uint8, device=DEV),
                           torch.empty(0, dtype=torch.uint8, device=DEV), sm, sm.clone(), sm.clone(),
                           0.9, 0.999, 1e-3, 0.0, 1e-8, 1, 4, 128, torch.zeros(3, dtype=torch.int64, device=DEV))


@pytest.mark.parametrize("storage,bits,B", [(orc.STORE_P4, 4, 64), (orc.STORE_P4, 4, 128), (orc.STORE_S8, 8, 128),
                                            (orc.STORE_S8, 6, 256), (orc.STORE_S16, 12, 128)])
def test_exact_and_near_ties_in_full_tiles(storage, bits, B):
    """m on (k + 1/2) d exactly, one float ulp below and above it, for every k and both signs,
    in whole one-wave tiles (the kernel's fast path): ties round away from zero, near-ties to
    the nearest code, bit-exact against the oracle.  Fresh state and beta1 = 1/2 make m = g / 2
    exact at step 1; each block's largest |m| = M sets d = (M + 1e-12) / 2^(bits-1) + 1e-12."""
    print(f"case: ties storage={storage} bits={bits} B={B}", flush=True)
    rng = np.random.default_rng(bits * 1000 + B)
    n = 4 * 512
    qm = 2 ** (bits - 1)
    g = np.zeros(n, np.float32)
    for blk in range(n // B):
        M = np.float32(10.0 ** rng.uniform(-6, -2))
        d = (M + np.float32(1e-12)) / np.float32(qm) + np.float32(1e-12)
        ks = rng.integers(0, qm, B)
        t = ((ks + 0.5) * np.float64(d)).astype(np.float32)
        kind = rng.integers(0, 3, B)
        t = np.where(kind == 1, np.nextafter(t, np.float32(0)), np.where(kind == 2, np.nextafter(t, np.float32(1)), t))
        t = np.minimum(t, M) * np.where(rng.random(B) < 0.5, np.float32(-1), np.float32(1))
        t[int(rng.integers(0, B))] = M * np.float32(1 if rng.random() < 0.5 else -1)
        g[blk * B:(blk + 1) * B] = t * np.float32(2.0)
    c = Case(n, B, storage, rng)
    p_prev = c.p.copy()
    c.oracle_step(g, 1, bits, beta1=0.5)
    mdq_hip.multi_tensor_step([c.entry(to_dev(g), 1, bits, beta1=0.5)], B)
    c.check(p_prev)
