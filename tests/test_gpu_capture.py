"""HIP graph capture.

A step over one tensor that keeps its storage (the reference's ``fused_mdq_adamw``, or a list of
one) is captured as one kernel node whose descriptor is a kernel argument: each replay steps the
captured tensors again with the captured constants, as a captured launch of the reference's kernel
does.  Replays, with eager work and synchronisations between them, are checked bit for bit after
every replay against the same step made eagerly on a twin state in a launch over two tensors, which
takes the descriptor-table kernel: the one-tensor kernel against the table-driven one.

Every other entry point uploads a descriptor table from staging buffers that later calls reuse, so
it refuses a capturing stream: STQ_ERR_INVALID before anything is queued.  Those captures are ended
and never replayed; calls after them work as before."""
import numpy as np
import pytest
import torch

import mdq_hip

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _state(n=4096, B=128):
    p = torch.randn(n, device=DEV) * 0.02
    g = torch.randn(n, device=DEV) * 1e-3
    m = torch.zeros(n, dtype=torch.int16, device=DEV)
    v = torch.zeros(n, dtype=torch.uint16, device=DEV)
    nb = n // B
    return [p, g, m, v, torch.zeros(nb, device=DEV), torch.zeros(nb, device=DEV), torch.full((nb,), -20.0, device=DEV)]


def _calls(t, t2):
    p, g, m, v, sm, sv, vm = t
    entries = [mdq_hip.TensorState(*x, 1, 16, 1e-3, 0.9, 0.999, 1e-8, 0.01) for x in (t, t2)]
    nm, nv = mdq_hip.empty_codes(m, mdq_hip.STORE_S8)
    return {
        "multi_tensor_step": lambda: mdq_hip.multi_tensor_step(entries, 128),
        "multi_tensor_step_noalloc": lambda: mdq_hip.MultiTensorPlan(entries[:1], 128).run(noalloc=True),
        "multi_tensor_restore": lambda: mdq_hip.multi_tensor_restore(
            [mdq_hip.TensorState(p, g, m, v, sm, sv, vm, 1, 8, 1e-3, 0.9, 0.999, 1e-8, 0.01)], [(nm, nv)], 128),
        "grad_stats": lambda: mdq_hip.grad_stats([g]),
        "convert_codes": lambda: mdq_hip.convert_codes([(m, v, nm, nv)]),
    }


@pytest.mark.parametrize("name", ["multi_tensor_step", "multi_tensor_step_noalloc", "multi_tensor_restore",
                                  "grad_stats", "convert_codes"])
def test_capture_is_refused(name):
    print(f"case: capture refusal {name}", flush=True)
    t, t2 = _state(), _state()
    before = [x.clone() for x in t + t2]
    call = _calls(t, t2)[name]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.stream(side):
        graph.capture_begin()
        try:
            call()
        except RuntimeError as e:
            err = str(e)
        finally:
            graph.capture_end()
    torch.cuda.synchronize()
    assert err is not None and "capturing a HIP graph" in err, err
    for a, b in zip(t + t2, before):             # nothing ran
        assert torch.equal(a, b)
    del graph
    # outside capture the same call works
    call()
    torch.cuda.synchronize()


CODE_DTYPES = {4: (torch.uint8, None), 8: (torch.int8, torch.uint8), 16: (torch.int16, torch.uint16)}


def _one_tensor(n, B, bits, offset, seed):
    """Two identical copies of one tensor's state; p and the grads views at `offset` elements
    into their buffers (offset 5: inside a 128-byte line, the staged tiles)."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    nb = (n + B - 1) // B
    mdt, vdt = CODE_DTYPES[bits]
    pb = torch.randn(n + offset, device=DEV, generator=gen) * 0.02
    if bits == 4:
        m = torch.randint(0, 256, (n,), device=DEV, generator=gen).to(torch.uint8)
        v = torch.empty(0, dtype=torch.uint8, device=DEV)
    else:
        lo = torch.iinfo(mdt).min // 2
        m = torch.randint(lo, -lo, (n,), device=DEV, generator=gen).to(mdt)
        v = torch.randint(0, 2 * -lo, (n,), device=DEV, generator=gen).to(vdt)
    sm = torch.rand(nb, device=DEV, generator=gen) * 1e-4
    sv = torch.rand(nb, device=DEV, generator=gen)
    vm = -20.0 + torch.rand(nb, device=DEV, generator=gen)
    twins = []
    for _ in range(2):
        pbuf, gbuf = pb.clone(), torch.zeros(n + offset, device=DEV)
        twins.append(dict(p=pbuf[offset:], g=gbuf[offset:], m=m.clone(), v=v.clone(), sm=sm.clone(),
                          sv=sv.clone(), vm=vm.clone(), keep=(pbuf, gbuf)))
    return twins


def _step(s, B, bits, step, rounding):
    mdq_hip.fused_step(s["p"], s["g"], s["m"], s["v"], s["sm"], s["sv"], s["vm"], 0.9, 0.999, 1e-3, 0.01, 1e-8,
                       step, bits, B, rounding=rounding, seed=11, tensor_id=4)


def _entry(s, bits, step, tensor_id):
    return mdq_hip.TensorState(s["p"], s["g"], s["m"], s["v"], s["sm"], s["sv"], s["vm"], step, bits,
                               1e-3, 0.9, 0.999, 1e-8, 0.01, tensor_id)


def _step_in_a_table(s, other, B, bits, step, rounding):
    """The same step as _step, in a launch over two tensors (the descriptor-table kernel)."""
    mdq_hip.multi_tensor_step([_entry(s, bits, step, 4), _entry(other, bits, step, 5)], B,
                              rounding=rounding, seed=11)


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("rounding", ["nearest", "stochastic"])
@pytest.mark.parametrize("B,n,offset", [(128, 512 * 40 + 77, 0), (64, 512 * 40, 5), (256, 512 * 12 + 3, 5)])
def test_one_tensor_step_is_captured_and_replays(bits, rounding, B, n, offset):
    print(f"case: captured one-tensor step bits={bits} {rounding} B={B} n={n} offset={offset}", flush=True)
    cap, ref = _one_tensor(n, B, bits, offset, seed=bits + B + offset)
    other = _one_tensor(300, B, bits, 0, seed=99)[0]
    step = 7
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    uploads = mdq_hip.step_table_uploads()
    with torch.cuda.stream(side):
        graph.capture_begin()
        _step(cap, B, bits, step, rounding)        # recorded, not run
        graph.capture_end()
    torch.cuda.synchronize()
    assert mdq_hip.step_table_uploads() == uploads, "the captured call uploaded a descriptor table"
    rng = np.random.default_rng(n + bits)
    for r in range(4):
        grads = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(DEV)
        cap["g"].copy_(grads)
        ref["g"].copy_(grads)
        torch.cuda.synchronize()
        graph.replay()
        _step_in_a_table(ref, other, B, bits, step, rounding)   # eager, the descriptor-table kernel
        torch.cuda.synchronize()
        for k in ("p", "m", "v", "sm", "sv", "vm"):
            assert torch.equal(cap[k].view(torch.uint8), ref[k].view(torch.uint8)), (r, k)
        for buf_c, buf_r in zip(cap["keep"], ref["keep"]):   # the padding in front of the views
            assert torch.equal(buf_c[:offset], buf_r[:offset])
        print(f"replay {r}: bit-identical to the eager table-driven step", flush=True)
    del graph
