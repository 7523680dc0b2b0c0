"""HIP graph capture is refused: every entry point that uploads a descriptor table returns
STQ_ERR_INVALID while its stream is capturing, before it queues anything, so no replay can
launch with another call's descriptors.  The captures are ended and never replayed; calls
after them work as before."""
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


def _calls(t):
    p, g, m, v, sm, sv, vm = t
    entry = mdq_hip.TensorState(p, g, m, v, sm, sv, vm, 1, 16, 1e-3, 0.9, 0.999, 1e-8, 0.01)
    nm, nv = mdq_hip.empty_codes(m, mdq_hip.STORE_S8)
    return {
        "fused_step": lambda: mdq_hip.fused_step(p, g, m, v, sm, sv, vm, 0.9, 0.999, 1e-3, 0.01, 1e-8, 1, 16, 128),
        "multi_tensor_step": lambda: mdq_hip.multi_tensor_step([entry], 128),
        "multi_tensor_restore": lambda: mdq_hip.multi_tensor_restore(
            [mdq_hip.TensorState(p, g, m, v, sm, sv, vm, 1, 8, 1e-3, 0.9, 0.999, 1e-8, 0.01)], [(nm, nv)], 128),
        "grad_stats": lambda: mdq_hip.grad_stats([g]),
        "convert_codes": lambda: mdq_hip.convert_codes([(m, v, nm, nv)]),
    }


@pytest.mark.parametrize("name", ["fused_step", "multi_tensor_step", "multi_tensor_restore", "grad_stats",
                                  "convert_codes"])
def test_capture_is_refused(name):
    print(f"case: capture refusal {name}", flush=True)
    t = _state()
    before = [x.clone() for x in t]
    call = _calls(t)[name]
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
    for a, b in zip(t, before):                  # nothing ran
        assert torch.equal(a, b)
    del graph
    # outside capture the same call works
    call()
    torch.cuda.synchronize()
