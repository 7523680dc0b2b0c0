"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

cfg1_small.npz   BASELINE config 1 in miniature: 4096 fp32 params ~N(0, 0.02) and ten
                 fp32 grad draws ~N(0, 1e-3) from torch.Generator().manual_seed(0) (params
                 first, then one grad vector per step), packed 4-bit, B = 128, nearest,
                 AdamW lr 1e-3, betas (0.9, 0.999), eps 1e-8, wd 0.01; the codes and scales
                 after every step and the params after steps 1 and 10.
cfg1_digests.json  the same recipe at the full config-1 size (4,194,304 params): SHA-256 of
                 the packed codes, of the three scale arrays and of the params after every step.

The fixtures freeze the oracle's outputs (so later edits cannot drift silently)
and give the GPU tests a recorded target.  The reference itself cannot run here
(CUDA-only), so these are not reference outputs.
"""
import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import mdq_oracle as orc  # noqa: E402

HP = dict(beta1=0.9, beta2=0.999, lr=1e-3, weight_decay=0.01, eps=1e-8)
B, STEPS = 128, 10


def cfg1_inputs(n):
    gen = torch.Generator().manual_seed(0)
    p = (torch.randn(n, generator=gen) * 0.02).numpy().copy()
    grads = [(torch.randn(n, generator=gen) * 1e-3).numpy().copy() for _ in range(STEPS)]
    return p, grads


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def run(n, record):
    p, grads = cfg1_inputs(n)
    cm, _cv, sm, sv, vm = orc.init_state(n, B, orc.STORE_P4)
    out = []
    for t, g in enumerate(grads, start=1):
        orc.step(p, g, cm, None, sm, sv, vm, step=t, bits=4, block_size=B, storage=orc.STORE_P4, **HP)
        out.append(record(p, cm, sm, sv, vm))
    return out


def main():
    n = 4096
    p0, grads = cfg1_inputs(n)
    steps = run(n, lambda p, cm, sm, sv, vm: (p.copy(), cm.copy(), sm.copy(), sv.copy(), vm.copy()))
    np.savez_compressed(
        os.path.join(HERE, "cfg1_small.npz"), p0=p0, grads=np.stack(grads),
        p_step1=steps[0][0], p_step10=steps[-1][0], codes=np.stack([s[1] for s in steps]),
        scale_m=np.stack([s[2] for s in steps]), scale_v=np.stack([s[3] for s in steps]),
        v_min=np.stack([s[4] for s in steps]))
    n = 4_194_304
    dig = run(n, lambda p, cm, sm, sv, vm: {"codes": sha(cm), "scales": sha(sm, sv, vm), "params": sha(p)})
    with open(os.path.join(HERE, "cfg1_digests.json"), "w") as f:
        json.dump({"n": n, "block_size": B, "bits": 4, "hyper": HP, "steps": dig}, f, indent=1)


if __name__ == "__main__":
    main()
