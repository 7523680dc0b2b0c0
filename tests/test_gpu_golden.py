"""The HIP kernels reproduce the recorded oracle digests of BASELINE config 1
(4,194,304 params, 10 steps): packed codes and scales bit-exact after every step."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import mdq_hip
from test_golden import HP, cfg1_inputs, sha

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_gpu_matches_cfg1_digests():
    print("case: config1 golden digests", flush=True)
    d = json.load(open(os.path.join(HERE, "cfg1_digests.json")))
    n, B = d["n"], d["block_size"]
    p0, grads = cfg1_inputs(n)
    dev = torch.device("cuda:0")
    nb = n // B
    p = torch.from_numpy(p0).to(dev)
    codes = torch.full((n,), 0x08, dtype=torch.uint8, device=dev)
    sm = torch.zeros(nb, device=dev)
    sv = torch.zeros(nb, device=dev)
    vm = torch.full((nb,), -20.0, device=dev)
    empty = torch.empty(0, dtype=torch.uint8, device=dev)
    for t, (g, want) in enumerate(zip(grads, d["steps"]), start=1):
        mdq_hip.fused_step(p, torch.from_numpy(g).to(dev), codes, empty, sm, sv, vm, HP["beta1"], HP["beta2"],
                           HP["lr"], HP["weight_decay"], HP["eps"], t, 4, B)
        assert sha(codes.cpu().numpy()) == want["codes"], f"codes differ at step {t}"
        assert sha(sm.cpu().numpy(), sv.cpu().numpy(), vm.cpu().numpy()) == want["scales"], f"scales differ at step {t}"
