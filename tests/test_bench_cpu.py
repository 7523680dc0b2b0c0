"""bench.py's host-side contract, on the CPU: the one-GPU exit, the metric names of the configs,
the algorithmic byte counts the roofline figure divides by, and the fields of the CPU-baseline
record (a short sample of the oracle)."""
import os
import subprocess
import sys

import pytest

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_every_config_has_shapes_and_a_metric():
    for name, (shapes_fn, gdt, bits, B) in bench.CONFIGS.items():
        shapes = shapes_fn()
        assert shapes and all(n > 0 for _, n in shapes)
        assert gdt in ("f32", "bf16") and bits in (4, 8, 16, 32) and B == 128
    assert set(bench.METRICS) <= set(bench.CONFIGS)
    # the headline metric is the one BASELINE.json names, on the LLaMA-7B set
    assert bench.METRICS["llama7b"].startswith("optimizer params updated/sec + achieved HBM GB/s (% peak), LLaMA-7B")


def test_parameter_counts_and_bytes_per_param():
    assert sum(n for _, n in bench.llama7b_shapes()) == 6_738_415_616
    assert len(bench.llama7b_shapes()) == 291
    assert sum(n for _, n in bench.gpt2_small_shapes()) == 124_439_808
    assert len(bench.gpt2_small_shapes()) == 148
    # p read + write, grad read, codes read + write, 3 fp32 scales read + written per block
    assert bench.bytes_per_param(2, 4, 128) == 12.1875
    assert bench.bytes_per_param(4, 4, 128) == 14.1875
    assert bench.bytes_per_param(4, 8, 64) == 16.375
    assert bench.bytes_per_param(2, 16, 128) == 18.1875
    sizes = bench.config5_sizes()
    assert len(sizes) == 257 and sum(sizes) == 363_174_740 and sum(n % 128 != 0 for n in sizes) == 254


@pytest.mark.timeout(300)
def test_cpu_baseline_record():
    c = bench.cpu_baseline("bf16", 4, 128, 0.5)
    assert c["kind"] == "port" and c["unit"] == "params/s" and c["cores"] >= 1
    assert c["value"] > 0 and c["value_1thread"] > 0
    assert abs(c["gbs"] - c["value"] * 12.1875 / 1e9) < 1e-9 * c["gbs"] + 1e-12
    assert c["cpu_model"] and "oracle/mdq_oracle.c" in c["sample"]
