"""bench.py's host-side contract, on the CPU: the one-GPU exit, the metric names of the configs,
the algorithmic byte counts the roofline figure divides by, the fields of the CPU-baseline
record (a short sample of the oracle), and the rocprofv3 summaries behind the committed
profiles (warm-up dispatches dropped, counters scaled by the calibration copies)."""
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


def _write_csv(path, header, rows):
    import csv
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_profile_summary_drops_warmup_and_calibrates_on_the_last_copies(tmp_path):
    """``--profile-summary`` on synthetic rocprofv3 CSVs: the kernel time averages only the
    dispatches after the warm-up ones (dispatch order, not file order), and FETCH_SIZE /
    WRITE_SIZE are scaled by what the last three copies of known size read, not by an earlier
    set-up copy of another size."""
    k = "void mdq::mdq_step_kernel<0, 0, 1, 7, false>(...)"
    cp = "__amd_rocclr_copyBuffer"
    # 2 warm-up dispatches of 20 ms, then 4 of 10 ms, listed out of order
    trace = [(k, 6, 0, 10_000_000), (k, 1, 0, 20_000_000), (k, 4, 0, 10_000_000), (k, 2, 0, 20_000_000),
             (k, 3, 0, 10_000_000), (k, 5, 0, 10_000_000), (cp, 7, 0, 1)]
    _write_csv(str(tmp_path / "tr" / "x" / "t_kernel_trace.csv"),
               ["Kernel_Name", "Dispatch_Id", "Start_Timestamp", "End_Timestamp"], trace)
    gib = 4
    copy_kib = gib * (1 << 30) / 1024
    fetch = [(k, 1, "FETCH_SIZE", 1000.0), (k, 2, "FETCH_SIZE", 3000.0),
             (cp, 3, "FETCH_SIZE", 123.0),                                    # set-up copy, another size
             (cp, 4, "FETCH_SIZE", copy_kib / 2), (cp, 5, "FETCH_SIZE", copy_kib / 2),
             (cp, 6, "FETCH_SIZE", copy_kib / 2)]
    write = [(k, 1, "WRITE_SIZE", 500.0), (k, 2, "WRITE_SIZE", 1500.0),
             (cp, 3, "WRITE_SIZE", 7.0),
             (cp, 4, "WRITE_SIZE", copy_kib), (cp, 5, "WRITE_SIZE", copy_kib), (cp, 6, "WRITE_SIZE", copy_kib)]
    hdr = ["Kernel_Name", "Dispatch_Id", "Counter_Name", "Counter_Value"]
    _write_csv(str(tmp_path / "f" / "f_counter_collection.csv"), hdr, fetch)
    _write_csv(str(tmp_path / "w" / "w_counter_collection.csv"), hdr, write)
    out = str(tmp_path / "summary")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--profile-summary", out,
                        "--config", "gpt2", "--trace", str(tmp_path / "tr"), "--fetch", str(tmp_path / "f"),
                        "--write", str(tmp_path / "w"), "--skip", "2", "--copy-gib", str(gib),
                        "--kernel", "mdq_step_kernel"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    import json
    with open(out + ".json") as f:
        d = json.load(f)
    assert d["dispatches"] == 6 and d["calls"] == 4 and d["avg_ns"] == 10_000_000
    assert d["avg_ns_with_warmup"] == (2 * 20_000_000 + 4 * 10_000_000) / 6
    assert d["fetch_scale"] == 2.0 and d["write_scale"] == 1.0
    # kernel: mean FETCH 2000 KiB x 2 + mean WRITE 1000 KiB x 1
    assert d["traffic_bytes"] == (2000.0 * 2 + 1000.0) * 1024
    alg = bench.bytes_per_param(4, 4, 128) * 124_439_808
    assert d["algorithmic_bytes"] == alg and abs(d["frac_of_peak"] - alg / 1e7 / 8000.0) < 1e-12
    with open(out + ".md") as f:
        md = f.read()
    assert "average over the 4 timed launches **10.000 ms**" in md


def test_dispatch_table_joins_trace_and_counters_by_dispatch(tmp_path):
    """``--dispatch-table`` on one synthetic rocprofv3 run (kernel trace + counters in one
    directory): rows follow dispatch order, other kernels are left out, the per-XCD busy
    cycles divided by the duration give the clock, and counters split over dimension rows add
    up before dividing."""
    k = "void mdq::mdq_step_kernel<0, 0, 0, 7, false>(...)"
    other = "elementwise_kernel"
    trace = [(k, 3, 0, 1_000_000), (k, 1, 0, 800_000), (other, 2, 0, 5), (k, 4, 0, 500_000)]
    _write_csv(str(tmp_path / "run" / "a" / "c_kernel_trace.csv"),
               ["Kernel_Name", "Dispatch_Id", "Start_Timestamp", "End_Timestamp"], trace)
    cnt = []
    for disp, ms, ghz, valu in ((1, 0.8, 2.0, 500.0), (3, 1.0, 1.2, 510.0), (4, 0.5, 2.2, 490.0)):
        busy = ghz * 1e9 * ms * 1e-3 * 8
        cnt += [(k, disp, "GRBM_GUI_ACTIVE", busy / 2), (k, disp, "GRBM_GUI_ACTIVE", busy / 2),
                (k, disp, "SQ_WAVES", 100.0), (k, disp, "SQ_INSTS_VALU", valu * 100.0)]
    cnt.append((other, 2, "SQ_WAVES", 7.0))
    _write_csv(str(tmp_path / "run" / "a" / "c_counter_collection.csv"),
               ["Kernel_Name", "Dispatch_Id", "Counter_Name", "Counter_Value"], cnt)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--dispatch-table", str(tmp_path / "run"),
                        "--kernel", "mdq_step_kernel"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    rows = [ln for ln in r.stdout.splitlines() if ln.startswith("| ") and ln[2].isdigit()]
    assert rows == ["| 1 | 0.800 | 500.0 | 2.00 |", "| 2 | 1.000 | 510.0 | 1.20 |", "| 3 | 0.500 | 490.0 | 2.20 |"]


def test_throughput_record_divides_the_algorithmic_bytes_by_the_event_time():
    """Each config's record under ``configs``: params/s on the wall clock, GB/s and the fraction of
    the 8 TB/s peak from the algorithmic bytes over the HIP-event time."""
    t = dict(ms_per_step=13.0, kernel_ms=12.5, steps=20, warmup=3, step=23)
    r = bench.throughput_record(t, 6_738_415_616, 291, 4, 128, "bf16", "stochastic", workload="w")
    assert abs(r["params_per_s"] - 6_738_415_616 / 13.0e-3) < 1e-9 * r["params_per_s"]
    alg = 12.1875 * 6_738_415_616
    assert abs(r["hbm_gbs"] - alg / 12.5e-3 / 1e9) < 1e-9 * r["hbm_gbs"]
    assert abs(r["frac"] - r["hbm_gbs"] / 8000.0) < 1e-15
    assert r["rounding"] == "stochastic" and r["workload"] == "w" and r["steps"] == 20
