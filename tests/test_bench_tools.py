"""CPU: the measurement helpers of bench.py that turn rocprofv3 CSV output into the figures the
bench line reports (per-launch HBM bytes from FETCH_SIZE / WRITE_SIZE scaled by a copy kernel
of known size; kernel-stats tables), and the one-GPU guard."""

import csv
import importlib.util
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


FIELDS = ["Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name", "Counter_Value"]


def write_counters(path, counter, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for i, (name, grid, value) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Grid_Size": grid, "Kernel_Name": name, "Counter_Name": counter,
                        "Counter_Value": value})


def test_pmc_summary_scales_by_the_calibration_copy(tmp_path):
    neg = "void at::native::vectorized_elementwise_kernel<4, at::native::neg_kernel_cuda(...)>"
    gemm = "void afd::mx_gemm_kernel<0, 4>(afd::MxGemmArgs)"
    copy_grid = 1024 * (1 << 20) // 16  # 1 GiB of fp32, 4 per lane
    # FETCH_SIZE reads half the bytes of the copy (scale 2), WRITE_SIZE all of them (scale 1);
    # a small neg launch of the input generator shares the copy's name and must be ignored
    write_counters(tmp_path / "f.csv", "FETCH_SIZE", [
        (neg, 4096, 10.0), (gemm, 256, 1000.0), (gemm, 256, 1200.0), (neg, copy_grid, 524288.0)])
    write_counters(tmp_path / "w.csv", "WRITE_SIZE", [
        (neg, 4096, 20.0), (gemm, 256, 50.0), (gemm, 256, 70.0), (neg, copy_grid, 1048576.0)])
    out = bench().pmc_summary(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), 1024, str(tmp_path / "t.json"))
    assert out["scale_fetch"] == 2.0 and out["scale_write"] == 1.0
    k = out["kernels"]["afd::mx_gemm_kernel<0, 4>"]
    assert k["fetch_bytes"] == 1100 * 2 * 1024 and k["write_bytes"] == 60 * 1024
    assert json.load(open(tmp_path / "t.json")) == out
    assert list(out["kernels"]) == ["afd::mx_gemm_kernel<0, 4>"]  # only the library's kernels


def test_pmc_summary_requires_the_copy(tmp_path):
    gemm = "void afd::mx_gemm_kernel<0, 4>(afd::MxGemmArgs)"
    write_counters(tmp_path / "f.csv", "FETCH_SIZE", [(gemm, 256, 1.0)])
    write_counters(tmp_path / "w.csv", "WRITE_SIZE", [(gemm, 256, 1.0)])
    with pytest.raises(SystemExit):
        bench().pmc_summary(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), 1024, None)


def test_stats_summary_table(tmp_path):
    path = tmp_path / "s.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Name", "Calls", "AverageNs", "MinNs", "MaxNs", "Percentage"])
        w.writeheader()
        w.writerow({"Name": "void afd::finalize_kernel(unsigned short const*)", "Calls": 5, "AverageNs": 66700.0,
                    "MinNs": 65000, "MaxNs": 70000, "Percentage": 7.5})
    table = bench().stats_summary(str(path)).splitlines()
    assert table[0].startswith("| kernel | calls | avg us")
    assert table[2] == "| `afd::finalize_kernel` | 5 | 66.70 | 65.00 | 70.00 | 7.50 |"


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "--gpus 2 is not supported" in r.stderr and not r.stdout
