"""bench.py's host-side logic on the CPU: the algorithmic byte and op counts its roofline objects
divide by, the counter aggregation behind `traffic`, and the one-GPU refusal."""
import csv
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_gemv_bytes_closed_form():
    # config 1's adaLN shape K = 3072 -> N = 18432 with uint4 codes, fp16 scales and packed
    # uint4 zero-points per 64: 28311552 + 1769472 + 442368 weight-side bytes, the int8 row and
    # its scale, bias and bf16 output
    n, k = bench.GEMV_N, 3072
    assert n == 18432
    expect = n * k // 2 + n * (k // 64) * 2 + n * (k // 64) // 2 + k + 4 + 2 * n + 2 * n
    assert bench.gemv_bytes(k) == expect == 30600196
    # an odd number of groups still stores a whole zero-point byte for the last one
    assert bench.gemv_bytes(192) - bench.gemv_bytes(128) == n * (192 - 128) // 2 + n * 2 + n * 1 + 64


def _write_counters(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(r)


def test_counter_means_use_the_largest_grid_and_the_largest_copy(tmp_path):
    p = tmp_path / "c.csv"
    rq, gemm, gemv, copy = bench.RQ_KERNEL, bench.GEMM_KERNEL, bench.GEMV_KERNEL, bench.COPY_KERNEL
    _write_counters(p, [
        {"Kernel_Name": f"void mq::{rq}<256, 0, 3, 0, 1>", "Grid_Size": 262144, "Counter_Name": "FETCH_SIZE", "Counter_Value": 9},
        {"Kernel_Name": f"void mq::{rq}<256, 0, 3, 0, 1>", "Grid_Size": 2096640, "Counter_Name": "FETCH_SIZE", "Counter_Value": 100},
        {"Kernel_Name": f"void mq::{rq}<256, 0, 3, 0, 1>", "Grid_Size": 2096640, "Counter_Name": "FETCH_SIZE", "Counter_Value": 102},
        {"Kernel_Name": f"void mq::{gemm}<0, 0, 0, false>", "Grid_Size": 393216, "Counter_Name": "FETCH_SIZE", "Counter_Value": 50},
        {"Kernel_Name": f"void mq::{gemv}<0, 0, 0, 1>", "Grid_Size": 294912, "Counter_Name": "FETCH_SIZE", "Counter_Value": 15},
        {"Kernel_Name": f"void mq::{gemv}<0, 0, 0, 1>", "Grid_Size": 294912, "Counter_Name": "FETCH_SIZE", "Counter_Value": 17},
        {"Kernel_Name": f"{copy}<int>", "Grid_Size": 1024, "Counter_Name": "FETCH_SIZE", "Counter_Value": 7},
        {"Kernel_Name": f"{copy}<int>", "Grid_Size": 4096, "Counter_Name": "FETCH_SIZE", "Counter_Value": 131072},
        {"Kernel_Name": f"void mq::{gemm}<0, 0, 0, false>", "Grid_Size": 393216, "Counter_Name": "WRITE_SIZE", "Counter_Value": 1},
    ])
    m = bench._counter_means(str(p), "FETCH_SIZE")
    assert m[rq] == pytest.approx(101.0)        # the M = 32760 launches, not the M = 4096 one
    assert m[gemm] == pytest.approx(50.0)
    assert m[gemv] == pytest.approx(16.0)
    assert m[copy] == pytest.approx(131072.0)   # the calibration copy, not a smaller one


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr and res.stdout == ""


def test_auxiliary_measurement_errors_are_reported_not_raised():
    assert bench._aux(lambda: {"ms": 1.0}) == {"ms": 1.0}
    err = bench._aux(lambda: 1 / 0)
    assert set(err) == {"error"} and err["error"].startswith("ZeroDivisionError")
