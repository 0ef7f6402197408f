"""bench.py's rocprofv3 summarizers on synthetic CSV files (no GPU): the
kernel-trace table and the HBM traffic JSON with its copy calibration."""

import csv
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _write(path, header, rows):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def _bench(*args):
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                         text=True, check=True)
    return out.stdout


def test_summarize_trace(tmp_path):
    _write(tmp_path / "run" / "k_kernel_stats.csv",
           ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs"],
           [["void swiftllm::(anonymous namespace)::paged_decode_kernel<128, 4>(X)", 10, 900000, 90000,
             90.0, 85000, 95000],
            ["__amd_rocclr_copyBuffer", 2, 100000, 50000, 10.0, 40000, 60000]])
    out = _bench("--summarize-trace", str(tmp_path))
    lines = out.strip().splitlines()
    assert lines[0].startswith("| Kernel |")
    assert "| paged_decode_kernel<128, 4>(X) | 10 | 90.00 | 85.00 | 95.00 | 90.0% |" in lines
    assert "| __amd_rocclr_copyBuffer | 2 | 50.00 | 40.00 | 60.00 | 10.0% |" in lines


def test_summarize_pmc_scales_by_the_calibration_copy(tmp_path):
    hdr = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    # 1 GiB copy: FETCH_SIZE reads half of it, WRITE_SIZE all of it (KiB)
    _write(tmp_path / "f" / "p_counter_collection.csv", hdr,
           [[1, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 524288.0],
            [2, "void swiftllm::(anonymous namespace)::k<1>(A)", "FETCH_SIZE", 1000.0],
            [3, "void swiftllm::(anonymous namespace)::k<1>(A)", "FETCH_SIZE", 3000.0],
            [4, "void swiftllm::(anonymous namespace)::other(B)", "FETCH_SIZE", 7.0]])
    _write(tmp_path / "w" / "p_counter_collection.csv", hdr,
           [[1, "__amd_rocclr_copyBuffer", "WRITE_SIZE", 1048576.0],
            [2, "void swiftllm::(anonymous namespace)::k<1>(A)", "WRITE_SIZE", 10.0],
            [3, "void swiftllm::(anonymous namespace)::k<1>(A)", "WRITE_SIZE", 30.0]])
    rec = json.loads(_bench("--summarize-pmc", str(tmp_path / "f"), str(tmp_path / "w"),
                            "--kernel", "k<1>", "--alg-bytes", "4096000", "--workload", "w"))
    assert rec["kernel"] == "k<1>(A)"
    assert rec["fetch_scale"] == 2.0 and rec["write_scale"] == 1.0
    # mean fetch 2000 KiB x 2 + mean write 20 KiB x 1
    assert rec["hbm_bytes_per_launch"] == (2000 * 2 + 20) * 1024
    assert rec["dispatches_averaged"] == 2
    assert rec["other_kernels_same_call"] == {"other(B)": {"fetch_kib": 7.0, "write_kib": 0.0}}
    assert rec["algorithmic_bytes_per_launch"] == 4096000
