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


def test_default_line_sub_records_cover_every_config(monkeypatch):
    """The default line's sub-records: configs 1 and 3-10 in one pass, the
    block-copy and MoE/prefill benches called with their own config number,
    and a config that raises recorded as an error instead of ending the run
    (no GPU: the bench functions are stand-ins)."""
    import argparse

    sys.path.insert(0, str(ROOT))
    import bench

    seen = []

    def rec(cfg):
        return {"us_per_call": float(cfg), "steps": 7, "n_gpus": 1}

    def decode(args, cfg, stream_gbs=None):
        seen.append(("decode", cfg))
        return rec(cfg)

    def moe(args, stream_gbs=None, log_prefix=""):
        seen.append(("moe", 5))
        return rec(5)

    def single(name):
        def run(args):
            seen.append((name, args.config))
            if args.config == 9:
                raise RuntimeError("planted failure")
            return rec(args.config)
        return run

    monkeypatch.setattr(bench, "bench_decode", decode)
    monkeypatch.setattr(bench, "bench_moe", moe)
    monkeypatch.setattr(bench, "bench_blocks", single("blocks"))
    monkeypatch.setattr(bench, "bench_moe_mlp", single("mlp"))
    monkeypatch.setattr(bench, "bench_prefill", single("prefill"))
    monkeypatch.setattr(bench, "bench_moe_decode", single("moe_decode"))
    args = argparse.Namespace(config=2, steps=7)
    subs = bench.other_configs(args, {"stream_read_gbs": None})
    assert sorted(subs, key=int) == ["1", "3", "4", "5", "6", "7", "8", "9", "10"]
    assert seen == [("decode", 1), ("decode", 3), ("decode", 4), ("moe", 5), ("blocks", 6),
                    ("blocks", 7), ("mlp", 8), ("prefill", 9), ("moe_decode", 10)]
    assert args.config == 2, "the headline's arguments are left as they were"
    assert subs["9"] == {"error": "RuntimeError('planted failure')"}
    for k in ("1", "3", "4", "5", "6", "7", "8", "10"):
        assert subs[k]["us_per_call"] == float(k) and subs[k]["steps_timed"] == 7
        assert "n_gpus" not in subs[k] and "steps" not in subs[k]
