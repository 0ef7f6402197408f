#!/usr/bin/env python3
"""Benchmark of the paged-attention decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1..10]
                    [--variant v2|v1] [--partition P] [--rotate R] [--no-cpu]
                    [--no-ceiling] [--ceiling stream|gather|store|rowcopy]

Workload: Llama-3-8B layer decode (32 query heads, 8 kv heads, head_dim 128,
block_size 16, batch 64, context lengths uniform in [512, 4096], randomly
permuted block tables over a pool of 1.25x the blocks needed, fp16 values
~ N(0, 0.5)). A step is one decode call over that batch with every input
already resident in HBM. R copies of the KV pool (default 4, ~3 GB) are
rotated between calls so no call finds its 604 MB of K/V in the 256 MB
Infinity Cache.

Prints one JSON line: the metric (KV-read GB/s), us/call, the roofline of the
decode kernel (algorithmic bytes / kernel time vs the 8 TB/s HBM peak), the
ceiling of the call's own memory access pattern and the NT read stream, both
measured in the same run with the kernels of libswiftllm_ceilings
(include/swiftllm_ceilings.h), and the fp32 CPU restatement timed on this host
as a reference point. `--ceiling X` times one of those kernels alone.

The other configurations are measured the same way: --config 1 (the tiny MHA
batch BASELINE states for the reference's CPU path; us/call, no roofline
claim), --config 3 (8 sequences of 32768 tokens, 64 query heads, split-K),
--config 4 (a ragged step: cache write of 256 new tokens, then decode),
--config 5 (MoE top-2 routing and dispatch of 4096 tokens, hidden 4096, 8
experts), and the "next" rows: --config 6/7 (block copies and swaps), 8 (the
Mixtral MoE layer's expert GEMMs), 9 (paged prefill) and 10 (the same MoE
layer at a 64-token decode batch, where the expert GEMMs stream weights).
With no --config the line is config 2's and carries every other config as a
sub-record under "configs", each timed in the same process on its own inputs.
"""

from __future__ import annotations

import argparse
import copy
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, choices=[1, 2, 3, 4, 5, 6, 7, 8, 9, 10], default=2,
                    help="1: tiny MHA decode (BASELINE's CPU-runnable case, us only); "
                         "2: Llama-3-8B decode (the metric's workload); 3: long-context split-K; "
                         "4: ragged step (cache write + decode); 5: MoE route + dispatch; "
                         "6: copy_blocks (copy-on-write, 32 layers); 7: swap_blocks out and in; "
                         "8: Mixtral MoE MLP (route, dispatch, expert GEMMs, combine); "
                         "9: Llama-3-8B paged prefill (8 prompts of 2048 tokens); "
                         "10: the Mixtral MoE layer at a 64-token decode batch (weights streamed)")
    ap.add_argument("--variant", choices=["v1", "v2"], default=None,
                    help="default: v1 for configs 1 and 2, v2 for configs 3 and 4")
    ap.add_argument("--ceiling", choices=["stream", "gather", "store", "rowcopy", "mfma"], default=None,
                    help="time one ceiling kernel alone (libswiftllm_ceilings) and print its JSON line: "
                         "the NT read stream; config 2/3/4's tile gather (--load-bytes); config 4's "
                         "cache-write stores (--store-mode); config 5's row copies; the expert GEMM's "
                         "MFMA stream on random operands (TFLOP/s)")
    ap.add_argument("--load-bytes", type=int, choices=[8, 16], default=16, help="--ceiling gather")
    ap.add_argument("--store-mode", type=int, choices=[0, 1, 2], default=1,
                    help="--ceiling store: 0 four rows per lane, 1 one line per 4 lanes, 2 whole rows")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="leave the live ceiling measurement out of the line (for profiles)")
    ap.add_argument("--partition", type=int, default=None,
                    help="v2 partition size in tokens, 0 = balanced (stream-K) scheduling; "
                         "default 4096 for configs 3 and 4")
    ap.add_argument("--rotate", type=int, default=None,
                    help="input copies rotated between calls (default 4 for decode, 8 for MoE)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--samples", type=int, default=200, help="launches timed one by one for p10/p50/p90")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="before warmup, one device-to-device copy of this many MiB (a kernel of known "
                         "traffic that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--summarize-trace", metavar="DIR", default=None,
                    help="no GPU work: print a markdown table of the rocprofv3 --kernel-trace --stats "
                         "output under DIR (k_kernel_stats.csv)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"), default=None,
                    help="no GPU work: print the HBM traffic JSON of --kernel from two rocprofv3 --pmc "
                         "runs (FETCH_SIZE, then WRITE_SIZE) of a bench command with --calib-copy-mib")
    ap.add_argument("--skip-side-partition", "--skip-partition512", dest="skip_partition512",
                    action="store_true",
                    help="config 3: do not also time 4096-token partitions beside BASELINE's 512 (for "
                         "profiles whose per-kernel averages should cover the main workload only)")
    ap.add_argument("--no-configs", action="store_true",
                    help="config 2: leave out the sub-records of configs 1 and 3-10 that the default "
                         "line carries (for profiles of config 2 alone)")
    ap.add_argument("--kernel", default=None, help="kernel name substring for --summarize-pmc")
    ap.add_argument("--alg-bytes", type=int, default=0,
                    help="algorithmic bytes per launch of --kernel (--summarize-pmc)")
    ap.add_argument("--workload", default="", help="workload label (--summarize-pmc)")
    return ap.parse_args()


def _find_csv(d, suffix):
    hits = sorted(Path(d).rglob(f"*{suffix}"))
    if not hits:
        raise SystemExit(f"no *{suffix} under {d}")
    return hits[0]


def _short(name):
    """Kernel name without the return type and namespaces."""
    name = name.replace("void ", "").replace("swiftllm::(anonymous namespace)::", "")
    return name


def summarize_trace(d):
    """Markdown table of a rocprofv3 --stats kernel summary."""
    import csv

    rows = list(csv.DictReader(open(_find_csv(d, "kernel_stats.csv"))))
    total = sum(float(r["TotalDurationNs"]) for r in rows) or 1.0
    print("| Kernel | Calls | Average (us) | Min (us) | Max (us) | Share |")
    print("|---|---|---|---|---|---|")
    for r in rows:
        print(f"| {_short(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
              f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
              f"{100.0 * float(r['TotalDurationNs']) / total:.1f}% |")


def _pmc_per_kernel(d, counter):
    """{kernel: [value per dispatch]} of one counter (KiB per dispatch)."""
    import csv
    from collections import defaultdict

    per = defaultdict(lambda: defaultdict(float))
    for r in csv.DictReader(open(_find_csv(d, "counter_collection.csv"))):
        if r["Counter_Name"] != counter:
            continue
        per[_short(r["Kernel_Name"])][r["Dispatch_Id"]] += float(r["Counter_Value"])
    return {k: list(v.values()) for k, v in per.items()}


def summarize_pmc(fetch_dir, write_dir, kernel, alg_bytes, workload):
    """HBM traffic per launch of `kernel`: FETCH_SIZE and WRITE_SIZE (KiB per
    dispatch), each scaled by what the counter reads for the calibration copy
    of known size that bench.py --calib-copy-mib issued in the same run (the
    largest __amd_rocclr_copyBuffer dispatch, which reads and writes
    --calib-copy-mib MiB)."""
    fetch = _pmc_per_kernel(fetch_dir, "FETCH_SIZE")
    write = _pmc_per_kernel(write_dir, "WRITE_SIZE")
    copy = [k for k in fetch if "copyBuffer" in k]
    if not copy:
        raise SystemExit("no calibration copy in the FETCH_SIZE run")
    calib_kib = float(int(os.environ.get("CALIB_MIB", "1024")) * 1024)
    f_scale = calib_kib / max(max(fetch[copy[0]]), 1e-9)
    w_scale = calib_kib / max(max(write[copy[0]]), 1e-9)
    name = [k for k in fetch if kernel in k]
    if not name:
        raise SystemExit(f"kernel {kernel!r} not in {sorted(fetch)}")
    name = name[0]
    f_kib = float(np.mean(fetch[name]))
    w_kib = float(np.mean(write.get(name, [0.0])))
    traffic = int(round(f_kib * 1024 * f_scale + w_kib * 1024 * w_scale))
    others = {k: {"fetch_kib": round(float(np.mean(v)), 1),
                  "write_kib": round(float(np.mean(write.get(k, [0.0]))), 1)}
              for k, v in fetch.items() if k != name and "copyBuffer" not in k}
    rec = {
        "kernel": name,
        "workload": workload,
        "hbm_bytes_per_launch": traffic,
        "fetch_kib_per_dispatch_raw": round(f_kib, 1),
        "write_kib_per_dispatch_raw": round(w_kib, 1),
        "fetch_scale": round(f_scale, 5),
        "write_scale": round(w_scale, 5),
        "calibration": f"one {int(calib_kib) // 1024} MiB device-to-device hipMemcpy in the same process "
                       f"(bench.py --calib-copy-mib): FETCH_SIZE read {max(fetch[copy[0]]):.1f} KiB and "
                       f"WRITE_SIZE {max(write[copy[0]]):.1f} KiB for {int(calib_kib)} KiB moved each way",
        "dispatches_averaged": len(fetch[name]),
        "other_kernels_same_call": others,
        "algorithmic_bytes_per_launch": alg_bytes or None,
    }
    print(json.dumps(rec, indent=1))


def main():
    args = parse()
    if args.summarize_trace:
        return summarize_trace(args.summarize_trace)
    if args.summarize_pmc:
        return summarize_pmc(*args.summarize_pmc, args.kernel or "", args.alg_bytes, args.workload)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the path has no multi-GPU mode.", file=sys.stderr)
        sys.exit(2)

    from swiftllm_amd import _hip, workloads
    from swiftllm_amd import paged_attention as pa
    from swiftllm_amd._hip import DeviceArray, Event, Stream

    if _hip.device_count() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)

    if args.calib_copy_mib > 0:
        calibrate(args.calib_copy_mib << 20)
    if args.ceiling:
        return bench_ceiling(args)
    if args.config == 5:
        print(json.dumps(bench_moe(args)), flush=True)
        return
    single = {6: bench_blocks, 7: bench_blocks, 8: bench_moe_mlp, 9: bench_prefill,
              10: bench_moe_decode}
    if args.config in single:
        print(json.dumps(single[args.config](args)), flush=True)
        return
    rec = bench_decode(args, args.config, variant=args.variant, partition=args.partition)
    if args.config == 2 and not args.no_configs:
        rec["configs"] = other_configs(args, rec)
    print(json.dumps(rec), flush=True)


# Default partition sizes of the split-K configs. Config 3: BASELINE states
# 512-token partitions (64 per sequence); the run also times 4096 beside it
# (measured fastest for long uniform contexts: 165 us, the same as 8192).
# Config 4 (ragged), with the split-K items started longest first: 4096 is
# fastest (175.7 us, against 177.4 at 2048, 182.0 at 1024 and 189.0 balanced).
DEFAULT_PARTITION = {3: 512, 4: 4096}
SIDE_PARTITION = {3: 4096}


def bench_decode(args, config, *, variant=None, partition=None, steps=None, warmup=None,
                 samples=None, stream_gbs=None, log_prefix="[bench]"):
    """One decode configuration (1-4) timed on its own inputs; returns its
    JSON record. A step is one decode call (config 4: the cache write of the
    step's new tokens, then the decode) with every input resident in HBM and
    `--rotate` copies of the KV pool rotated between calls so no call finds
    its K/V in the 256 MB Infinity Cache. `stream_gbs`, when given, is a
    stream ceiling already measured in this process."""
    from swiftllm_amd import _hip, workloads
    from swiftllm_amd import paged_attention as pa
    from swiftllm_amd._hip import DeviceArray, Event, Stream

    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    samples = args.samples if samples is None else samples
    rotate = 4 if args.rotate is None else args.rotate
    if variant is None:
        variant = "v1" if config in (1, 2) else "v2"
    if partition is None:
        partition = DEFAULT_PARTITION.get(config, 4096)
    t0 = time.time()
    w = workloads.decode_config(config, seed=args.seed)
    sh = w.shape
    kv_bytes = w.kv_bytes()
    alg_bytes = kv_bytes + w.other_bytes()
    print(f"{log_prefix} config {config}: workload generated in {time.time() - t0:.1f}s: "
          f"S={sh['num_seqs']} sum(ctx)={int(w.context_lens.sum())} pool={sh['num_blocks']} blocks "
          f"kv_bytes={kv_bytes / 1e6:.1f} MB", file=sys.stderr, flush=True)

    stream = Stream()
    q = DeviceArray.from_numpy(w.q)
    bt = DeviceArray.from_numpy(w.block_tables)
    ctx = DeviceArray.from_numpy(w.context_lens)
    out = DeviceArray(w.q.shape, np.float16)
    pools = [(DeviceArray.from_numpy(w.key_cache), DeviceArray.from_numpy(w.value_cache))
             for _ in range(max(1, rotate))]
    slots = None
    if config == 4:
        k_new = DeviceArray.from_numpy(w.new_key)
        v_new = DeviceArray.from_numpy(w.new_value)
        slots = DeviceArray.from_numpy(w.slot_mapping)

    def make_step(var, part):
        ws = None
        if var == "v2":
            ws = pa.workspace(pa.paged_attention_v2_workspace_size(
                sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"], sh["head_dim"], sh["block_size"],
                sh["max_num_blocks_per_seq"], part), stream)

        def step(i):
            kc, vc = pools[i % len(pools)]
            if config == 4:
                pa.launch_reshape_and_cache(k_new, v_new, kc, vc, slots, sh["num_seqs"],
                                            sh["num_kv_heads"], sh["head_dim"], sh["block_size"],
                                            num_blocks=sh["num_blocks"], stream=stream)
            if var == "v2":
                pa.paged_attention_v2(out, ws, q, kc, vc, bt, ctx, w.scale, sh["num_seqs"],
                                      sh["num_heads"], sh["num_kv_heads"], sh["head_dim"],
                                      sh["block_size"], sh["max_num_blocks_per_seq"], part,
                                      num_blocks=sh["num_blocks"], stream=stream)
            else:
                pa.paged_attention_v1(out, q, kc, vc, bt, ctx, w.scale, sh["num_seqs"],
                                      sh["num_heads"], sh["num_kv_heads"], sh["head_dim"],
                                      sh["block_size"], sh["max_num_blocks_per_seq"],
                                      num_blocks=sh["num_blocks"], stream=stream)
        return step, ws

    step, _ws = make_step(variant, partition)
    for i in range(warmup):
        step(i)
    stream.synchronize()
    print(f"{log_prefix} config {config}: warmup {warmup} done", file=sys.stderr, flush=True)

    # Timed region: K back-to-back launches on one stream between two events.
    start, end = Event(), Event()
    _hip.synchronize()
    start.record(stream)
    for i in range(steps):
        step(i)
    end.record(stream)
    end.synchronize()
    _hip.synchronize()
    ms = start.elapsed_ms(end) / steps
    print(f"{log_prefix} config {config}: timed {steps} steps: {ms * 1e3:.2f} us/call",
          file=sys.stderr, flush=True)

    # Per-launch distribution: each launch bracketed by its own events.
    evs = [(Event(), Event()) for _ in range(samples)]
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        step(i)
        b.record(stream)
    stream.synchronize()
    per = np.array([a.elapsed_ms(b) * 1e3 for a, b in evs]) if evs else np.array([ms * 1e3])
    p10, p50, p90 = (float(np.percentile(per, x)) for x in (10, 50, 90))

    # Single-launch latency: one call on an idle GPU (the stream drained before
    # and after), from its first event to its last.
    single = []
    for i in range(samples and 20):
        a, b = Event(), Event()
        stream.synchronize()
        a.record(stream)
        step(i)
        b.record(stream)
        b.synchronize()
        single.append(a.elapsed_ms(b) * 1e3)
    single_p50 = float(np.median(single)) if single else None

    # The other partition size of a split-K config, timed beside it in the
    # same run on the same inputs.
    side = None
    side_part = SIDE_PARTITION.get(config)
    if variant == "v2" and side_part is not None and side_part != partition and not args.skip_partition512:
        side_step, _side_ws = make_step("v2", side_part)
        ms_side = timed(side_step, stream, steps, min(warmup, 20), 0)[0]
        side = {"partition_tokens": side_part, "us_per_call": round(ms_side * 1e3, 3),
                "kv_gbs": round(kv_bytes / (ms_side * 1e-3) / 1e9, 2),
                "hbm_peak_frac": round(alg_bytes / (ms_side * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        print(f"{log_prefix} config {config}: partition {side_part}: {ms_side * 1e3:.2f} us/call",
              file=sys.stderr, flush=True)

    value = kv_bytes / (ms * 1e-3) / 1e9          # KV-read GB/s
    achieved = alg_bytes / (ms * 1e-3) / 1e9      # all algorithmic bytes / kernel time
    part_tag = f"_p{partition}" if (variant == "v2" and config == 3 and partition != 4096) else ""
    traffic = read_traffic(f"decode_config{config}{part_tag}_traffic.json")

    # Ceilings measured in this run, after the timed calls (the store probe
    # overwrites cache contents): the same K/V tiles read by the gather
    # kernel alone (and for config 4 the cache write's stores alone), and the
    # NT sequential read stream.
    ceiling = None
    if not args.no_ceiling and config != 1:
        ceiling = decode_ceiling(w, pools, bt, stream, max(steps // 4, 20), kv_bytes,
                                 partition if variant == "v2" else 0, slots)
        if stream_gbs is None:
            stream_gbs = measure_stream(stream)[0]
        print(f"{log_prefix} config {config}: ceiling {ceiling['value']:.0f} GB/s "
              f"({ceiling['us_per_call']:.2f} us), stream {stream_gbs:.0f} GB/s", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        import oracle

        threads = oracle.lib().oracle_max_threads()
        oracle.decode_f32(w.q, w.key_cache, w.value_cache, w.block_tables, w.context_lens, w.scale)
        times = []
        t_budget = time.time()
        while len(times) < 5 and (time.time() - t_budget) < 20.0:
            t1 = time.perf_counter()
            oracle.decode_f32(w.q, w.key_cache, w.value_cache, w.block_tables, w.context_lens, w.scale)
            times.append(time.perf_counter() - t1)
        cpu_s = float(np.median(times))
        cpu = {"value": round(kv_bytes / cpu_s / 1e9, 3), "unit": "GB/s", "cores": int(threads),
               "kind": "port", "us_per_call": round(cpu_s * 1e6, 1), **host_info(),
               "sample": f"full config-{config} batch (same inputs, decode only), fp32 C restatement "
                         f"(oracle/oracle.c, OpenMP over (seq, kv head)), median of {len(times)} runs"}
        print(f"{log_prefix} config {config}: cpu baseline {cpu_s * 1e3:.1f} ms/call on {threads} threads",
              file=sys.stderr, flush=True)

    workload_name = {1: "tiny-mha-decode", 2: "llama3-8b-decode-layer", 3: "llama3-70b-long-context-splitk",
                     4: "ragged-continuous-batching-step"}[config]
    ctx_desc = {1: "uniform[1,256]", 2: "uniform[512,4096]", 3: "32768 (all)",
                4: "lognormal(median 600, sigma 1) clip [1,8192]"}[config]
    rec = {
        "metric": "paged-attn decode KV-read GB/s (% HBM peak) + us/call @ Llama-3-8B shape",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 6),
        "us_per_call": round(ms * 1e3, 3),
        "us_per_call_p10_p50_p90": [round(p10, 2), round(p50, 2), round(p90, 2)],
        "us_single_launch_p50": round(single_p50, 2) if single_p50 is not None else None,
        "hbm_peak_frac": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 in/out, f32 accumulate",
        "data": "synthetic (seeded normal fp16 values, random permuted block tables)",
        "config": {
            "workload": workload_name,
            "num_seqs": sh["num_seqs"], "num_heads": sh["num_heads"],
            "num_kv_heads": sh["num_kv_heads"], "head_dim": sh["head_dim"],
            "block_size": sh["block_size"], "context_lens": ctx_desc,
            "sum_context": int(w.context_lens.sum()), "pool_blocks": sh["num_blocks"],
            "kernel": f"paged_attention_{variant}" + (f"/partition{partition}" if variant == "v2" else "")
                      + ("+reshape_and_cache" if config == 4 else ""),
            "kv_pool_copies_rotated": len(pools), "seed": args.seed,
            "kv_bytes_per_call": kv_bytes, "algorithmic_bytes_per_call": alg_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "ceiling": ceiling,
        "ceiling_frac": round(value / ceiling["value"], 4) if ceiling else None,
        "stream_read_gbs": round(stream_gbs, 2) if stream_gbs else None,
        "stream_frac": round(value / stream_gbs, 4) if stream_gbs else None,
        "cpu_baseline": cpu,
    }
    if variant == "v2":
        rec["config"]["partition_tokens"] = partition
    if config == 1:
        # latency-bound (1 MB per call): us/call only, no roofline claim
        rec["metric"] = "paged-attn decode us/call @ tiny MHA (BASELINE config 1, CPU-runnable case)"
        rec["value"], rec["unit"], rec["higher_is_better"] = round(ms * 1e3, 3), "us", False
        rec["roofline"] = None
        rec["ceiling_frac"] = rec["stream_frac"] = None
        if cpu:
            cpu.update(value=cpu["us_per_call"], unit="us")
    if side is not None:
        rec[f"partition{side['partition_tokens']}"] = side
    return rec


# Keys of a configuration's record that the line's own header already states.
_SUB_DROP = ("n_gpus", "scaling", "vs_baseline", "higher_is_better", "steps", "warmup")


def other_configs(args, main_rec):
    """Every other config, each on its own seeded inputs, timed in this
    process after the headline config 2, as sub-records of its line.
    BASELINE configs 1, 3, 4 and 5: us/call, the roofline of the algorithmic
    bytes against 8 TB/s with the committed HBM traffic, the live ceiling of
    the call's own access pattern, and the CPU restatement on this host
    (config 3 at BASELINE's 512-token partitions, with 4096-token partitions
    timed beside it). Configs 6-10 (block copies, the MoE layer at 4096 and
    64 tokens, paged prefill): their own records without a CPU leg. A config
    that fails records its error instead, so the headline line is printed
    whatever happens to the others."""
    stream_gbs = main_rec.get("stream_read_gbs")
    single = {6: bench_blocks, 7: bench_blocks, 8: bench_moe_mlp, 9: bench_prefill,
              10: bench_moe_decode}
    subs = {}
    for cfg in (1, 3, 4, 5, 6, 7, 8, 9, 10):
        try:
            if cfg == 5:
                rec = bench_moe(args, stream_gbs=stream_gbs, log_prefix="[bench]")
            elif cfg in single:
                sub_args = copy.copy(args)
                sub_args.config = cfg
                rec = single[cfg](sub_args)
            else:
                rec = bench_decode(args, cfg, stream_gbs=stream_gbs)
        except Exception as e:  # recorded, so that the headline still prints
            print(f"[bench] config {cfg} failed: {e!r}", file=sys.stderr, flush=True)
            subs[str(cfg)] = {"error": repr(e)}
            continue
        rec["steps_timed"] = rec.get("steps")
        subs[str(cfg)] = {k: v for k, v in rec.items() if k not in _SUB_DROP}
    return subs


def calibrate(nbytes):
    """Kernels of known traffic for scaling rocprofv3's FETCH_SIZE and
    WRITE_SIZE: one device-to-device copy of `nbytes` (reads and writes
    `nbytes`) and one workspace clear of `nbytes` (writes `nbytes`)."""
    from swiftllm_amd import _hip, _lib
    from swiftllm_amd import paged_attention as pa
    from swiftllm_amd._hip import DeviceArray

    src, dst = DeviceArray((nbytes // 4,), np.uint32), DeviceArray((nbytes // 4,), np.uint32)
    src.fill_byte(1)
    _hip.synchronize()
    _hip.check(_hip.hip().hipMemcpy(dst.ptr, src.ptr, nbytes, _hip.HIP_MEMCPY_D2D), "calibration copy")
    pa.check_status(_lib.lib().swiftllm_hip_workspace_clear(dst.ptr, nbytes, None))
    _hip.synchronize()
    src.free()
    dst.free()


def host_info():
    """Host CPU threads this process may run on and the CPU model, stated
    beside every CPU baseline."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": nproc, "cpu_model": model}


STREAM_BYTES = 2 << 30  # beyond the 256 MB Infinity Cache


def measure_stream(stream, steps=20):
    """The NT sequential read stream of libswiftllm_ceilings over a 2 GiB
    buffer: (GB/s, us per launch), launches back to back."""
    from swiftllm_amd import ceilings
    from swiftllm_amd._hip import DeviceArray

    buf = DeviceArray((STREAM_BYTES // 4,), np.uint32)
    buf.fill_byte(0x5A)
    sink = DeviceArray((1,), np.uint32)
    ms = timed(lambda i: ceilings.read_stream(buf, STREAM_BYTES, sink, stream), stream, steps, 3, 0)[0]
    buf.free()
    return STREAM_BYTES / (ms * 1e-3) / 1e9, ms * 1e3


def measure_gather(w, pools, bt, stream, steps, load_bytes, partition_tokens):
    """The decode's K/V tile reads alone (libswiftllm_ceilings tile gather)
    over the same rotated pools and block tables, in the decode's work items
    (whole (sequence, kv head) units for the single pass, partitions of
    partition_tokens for split-K): us per call, launches back to back."""
    from swiftllm_amd import _hip, ceilings
    from swiftllm_amd._hip import DeviceArray

    sh = w.shape
    Hkv = sh["num_kv_heads"]
    items = ceilings.gather_items(w.context_lens, Hkv, partition_tokens, _hip.cu_count())
    d_items = DeviceArray.from_numpy(items)
    sink = DeviceArray((1,), np.uint32)

    def step(i):
        kc, vc = pools[i % len(pools)]
        ceilings.tile_gather(kc, vc, bt, d_items, len(items), sh["num_seqs"], Hkv, sh["head_dim"],
                             sh["max_num_blocks_per_seq"], sh["num_blocks"], load_bytes, sink, stream)

    return timed(step, stream, steps, 10, 0)[0] * 1e3


def measure_store(w, pools, slots, stream, steps, mode):
    """reshape_and_cache's stores alone (libswiftllm_ceilings cache store,
    `mode` as in include/swiftllm_ceilings.h) at the workload's slots, into
    the same rotated pools: us per call."""
    from swiftllm_amd import ceilings

    sh = w.shape

    def step(i):
        kc, vc = pools[i % len(pools)]
        ceilings.cache_store(kc, vc, slots, sh["num_seqs"], sh["num_kv_heads"], sh["head_dim"],
                             sh["num_blocks"], mode, stream)

    return timed(step, stream, steps, 10, 0)[0] * 1e3


# The MFMA stream's grid: the gated expert GEMM of config 8 (32 row tiles x
# 112 column tiles of 256 x 128 outputs, k = 4096 in 64 stages of 64).
MFMA_GROUPS, MFMA_STAGES = 32 * 112, 64


def measure_mfma(stream, steps=10, seed=0):
    """Dense fp16 MFMA rate this box sustains on random operands: the
    expert GEMM's matrix instructions alone (libswiftllm_ceilings MFMA
    stream) over the gated GEMM's grid. Returns (TFLOP/s, us per launch)."""
    from swiftllm_amd import ceilings
    from swiftllm_amd._hip import DeviceArray

    rng = np.random.default_rng(seed)
    ops = DeviceArray.from_numpy(rng.standard_normal(1 << 19).astype(np.float16))  # 1 MiB
    sink = DeviceArray((1,), np.uint32)

    def step(i):
        ceilings.mfma_stream(ops, ops.nbytes, MFMA_GROUPS, MFMA_STAGES, sink, stream)

    us = timed(step, stream, steps, 3, 0)[0] * 1e3
    flop = ceilings.MFMA_FLOP_PER_GROUP_STAGE * MFMA_GROUPS * MFMA_STAGES
    return flop / (us * 1e-6) / 1e12, us


def mfma_ceiling(stream, no_ceiling):
    if no_ceiling:
        return None
    tflops, us = measure_mfma(stream)
    return {"pattern": "the expert GEMM's MFMA instructions alone (libswiftllm_ceilings MFMA stream: "
                       "its grid, 8 waves per workgroup, 128 x 64 wave tiles of v_mfma_f32_32x32x16_f16, "
                       "random fp16 operands in registers, no memory traffic)",
            "value": round(tflops, 2), "unit": "TFLOP/s", "us_per_launch": round(us, 3)}


def decode_ceiling(w, pools, bt, stream, steps, kv_bytes, partition_tokens, slots=None):
    """The access-pattern ceiling of a decode call: the tile gather at 8- and
    16-byte loads in the decode's own work items (the faster counts), plus
    for a ragged step the cache write's stores (modes 0 and 1, the faster
    counts). Returns the ceiling record; its value is K/V bytes / the
    pattern's time, like `value`. Run it after the timed calls: the store
    probe overwrites cache contents."""
    g8 = measure_gather(w, pools, bt, stream, steps, 8, partition_tokens)
    g16 = measure_gather(w, pools, bt, stream, steps, 16, partition_tokens)
    rec = {"pattern": "tile gather of the call's K/V tiles in its work items (libswiftllm_ceilings, "
                      "NT loads)", "partition_tokens": partition_tokens,
           "gather8_us": round(g8, 3), "gather16_us": round(g16, 3)}
    t = min(g8, g16)
    if slots is not None:
        st = [measure_store(w, pools, slots, stream, steps, m) for m in (0, 1, 2)]
        rec["pattern"] += " + reshape_and_cache's 2-byte stores"
        rec["store_us_4rows_per_lane"] = round(st[0], 3)
        rec["store_us_line_per_4_lanes"] = round(st[1], 3)
        rec["store_us_whole_rows"] = round(st[2], 3)
        t += min(st[0], st[1])
    rec.update(value=round(kv_bytes / (t * 1e-6) / 1e9, 2), unit="GB/s", us_per_call=round(t, 3))
    return rec


def read_traffic(name):
    """HBM bytes per launch of the dominant kernel, from the committed
    rocprofv3 counter summary, or None when there is none."""
    tf = ROOT / "profiles" / name
    if not tf.exists():
        return None
    try:
        return json.loads(tf.read_text()).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def timed(step, stream, steps, warmup, samples):
    """Warmup, then `steps` launches between two events on `stream`, then
    `samples` individually timed launches. Returns (ms per step, p10, p50, p90 in us)."""
    from swiftllm_amd import _hip
    from swiftllm_amd._hip import Event

    for i in range(warmup):
        step(i)
    stream.synchronize()
    start, end = Event(), Event()
    _hip.synchronize()
    start.record(stream)
    for i in range(steps):
        step(i)
    end.record(stream)
    end.synchronize()
    ms = start.elapsed_ms(end) / steps
    evs = [(Event(), Event()) for _ in range(samples)]
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        step(i)
        b.record(stream)
    stream.synchronize()
    per = np.array([a.elapsed_ms(b) * 1e3 for a, b in evs]) if evs else np.array([ms * 1e3])
    return (ms,) + tuple(float(np.percentile(per, x)) for x in (10, 50, 90))


def bench_ceiling(args):
    """`--ceiling`: one access-pattern kernel of libswiftllm_ceilings timed
    alone, for its rocprofv3 profile and as the committed source of the
    ceilings the other lines measure live. Prints one JSON line (GB/s of the
    pattern's own bytes)."""
    from swiftllm_amd import ceilings, workloads
    from swiftllm_amd._hip import DeviceArray, Stream

    stream = Stream()
    steps = max(args.steps // 4, 20)
    if args.ceiling == "stream":
        gbs, us = measure_stream(stream, steps)
        nbytes, work = STREAM_BYTES, {"workload": "nt-read-stream", "bytes_per_call": STREAM_BYTES,
                                      "loads": "16-byte nontemporal, grid-stride"}
    elif args.ceiling in ("gather", "store"):
        cfg = args.config if args.config in (2, 3, 4) else (4 if args.ceiling == "store" else 2)
        w = workloads.decode_config(cfg, seed=args.seed)
        sh = w.shape
        pools = [(DeviceArray.from_numpy(w.key_cache), DeviceArray.from_numpy(w.value_cache))
                 for _ in range(max(1, args.rotate or 4))]
        bt, ctx = DeviceArray.from_numpy(w.block_tables), DeviceArray.from_numpy(w.context_lens)
        if args.ceiling == "gather":
            part = args.partition if args.partition is not None else {2: 0, 3: 4096, 4: 4096}[cfg]
            us = measure_gather(w, pools, bt, stream, steps, args.load_bytes, part)
            nbytes = w.kv_bytes()
            work = {"workload": f"config{cfg}-tile-gather", "load_bytes": args.load_bytes,
                    "partition_tokens": part, "kv_bytes_per_call": nbytes,
                    "kv_pool_copies_rotated": len(pools)}
        else:
            if w.slot_mapping is None:
                raise SystemExit("--ceiling store needs config 4 (a ragged step with new tokens)")
            slots = DeviceArray.from_numpy(w.slot_mapping)
            us = measure_store(w, pools, slots, stream, steps, args.store_mode)
            nbytes = 2 * sh["num_seqs"] * sh["num_kv_heads"] * sh["head_dim"] * 2
            work = {"workload": f"config{cfg}-cache-write-stores", "store_mode": args.store_mode,
                    "tokens": sh["num_seqs"], "bytes_written_per_call": nbytes,
                    "kv_pool_copies_rotated": len(pools)}
        gbs = nbytes / (us * 1e-6) / 1e9
    elif args.ceiling == "mfma":
        tflops, us = measure_mfma(stream, steps=max(args.steps // 10, 10), seed=args.seed)
        rec = {"metric": "MFMA stream ceiling TFLOP/s (libswiftllm_ceilings)", "value": round(tflops, 2),
               "unit": "TFLOP/s", "n_gpus": 1, "us_per_call": round(us, 3),
               "mfma_peak_frac": round(tflops / 2500.0, 4), "higher_is_better": True,
               "dtype": "f16 operands, f32 accumulate (v_mfma_f32_32x32x16_f16)",
               "data": "synthetic (seeded standard normal fp16 operands)",
               "config": {"workload": "expert-gemm-mfma-stream", "workgroups": MFMA_GROUPS,
                          "stages": MFMA_STAGES, "waves_per_workgroup": 8,
                          "flop_per_launch": ceilings.MFMA_FLOP_PER_GROUP_STAGE * MFMA_GROUPS * MFMA_STAGES}}
        print(json.dumps(rec), flush=True)
        return
    else:
        wl = workloads.moe_config(seed=args.seed)
        T, hidden = wl.x.shape
        K = wl.top_k
        copies = max(1, args.rotate or 8)
        rng = np.random.default_rng(args.seed)
        rows = [DeviceArray.from_numpy(rng.permutation(T * K).astype(np.int32).reshape(T, K))
                for _ in range(copies)]
        xs = [DeviceArray.from_numpy(wl.x) for _ in range(copies)]
        dst = [DeviceArray((T * K, hidden), np.float16) for _ in range(copies)]

        def step(i):
            c = i % copies
            ceilings.row_copy(xs[c], dst[c], rows[c], T, K, hidden, T * K, stream)

        us = timed(step, stream, steps, 10, 0)[0] * 1e3
        nbytes = 2 * T * hidden + 2 * T * K * hidden
        gbs = nbytes / (us * 1e-6) / 1e9
        work = {"workload": "config5-row-copy", "tokens": T, "hidden": hidden, "top_k": K,
                "bytes_per_call": nbytes, "copies_rotated": copies}
    rec = {"metric": f"{args.ceiling} ceiling GB/s (libswiftllm_ceilings)", "value": round(gbs, 2),
           "unit": "GB/s", "n_gpus": 1, "us_per_call": round(us, 3),
           "hbm_peak_frac": round(gbs / HBM_PEAK_GBS, 4), "higher_is_better": True,
           "dtype": "u8 (memory access pattern only)", "data": "synthetic", "config": work}
    print(json.dumps(rec), flush=True)


def bench_moe(args, stream_gbs=None, log_prefix="[bench]"):
    """Config 5: Mixtral-8x7B-style routing + dispatch (4096 tokens, hidden 4096,
    8 experts, top-2). Eight copies of the activations and outputs rotate so
    the 256 MB Infinity Cache cannot hold a call's 100.9 MB. Returns the JSON
    record; `stream_gbs`, when given, is a stream ceiling already measured in
    this process."""
    from swiftllm_amd import moe, workloads
    from swiftllm_amd._hip import DeviceArray, Stream

    wl = workloads.moe_config(seed=args.seed)
    T, hidden = wl.x.shape
    E, K = wl.num_experts, wl.top_k
    stream = Stream()
    copies = max(1, args.rotate or 8)
    xs = [DeviceArray.from_numpy(wl.x) for _ in range(copies)]
    logits = [DeviceArray.from_numpy(wl.logits) for _ in range(copies)]
    bufs = [moe.DispatchBuffers.allocate(T, E, K, hidden) for _ in range(copies)]
    ids = [DeviceArray((T, K), np.int32) for _ in range(copies)]
    wts = [DeviceArray((T, K), np.float32) for _ in range(copies)]

    def step(i):
        c = i % copies
        moe.moe_route_dispatch(logits[c], xs[c], K, ids[c], wts[c], bufs[c], stream)

    def step_two_calls(i):
        c = i % copies
        moe.moe_route(logits[c], K, ids[c], wts[c], stream)
        moe.moe_dispatch(ids[c], xs[c], E, bufs[c], stream)

    ms2 = timed(step_two_calls, stream, max(args.steps // 4, 1), args.warmup, 0)[0]
    ms, p10, p50, p90 = timed(step, stream, args.steps, args.warmup, args.samples)
    alg = wl.bytes()
    value = alg / (ms * 1e-3) / 1e9
    print(f"{log_prefix} config 5: timed {args.steps} steps: {ms * 1e3:.2f} us/call "
          f"(route then dispatch: {ms2 * 1e3:.2f})", file=sys.stderr, flush=True)

    # Ceiling measured in this run: the call's row copies alone (each row read
    # once, written to its top-k destinations at the rows the dispatch chose),
    # over the same rotated buffers; and the NT sequential read stream.
    ceiling = None
    if not args.no_ceiling:
        from swiftllm_amd import ceilings

        rows = [b.inverse for b in bufs]

        def copy_step(i):
            c = i % copies
            ceilings.row_copy(xs[c], bufs[c].x_perm, rows[c], T, K, hidden, T * K, stream)

        t_copy = timed(copy_step, stream, max(args.steps // 4, 20), 10, 0)[0] * 1e3
        ceiling = {"pattern": "the call's row copies alone (libswiftllm_ceilings row copy, 16-byte "
                              "NT loads and stores, destinations from the dispatch)",
                   "value": round(alg / (t_copy * 1e-6) / 1e9, 2), "unit": "GB/s",
                   "us_per_call": round(t_copy, 3)}
        if stream_gbs is None:
            stream_gbs = measure_stream(stream)[0]
    cpu = None
    if not args.no_cpu:
        import oracle

        oracle.moe_route_dispatch_serial(wl.logits, wl.x, K)
        t_budget, times = time.time(), []
        while len(times) < 5 and time.time() - t_budget < 20.0:
            t1 = time.perf_counter()
            oracle.moe_route_dispatch_serial(wl.logits, wl.x, K)
            times.append(time.perf_counter() - t1)
        cpu_s = float(np.median(times))
        cpu = {"value": round(alg / cpu_s / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "us_per_call": round(cpu_s * 1e6, 1), **host_info(),
               "sample": f"full config-5 batch: C restatement on one thread (oracle/oracle.c "
                         f"oracle_moe_route_dispatch_serial: fp32 softmax, top-2, serial counting "
                         f"sort, row copies), median of {len(times)} runs"}
    rec = {
        "metric": "MoE top-2 route + dispatch GB/s (algorithmic bytes) + us/call @ Mixtral-8x7B shape",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "us_per_call": round(ms * 1e3, 3),
        "us_per_call_p10_p50_p90": [round(p10, 2), round(p50, 2), round(p90, 2)],
        "us_per_call_route_then_dispatch": round(ms2 * 1e3, 3),
        "hbm_peak_frac": round(value / HBM_PEAK_GBS, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 routing, f16 rows (bit copies)",
        "data": "synthetic (seeded N(0,1) logits and activations)",
        "config": {"workload": "mixtral-8x7b-moe-dispatch", "num_tokens": T, "hidden": hidden,
                   "num_experts": E, "top_k": K, "copies_rotated": copies,
                   "algorithmic_bytes_per_call": alg,
                   "entry": "swiftllm_hip_moe_route_dispatch (rank with routing, then permute)"},
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic("moe_config5_traffic.json")},
        "ceiling": ceiling,
        "ceiling_frac": round(value / ceiling["value"], 4) if ceiling else None,
        "stream_read_gbs": round(stream_gbs, 2) if stream_gbs else None,
        "stream_frac": round(value / stream_gbs, 4) if stream_gbs else None,
        "cpu_baseline": cpu,
    }
    return rec


def bench_prefill(args):
    """Config 9: paged prefill at the Llama-3-8B layer shape (32 query heads,
    8 kv heads, head_dim 128): 8 prompts of 2048 tokens packed (16384
    tokens), their K/V already in a randomly permuted block pool. A step is
    one causal-attention call over the batch."""
    from swiftllm_amd import paged_attention as pa
    from swiftllm_amd import workloads
    from swiftllm_amd._hip import DeviceArray, Stream

    w = workloads.prefill_config((2048,) * 8, 32, 8, 128, seed=args.seed, poison=False)
    T, H, D = w.q.shape
    S = len(w.context_lens)
    stream = Stream()
    q = DeviceArray.from_numpy(w.q)
    kc, vc = DeviceArray.from_numpy(w.key_cache), DeviceArray.from_numpy(w.value_cache)
    sm, ctx = DeviceArray.from_numpy(w.slot_mapping), DeviceArray.from_numpy(w.context_lens)
    out = DeviceArray((T, H, D), np.float16)

    def step(i):
        pa.launch_paged_prefill(out, q, kc, vc, sm, ctx, w.scale, S, H, 8, D, 16, 2048,
                                num_blocks=w.key_cache.shape[0], stream=stream)

    steps = max(args.steps // 10, 10)
    warmup = min(args.warmup, 10)
    ms, p10, p50, p90 = timed(step, stream, steps, warmup, min(args.samples, 50))
    tflops = w.flops() / (ms * 1e-3) / 1e12
    rec = {
        "metric": "paged prefill TFLOP/s (causal attention) + us/call @ Llama-3-8B layer, 8 x 2048 tokens",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 6), "us_per_call": round(ms * 1e3, 3),
        "us_per_call_p10_p50_p90": [round(p10, 2), round(p50, 2), round(p90, 2)],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 in/out, f32 accumulate", "data": "synthetic (seeded normal fp16 Q/K/V)",
        "config": {"workload": "llama3-8b-prefill-layer", "prompts": S, "prompt_len": 2048,
                   "num_heads": H, "num_kv_heads": 8, "head_dim": D, "block_size": 16,
                   "flops_per_call": w.flops(), "algorithmic_bytes_per_call": w.bytes()},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4),
                     "traffic": read_traffic("prefill_config9_traffic.json")},
        "cpu_baseline": None,
    }
    ceiling = mfma_ceiling(stream, args.no_ceiling)
    rec["ceiling"] = ceiling
    rec["ceiling_frac"] = round(tflops / ceiling["value"], 4) if ceiling else None
    return rec


def bench_moe_decode(args):
    """Config 10: the Mixtral-8x7B MoE layer of config 8 at a decode batch of
    64 tokens (top-2 of 8 experts: about 16 rows per expert). Every expert's
    rows are one short tail, so both expert GEMMs run in the thin kernel and
    the call streams the gate, up and down weights of every expert that
    received a token: HBM-bound. Algorithmic bytes per call = those weights +
    the activations the call reads and writes (x, its permuted copy, the
    intermediate, the expert outputs, the output); value = those bytes / call
    time. The live ceiling is the sequential nontemporal read stream."""
    from swiftllm_amd import moe, workloads
    from swiftllm_amd._hip import DeviceArray, Stream

    wl = workloads.moe_config(seed=args.seed, num_tokens=64)
    T, hidden = wl.x.shape
    E, K, I = wl.num_experts, wl.top_k, 14336
    rng = np.random.default_rng(args.seed + 1)
    stream = Stream()

    def stacked(n, k):
        return DeviceArray.from_numpy(workloads.expert_weights(rng, E, n, k))

    wg, wu, wd = stacked(I, hidden), stacked(I, hidden), stacked(hidden, I)
    mlp = moe.MoeMlp(E, K, wg, wu, wd)
    x, logits = DeviceArray.from_numpy(wl.x), DeviceArray.from_numpy(wl.logits)

    def step(i):
        mlp.forward(logits, x, stream)

    ms, p10, p50, p90 = timed(step, stream, args.steps, args.warmup, min(args.samples, 50))
    counts = mlp.buffers(T, hidden)["dispatch"].counts.numpy()
    used = int((counts > 0).sum())
    rows = T * K
    weight_bytes = used * 3 * hidden * I * 2
    act_bytes = 2 * (T * hidden + 2 * rows * hidden + 2 * rows * I + 2 * rows * hidden + T * hidden)
    alg = weight_bytes + act_bytes
    value = alg / (ms * 1e-3) / 1e9
    stream_gbs = None if args.no_ceiling else measure_stream(stream)[0]
    rec = {
        "metric": "MoE MLP decode GB/s (expert weights streamed) + us/call @ Mixtral-8x7B layer, 64 tokens",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "us_per_call": round(ms * 1e3, 3),
        "us_per_call_p10_p50_p90": [round(p10, 2), round(p50, 2), round(p90, 2)],
        "hbm_peak_frac": round(value / HBM_PEAK_GBS, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16 in/out, f32 accumulate",
        "data": "synthetic (seeded normal activations, logits, weights)",
        "config": {"workload": "mixtral-8x7b-moe-mlp-decode", "num_tokens": T, "hidden": hidden,
                   "intermediate": I, "num_experts": E, "top_k": K, "experts_used": used,
                   "rows_per_expert": [int(c) for c in counts],
                   "algorithmic_bytes_per_call": alg, "weight_bytes_per_call": weight_bytes,
                   "flops_per_call": 2 * rows * hidden * I * 3,
                   "kernels": "rank+route, permute, thin expert GEMM (gated), thin expert GEMM, combine"},
        # achieved: the whole call's algorithmic bytes / call time (all five kernels),
        # a lower bound on the dominant kernel's own rate; traffic: HBM bytes per
        # launch of the dominant kernel, the gated thin GEMM (1.88 GB of weights)
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic("moe_decode_config10_traffic.json")},
        "ceiling": {"pattern": "sequential nontemporal read stream (libswiftllm_ceilings)",
                    "value": round(stream_gbs, 2), "unit": "GB/s"} if stream_gbs else None,
        "ceiling_frac": round(value / stream_gbs, 4) if stream_gbs else None,
        "cpu_baseline": None,
    }
    return rec


def bench_moe_mlp(args):
    """Config 8: the whole Mixtral-8x7B MoE layer after the router: top-2 of
    8 experts for 4096 tokens (config 5's inputs), the gated expert GEMM
    (hidden 4096 -> 2 x 14336 with SiLU * up fused), the down GEMM
    (14336 -> 4096) and the weighted combine. Weights are random fp16 and
    differ between experts (workloads.expert_weights)."""
    from swiftllm_amd import moe, workloads
    from swiftllm_amd._hip import DeviceArray, Stream

    wl = workloads.moe_config(seed=args.seed)
    T, hidden = wl.x.shape
    E, K, I = wl.num_experts, wl.top_k, 14336
    rng = np.random.default_rng(args.seed + 1)
    stream = Stream()

    def stacked(n, k):
        return DeviceArray.from_numpy(workloads.expert_weights(rng, E, n, k))

    wg, wu, wd = stacked(I, hidden), stacked(I, hidden), stacked(hidden, I)
    mlp = moe.MoeMlp(E, K, wg, wu, wd)
    x, logits = DeviceArray.from_numpy(wl.x), DeviceArray.from_numpy(wl.logits)

    def step(i):
        mlp.forward(logits, x, stream)

    steps = max(args.steps // 10, 10)
    warmup = min(args.warmup, 10)
    ms, p10, p50, p90 = timed(step, stream, steps, warmup, min(args.samples, 20))
    flops = 2 * T * K * hidden * I * 3
    tflops = flops / (ms * 1e-3) / 1e12
    rec = {
        "metric": "MoE MLP TFLOP/s (expert GEMMs) + us/call @ Mixtral-8x7B layer, 4096 tokens",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 6), "us_per_call": round(ms * 1e3, 3),
        "us_per_call_p10_p50_p90": [round(p10, 2), round(p50, 2), round(p90, 2)],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 in/out, f32 accumulate", "data": "synthetic (seeded normal activations, logits, weights)",
        "config": {"workload": "mixtral-8x7b-moe-mlp", "num_tokens": T, "hidden": hidden,
                   "intermediate": I, "num_experts": E, "top_k": K, "flops_per_call": flops,
                   "kernels": "rank+route, permute, expert GEMM (gated), expert GEMM, combine"},
        # achieved: the whole call's expert-GEMM flops / call time (all five kernels);
        # traffic: HBM bytes per launch of the dominant kernel, the gated GEMM
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4),
                     "traffic": read_traffic("moe_mlp_config8_traffic.json")},
        "cpu_baseline": None,
    }
    ceiling = mfma_ceiling(stream, args.no_ceiling)
    rec["ceiling"] = ceiling
    rec["ceiling_frac"] = round(tflops / ceiling["value"], 4) if ceiling else None
    return rec


def bench_blocks(args):
    """Config 6: copy-on-write of 128 block pairs in the K and V caches of 32
    Llama-3-8B layers (8 kv heads, head_dim 128, block_size 16: 32 KiB per
    block and array, 256 MiB read + 256 MiB written per call), two mappings
    alternating. Config 7: swap-out of 1024 blocks of one such cache array to
    pinned host memory and swap-in of 1024 others (32 MiB each way)."""
    from swiftllm_amd import paged_attention as pa
    from swiftllm_amd._hip import DeviceArray, HostArray, Stream

    stream = Stream()
    Hkv, D, BS = 8, 128, 16
    block = Hkv * D * BS * 2
    rng = np.random.default_rng(args.seed)
    if args.config == 6:
        layers, NB, pairs = 32, 1024, 128
        kcs = [DeviceArray((NB * block // 4,), np.uint32) for _ in range(layers)]
        vcs = [DeviceArray((NB * block // 4,), np.uint32) for _ in range(layers)]
        for c in kcs + vcs:
            c.fill_byte(0x3C)
        maps = []
        for _ in range(2):
            ids = rng.permutation(NB)[:2 * pairs]
            maps.append(DeviceArray.from_numpy(np.stack([ids[:pairs], ids[pairs:]], 1).astype(np.int64)))

        def step(i):
            pa.copy_blocks(kcs, vcs, maps[i % 2], pairs, Hkv, D, BS, stream)

        moved = pairs * 2 * layers * block
        alg = 2 * moved
        work = {"workload": "copy-blocks-cow", "layers": layers, "pairs": pairs,
                "block_bytes_per_array": block, "pool_blocks": NB, "mappings_alternated": 2,
                "algorithmic_bytes_per_call": alg}
        metric = "copy_blocks GB/s (bytes read + written) @ 32 Llama-3-8B layers"
        roof = {"bound": "hbm", "peak": HBM_PEAK_GBS}
    else:
        nblk, NBD, NBH = 1024, 4096, 4096
        dev = DeviceArray((NBD * block // 4,), np.uint32)
        host = HostArray((NBH * block // 4,), np.uint32)
        dev.fill_byte(0x3C)
        host.array()[...] = 0x3C3C3C3C
        out_map = DeviceArray.from_numpy(np.stack([rng.permutation(NBD)[:nblk],
                                                   rng.permutation(NBH)[:nblk]], 1).astype(np.int64))
        in_map = DeviceArray.from_numpy(np.stack([rng.permutation(NBH)[:nblk],
                                                  rng.permutation(NBD)[:nblk]], 1).astype(np.int64))

        def step(i):
            pa.swap_blocks(dev, host, out_map, nblk, block, stream)
            pa.swap_blocks(host, dev, in_map, nblk, block, stream)

        alg = 2 * nblk * block
        work = {"workload": "swap-blocks-out-in", "blocks_each_way": nblk, "block_bytes": block,
                "host_memory": "hipHostMalloc pinned", "algorithmic_bytes_per_call": alg}
        metric = "swap_blocks GB/s over the host link (out + in) @ Llama-3-8B blocks"
        # PCIe 5.0 x16 moves 64 GB/s each way; out and in run one after the other.
        roof = {"bound": "pcie", "peak": 64.0}
    # A swap call takes about a millisecond: fewer steps keep the run short.
    steps = args.steps if args.config == 6 else max(args.steps // 20, 5)
    warmup = args.warmup if args.config == 6 else 3
    ms, p10, p50, p90 = timed(step, stream, steps, warmup, args.samples if args.config == 6 else 0)
    value = alg / (ms * 1e-3) / 1e9
    rec = {
        "metric": metric, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(ms, 6), "us_per_call": round(ms * 1e3, 3),
        "us_per_call_p10_p50_p90": [round(p10, 2), round(p50, 2), round(p90, 2)],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8 (bit copies)",
        "data": "synthetic (filled pools)", "config": work,
        "roofline": dict(roof, achieved=round(value, 2), unit="GB/s",
                         frac=round(value / roof["peak"], 4), traffic=None),
        "cpu_baseline": None,
    }
    return rec


if __name__ == "__main__":
    main()
