#!/usr/bin/env python3
"""Field scan benchmark on one MI355X (the hot path of Fields LM's native Field block).

A "step" is one ``fl_scan_forward`` over one batch of config 2 (B=8, T=2048, d_model=1024,
C=512): bf16 raw [8,2048,1536] resident in HBM -> fp32 read [8,2048,2048], state carried across
chunks. ``value`` is tokens/s of the whole step; ``roofline`` prices the same launch against
MI355X's 8 TB/s HBM with the algorithmic bytes 3C*2 + 4C*4 = 11,264 B/token; ``cpu_baseline``
times the torch restatement of the reference's CPU path (oracle/reference_path.py) on the
host's cores on the same workload.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline] [--no-extras]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
METRIC = "Field scan tokens/s + % HBM peak (B8 T2048 d1024); decode tok/s at B64"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def copy_calibration() -> int:
    """Plain device copy of a known size (256 MiB, 10 times): the reference reading for the
    FETCH_SIZE / WRITE_SIZE counters (profiles/*pmc*.txt give the scale factors)."""
    import torch

    n = 256 * 2**20 // 4
    x = torch.randn(n, device="cuda")
    y = torch.empty_like(x)
    for _ in range(10):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": n * 4, "launches": 10}), flush=True)
    return 0


def measured_traffic(workload: str):
    """HBM bytes per launch of the scan from the committed rocprofv3 --pmc summary, or None."""
    path = REPO / "profiles" / f"fl_scan_lookback_kernel_{workload}_pmc.txt"
    if not path.exists():
        return None
    vals = {}
    for line in path.read_text().splitlines():
        if "=" in line and not line.startswith("#") and not line.startswith("cmd"):
            k, v = line.split("=", 1)
            try:
                vals[k.strip()] = float(v.strip())
            except ValueError:
                pass
    try:
        return (vals["fetch_kib"] * vals["fetch_factor"] + vals["write_kib"] * vals["write_factor"]) * 1024
    except KeyError:
        return None


def time_plan(plan, steps: int, warmup: int):
    """Returns (wall ms per step, event ms per step). Events sit on the launch stream."""
    import torch

    stream = torch.cuda.current_stream(plan.device)
    for _ in range(warmup):
        plan.run(stream)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        plan.run(stream)
    end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ev_ms = start.elapsed_time(end) / steps
    return wall_ms, ev_ms


def cpu_baseline(workload_name: str, runs: int = 5):
    """Reference CPU path restatement (oracle/reference_path.py) on the host cores."""
    import torch

    import oracle  # noqa: F401  (checker package; used here only as the timed CPU baseline)
    from oracle import reference_path as ref
    from fields_lm_amd.workloads import make_scan_workload

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    wl = make_scan_workload(workload_name, "cuda")
    raw = wl.raw.float().cpu()
    tr, ti, gamma = wl.tr.cpu(), wl.ti.cpu(), wl.gamma.cpu()
    ref.field_read(raw, tr, ti, gamma, 32)  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        ref.field_read(raw, tr, ti, gamma, 32)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": wl.tokens / med,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{workload_name} (B={raw.shape[0]}, T={raw.shape[1]}, C={wl.channels}) raw upcast to "
                   f"fp32; reference_field_read/hierarchical_scan(block 32) restated op for op in torch "
                   f"complex64; median of {runs} runs after 1 warm-up; {med:.3f} s per run; "
                   f"cpu={platform.processor() or platform.machine()}"),
    }


def decode_timing(batch: int = 64, dim: int = 1024, tokens: int = 256):
    """Fused decode step of one Field block at B=64: per-step device time inside a HIP graph of
    ``tokens`` consecutive steps, and eager single-step latency."""
    import torch

    from fields_lm_amd import field_decode_step
    from fields_lm_amd.workloads import make_scan_workload

    wl = make_scan_workload("scan_b8_t2048_d1024", "cuda", batch=batch, length=tokens)
    raw = wl.raw  # [B, tokens, 3C] bf16
    C = wl.channels
    state = torch.zeros(batch, 2 * C, device="cuda")
    out = torch.empty(tokens, batch, 4 * C, device="cuda")
    steps = [raw[:, t] for t in range(tokens)]
    for t in range(4):
        field_decode_step(steps[t], wl.tr, wl.ti, wl.gamma, state, out=out[t])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for t in range(tokens):
            field_decode_step(steps[t], wl.tr, wl.ti, wl.gamma, state, out=out[t])
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 5
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    graph_us = start.elapsed_time(end) * 1e3 / (reps * tokens)
    lat = []
    for t in range(64):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        field_decode_step(steps[t], wl.tr, wl.ti, wl.gamma, state, out=out[t])
        torch.cuda.synchronize()
        lat.append((time.perf_counter() - t0) * 1e6)
    bytes_step = batch * (3 * C * 2 + 2 * C * 4 * 2 + 4 * C * 4)
    return {
        "batch": batch,
        "graph_us_per_step": graph_us,
        "graph_tokens_per_s": batch / (graph_us * 1e-6),
        "eager_p50_us": statistics.median(lat),
        "bytes_per_step": bytes_step,
        "graph_gbs": bytes_step / (graph_us * 1e-6) / 1e9,
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="scan_b8_t2048_d1024")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy (counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the Field scan shards over batch rows and channels "
              "with no communication, and this build runs on a single MI355X. Use --gpus 1.",
              file=sys.stderr, flush=True)
        return 2

    import torch

    from fields_lm_amd import ScanPlan
    from fields_lm_amd.workloads import make_scan_workload, scan_bytes_per_token

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    log(f"[bench] device={torch.cuda.get_device_name(dev)} workload={args.workload}")
    wl = make_scan_workload(args.workload, dev)
    plan = ScanPlan(wl.raw, wl.tr, wl.ti, wl.gamma)
    wall_ms, ev_ms = time_plan(plan, args.steps, args.warmup)
    bpt = scan_bytes_per_token(wl.channels, wl.raw.dtype)
    alg_bytes = bpt * wl.tokens
    achieved = alg_bytes / (ev_ms * 1e-3) / 1e9
    log(f"[bench] {args.workload}: wall {wall_ms * 1e3:.1f} us/step, events {ev_ms * 1e3:.1f} us/step, "
        f"{achieved:.0f} GB/s")

    result = {
        "metric": METRIC,
        "value": wl.tokens / (wall_ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": args.workload,
            "B": wl.raw.shape[0], "T": wl.raw.shape[1], "d_model": 2 * wl.channels,
            "raw_dtype": "bf16", "read_dtype": "fp32", "state_dtype": "fp32",
            "bytes_per_token": bpt, "parallelism": "single-gpu",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "fl_scan_lookback_kernel (one launch per step)",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(args.workload),
            "algorithmic_bytes": alg_bytes,
            "event_us_per_launch": ev_ms * 1e3,
        },
    }

    if not args.no_extras:
        extras = {}
        del plan
        torch.cuda.empty_cache()
        # fp32 raw on the same shape
        wl32 = make_scan_workload(args.workload, dev, dtype=torch.float32)
        p32 = ScanPlan(wl32.raw, wl32.tr, wl32.ti, wl32.gamma)
        _, e32 = time_plan(p32, 50, 5)
        b32 = scan_bytes_per_token(wl32.channels, torch.float32) * wl32.tokens
        extras["fp32_raw"] = {"us_per_step": e32 * 1e3, "tokens_per_s": wl32.tokens / (e32 * 1e-3),
                              "gbs": b32 / (e32 * 1e-3) / 1e9}
        del p32, wl32
        torch.cuda.empty_cache()
        # config 4: long context
        wll = make_scan_workload("scan_b1_t65536_d1024", dev)
        pl = ScanPlan(wll.raw, wll.tr, wll.ti, wll.gamma)
        _, el = time_plan(pl, 20, 3)
        bl = scan_bytes_per_token(wll.channels, wll.raw.dtype) * wll.tokens
        extras["long_context_b1_t65536"] = {"us_per_step": el * 1e3, "tokens_per_s": wll.tokens / (el * 1e-3),
                                            "gbs": bl / (el * 1e-3) / 1e9,
                                            "frac_hbm_peak": bl / (el * 1e-3) / 1e9 / HBM_PEAK_GBS}
        del pl, wll
        torch.cuda.empty_cache()
        extras["decode_b64_one_block"] = decode_timing()
        result["extras"] = extras

    if not args.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(args.workload)

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
