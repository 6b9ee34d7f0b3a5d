#!/usr/bin/env python3
"""Field scan benchmark on one MI355X (the hot path of Fields LM's native Field block).

A "step" is one ``fl_scan_forward`` over one batch of config 2 (B=8, T=2048, d_model=1024,
C=512): bf16 raw [8,2048,1536] resident in HBM -> fp32 read [8,2048,2048], state carried across
chunks. ``value`` is tokens/s of the whole step; ``roofline`` prices the same launch against
MI355X's 8 TB/s HBM with the algorithmic bytes 3C*2 + 4C*4 = 11,264 B/token; ``cpu_baseline``
times the torch restatement of the reference's CPU path (oracle/reference_path.py) on the
host's cores on the same workload.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--variant V] [--no-cpu-baseline]
                    [--no-extras] [--decode-only] [--copy-ceilings]

``--variant`` picks the timed scan: read_fp32 (the headline: fp32 read, 11,264 B/token),
read_bf16 (7,168 B/token), norm_bf16 / norm_fp32 (read_norm fused into the epilogue).
"""
from __future__ import annotations

import argparse
import ctypes
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
BWD_WAVE_ROWS = 8  # steps per wave of the backward kernel: one stored state read per wave
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


def device_copy_ceiling(scan_bytes: int, scan_gbs: float) -> dict:
    """Measured device-to-device copy rate on this box (torch ``copy_`` of contiguous buffers, HIP
    events over back-to-back copies): one copy moving the scan step's algorithmic bytes (read half,
    write half; the working set fits the 256 MB Infinity Cache, as the scan's does), and one moving
    2 GiB (HBM only). Reported beside the scan's own rate."""
    import torch

    out = {}
    for key, nbytes, reps in (("same_bytes_as_scan_step", scan_bytes, 100), ("two_gib", 2 << 30, 10)):
        n = nbytes // 2 // 4
        x = torch.empty(n, device="cuda").uniform_()
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(reps):
            y.copy_(x)
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) / reps * 1e3
        gbs = 2 * n * 4 / (us * 1e-6) / 1e9
        out[key] = {"bytes_moved": 2 * n * 4, "us_per_copy": us, "gbs": gbs,
                    "scan_fraction_of_copy": scan_gbs / gbs}
        del x, y
        torch.cuda.empty_cache()
    return out


VARIANTS = {  # name -> (ScanPlan keyword arguments, read bytes per element, profile suffix)
    "read_fp32": ({}, 4, ""),
    "read_bf16": ({"read_dtype": "bf16"}, 2, "_read_bf16"),
    "norm_bf16": ({"read_dtype": "bf16", "norm": True}, 2, "_norm_bf16"),
    "norm_fp32": ({"norm": True}, 4, "_norm_fp32"),
}


ALGOS = {"auto": 0, "lookback": 2, "chunked3": 1}  # fl_scan_forward_ex algo codes


def measured_traffic(workload: str, variant: str = "read_fp32"):
    """HBM bytes per launch of the scan from the committed rocprofv3 --pmc summary, or None."""
    path = REPO / "profiles" / f"fl_scan_lookback_kernel_{workload}{VARIANTS[variant][2]}_pmc.txt"
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


INFINITY_CACHE_BYTES = 256 * 2**20
COLD_SET_BYTES = 1 << 30  # rotated buffer sets add up to at least this: 4x the Infinity Cache
PREPARE_LAUNCHES = 100  # untimed launches before the warm-up steps of every timed loop
START_DELAY_US = 200.0  # device time queued ahead of a timed loop's start event


_DELAY_LIB = []


def device_delay(stream, us: float = START_DELAY_US) -> bool:
    """Queues ``us`` microseconds of device time on ``stream`` (``fl_bench_device_delay``: one
    wave sleeping on the wall clock, which always ends); False when the bench library is absent.
    Queued after the synchronize that opens a timed loop and before its start event, it keeps the
    device from reaching the start event while the host is still enqueueing the first timed
    launch. Otherwise that wait (tens of µs after a synchronize) lands inside the events: 20 steps
    of the config-2 scan read ≈ 2 µs per step slower than 200 steps."""
    import ctypes

    if not _DELAY_LIB:
        from fields_lm_amd.build import BENCH_LIB_PATH

        lib = None
        if BENCH_LIB_PATH.exists():
            lib = ctypes.CDLL(str(BENCH_LIB_PATH))
            lib.fl_bench_device_delay.restype = ctypes.c_int
            lib.fl_bench_device_delay.argtypes = [ctypes.c_double, ctypes.c_void_p]
        _DELAY_LIB.append(lib)
    lib = _DELAY_LIB[0]
    if lib is None:
        return False
    rc = lib.fl_bench_device_delay(float(us), ctypes.c_void_p(stream.cuda_stream))
    if rc != 0:
        raise RuntimeError(f"fl_bench_device_delay: error {rc}")
    return True


def time_plan(plans, steps: int, warmup: int):
    """Times ``steps`` launches; returns (wall ms per step, event ms per step).

    ``plans`` is one plan or a list of plans over distinct buffer sets, launched in rotation
    (step i runs plans[i % n]); with sets adding up to more than the 256 MB Infinity Cache,
    every launch finds its inputs in HBM only (cold). The events sit on the launch stream,
    inside the synchronize bracket that the wall clock spans; a device delay (``device_delay``)
    queued ahead of the start event keeps the host's first enqueue out of the events. The wall
    clock includes that delay."""
    import torch

    plans = plans if isinstance(plans, (list, tuple)) else [plans]
    stream = torch.cuda.current_stream(plans[0].device)
    # preparation before the warm-up steps: every buffer set touched and the GPU out of its idle
    # clocks (the first timed loop of a process otherwise runs about 1 us per launch slower)
    for i in range(max(PREPARE_LAUNCHES, 4 * len(plans))):
        plans[i % len(plans)].run(stream)
    torch.cuda.synchronize()
    for i in range(max(warmup, len(plans))):
        plans[i % len(plans)].run(stream)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    device_delay(stream)
    start.record(stream)
    for i in range(steps):
        plans[i % len(plans)].run(stream)
    end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ev_ms = start.elapsed_time(end) / steps
    return wall_ms, ev_ms


def cold_sets(set_bytes: int) -> int:
    """Number of rotated buffer sets for a cold-cache timing: at least 4, and together at least
    1 GiB, so that between two launches on one set more than the Infinity Cache has streamed."""
    return max(4, -(-COLD_SET_BYTES // max(set_bytes, 1)))


def scan_plans(wl, n_sets: int, **kw):
    """``n_sets`` ScanPlans over copies of the workload's raw (each with its own read, state and
    workspace); the first uses the workload's tensor itself."""
    from fields_lm_amd import ScanPlan

    raws = [wl.raw] + [wl.raw.clone() for _ in range(n_sets - 1)]
    return [ScanPlan(r, wl.tr, wl.ti, wl.gamma, **kw) for r in raws]


def plan_set_bytes(plan) -> int:
    return (plan.raw.numel() * plan.raw.element_size() + plan.read.numel() * plan.read.element_size()
            + plan.ws_bytes)


def scan_timing(wl, kw: dict, steps: int, warmup: int) -> dict:
    """One scan variant on a workload, cold (rotated buffer sets) and hot (one set replayed), with
    its algorithmic bytes per token (raw read once, the output written once)."""
    import torch

    plans = scan_plans(wl, 1, **kw)
    n_sets = cold_sets(plan_set_bytes(plans[0]))
    plans += scan_plans(wl, n_sets, **kw)[1:]
    _, cold = time_plan(plans, steps, warmup)
    _, hot = time_plan(plans[0], steps, warmup)
    from fields_lm_amd.workloads import scan_bytes_per_token

    bpt = scan_bytes_per_token(wl.channels, wl.raw.dtype, plans[0].read.element_size())
    nb = bpt * wl.tokens
    del plans
    torch.cuda.empty_cache()
    return {"us_per_step": cold * 1e3, "tokens_per_s": wl.tokens / (cold * 1e-3),
            "bytes_per_token": bpt, "gbs": nb / (cold * 1e-3) / 1e9,
            "frac_hbm_peak": nb / (cold * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "hot_us_per_step": hot * 1e3, "hot_frac_hbm_peak": nb / (hot * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "cache": f"cold: {n_sets} rotated buffer sets; hot: one set replayed"}


class _CopyPlan:
    """One measurement copy (``libfields_bench.so``) over one buffer set, with the ``run(stream)``
    and ``device`` of a ScanPlan so that :func:`time_plan` times it the same way."""

    def __init__(self, lib, kind: str, raw, out, out_elem_bytes: int):
        self.lib, self.kind, self.raw, self.out, self.osz = lib, kind, raw, out, out_elem_bytes
        self.device = raw.device

    def run(self, stream=None):
        import ctypes

        import torch

        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        h = ctypes.c_void_p(s.cuda_stream)
        B, T, C3 = self.raw.shape
        if self.kind == "tile":
            rc = self.lib.fl_bench_tile_copy(ctypes.c_void_p(self.raw.data_ptr()),
                                             ctypes.c_void_p(self.out.data_ptr()), B, T, C3 // 3,
                                             self.osz, h)
        else:
            rc = self.lib.fl_bench_stream_copy(ctypes.c_void_p(self.raw.data_ptr()),
                                               ctypes.c_void_p(self.out.data_ptr()),
                                               self.raw.numel() * self.raw.element_size(),
                                               self.out.numel(), h)
        if rc != 0:
            raise RuntimeError(f"copy kernel {self.kind}: error {rc}")


def copy_ceilings(wl, scan_us: dict, steps: int = 100, warmup: int = 10) -> dict:
    """Cold copy ceilings of the scan's byte mix on this box, beside the scan's own cold time:
    ``fl_bench_tile_copy`` (the scan's access pattern, tiles, grid, occupancy and tile order,
    without its arithmetic or look-back) and ``fl_bench_stream_copy`` (a streaming copy of the
    same bytes), for the fp32 and the bf16 read; buffer sets rotated as for the scan."""
    import ctypes

    import torch

    from fields_lm_amd.build import BENCH_LIB_PATH

    if not BENCH_LIB_PATH.exists():
        return {"skipped": f"{BENCH_LIB_PATH.name} not built (python -m fields_lm_amd.build)"}
    lib = ctypes.CDLL(str(BENCH_LIB_PATH))
    lib.fl_bench_tile_copy.restype = ctypes.c_int
    lib.fl_bench_tile_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 3 + \
        [ctypes.c_int, ctypes.c_void_p]
    lib.fl_bench_stream_copy.restype = ctypes.c_int
    lib.fl_bench_stream_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                         ctypes.c_size_t, ctypes.c_void_p]
    B, T, C3 = wl.raw.shape
    C = C3 // 3
    if T % 128 or C % 64 or wl.raw.element_size() != 2:
        return {"skipped": "the tile pattern needs bf16 raw, T % 128 == 0 and C % 64 == 0"}
    out = {}
    for key, osz in (("fp32_read", 4), ("bf16_read", 2)):
        raw_bytes = wl.raw.numel() * wl.raw.element_size()
        out_bytes = B * T * 4 * C * osz
        n_sets = cold_sets(raw_bytes + out_bytes)
        raws = [wl.raw] + [wl.raw.clone() for _ in range(n_sets - 1)]
        outs = [torch.empty(out_bytes, device=wl.raw.device, dtype=torch.uint8) for _ in range(n_sets)]
        res = {"bytes": raw_bytes + out_bytes, "scan_us": scan_us[key]}
        for kind in ("tile", "stream"):
            plans = [_CopyPlan(lib, kind, r, o, osz) for r, o in zip(raws, outs)]
            _, ms = time_plan(plans, steps, warmup)
            name = "tile_pattern" if kind == "tile" else "streaming"
            res[f"{name}_us"] = ms * 1e3
            res[f"{name}_frac_hbm_peak"] = (raw_bytes + out_bytes) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS
            if scan_us[key] is not None:
                res[f"scan_over_{name}"] = scan_us[key] / (ms * 1e3)
        out[key] = res
        del raws, outs
        torch.cuda.empty_cache()
    out["note"] = ("cold, HIP events; the scan's time over a copy of its own access pattern "
                   "(scan_over_tile_pattern) and over a streaming copy of the same bytes")
    return out


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def dtype_name(dtype) -> str:
    import torch

    return {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp16"}.get(dtype, str(dtype))


def cpu_baseline(workload_name: str, min_runs: int = 5, budget_s: float = 10.0, max_runs: int = 400):
    """Reference CPU path restatement (oracle/reference_path.py) on the host cores: whole passes
    over the workload, repeated until ``budget_s`` seconds of CPU work (at least ``min_runs``,
    at most ``max_runs`` passes); the median pass time gives tokens/s."""
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
    while len(times) < max_runs and (len(times) < min_runs or sum(times) < budget_s):
        t0 = time.perf_counter()
        ref.field_read(raw, tr, ti, gamma, 32)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    runs = len(times)
    return {
        "value": wl.tokens / med,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{workload_name} (B={raw.shape[0]}, T={raw.shape[1]}, C={wl.channels}) raw upcast to "
                   f"fp32; reference_field_read/hierarchical_scan(block 32) restated op for op in torch "
                   f"complex64; median of {runs} passes ({sum(times):.1f} s of CPU work) after 1 "
                   f"warm-up; {med:.3f} s per pass"),
        "cpu_model": cpu_model(),
    }


def _graph_us_per_call(fn_list, reps: int = 5) -> float:
    """Capture the calls of ``fn_list`` in one HIP graph; device time per call over ``reps`` replays."""
    import torch

    for fn in fn_list[:2]:
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for fn in fn_list:
            fn()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    device_delay(torch.cuda.current_stream())  # the first replay's launch stays out of the events
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / (reps * len(fn_list))


def _eager_p50_us(fn, n: int = 64) -> float:
    import torch

    lat = []
    for _ in range(n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        lat.append((time.perf_counter() - t0) * 1e6)
    return statistics.median(lat)


def _torch_step(raw_t, lam, gamma, s):
    """Stock-PyTorch eager single-token Field step (complex64), the comparator for the fused
    kernel: the gates and update of the reference's recurrence for one token."""
    import torch

    c = lam.numel()
    zr, zi, zv = raw_t.float().split(c, dim=-1)
    inj = torch.complex(torch.tanh(zr), torch.tanh(zi))
    v = 0.9 * torch.sigmoid(zv)
    m = lam * s
    disp = v * m
    s_new = (1.0 - v) * m + gamma * v * inj
    return torch.cat([s_new.real, s_new.imag, disp.real, disp.imag], -1), s_new


def decode_comparison(batch: int = 64, dim: int = 1024, prompt: int = 2048, tokens: int = 256):
    """Decode at B=64 (config 5's per-token Field work), one Field block:

    * kernel: fl_decode_norm_step (state update + displaced readout + read_norm, one launch)
      and fl_decode_step, per step inside a HIP graph of ``tokens`` consecutive steps;
    * block_step: the whole FieldBlock.step (projections, fused step, gate, SwiGLU), bf16
      weights, per token inside a HIP graph of 32 tokens, and eager p50;
    * reference procedure: the reference has no incremental state, so token t's Field output
      needs the block re-run over the whole prefix (length prompt + t >= prompt): timed as one
      FieldBlock.forward over [B, prompt] with this package's kernels (a lower bound of the
      reference's per-token cost);
    * torch_eager_step: a stock-PyTorch eager single-token step (complex64 ops), p50.
    """
    import torch

    from fields_lm_amd import FieldBlock, field_decode_norm_step, field_decode_step
    from fields_lm_amd.workloads import make_scan_workload

    dev = torch.device("cuda:0")
    wl = make_scan_workload("scan_b8_t2048_d1024", dev, batch=batch, length=tokens)
    raw = wl.raw  # [B, tokens, 3C] bf16
    C = wl.channels
    w = torch.ones(4 * C, device=dev)
    state = torch.zeros(batch, 2 * C, device=dev)
    out32 = torch.empty(tokens, batch, 4 * C, device=dev)
    out16 = torch.empty(tokens, batch, 4 * C, device=dev, dtype=torch.bfloat16)
    steps = [raw[:, t] for t in range(tokens)]
    plain_us = _graph_us_per_call(
        [lambda t=t: field_decode_step(steps[t], wl.tr, wl.ti, wl.gamma, state, out=out32[t])
         for t in range(tokens)])
    norm_us = _graph_us_per_call(
        [lambda t=t: field_decode_norm_step(steps[t], wl.tr, wl.ti, wl.gamma, state, w,
                                            out=out16[t], out_dtype=torch.bfloat16)
         for t in range(tokens)])
    kernel_p50 = _eager_p50_us(lambda: field_decode_norm_step(steps[0], wl.tr, wl.ti, wl.gamma, state, w,
                                                              out=out16[0], out_dtype=torch.bfloat16))
    lam = torch.complex(wl.tr, wl.ti)
    s_c = torch.zeros(batch, C, device=dev, dtype=torch.complex64)
    torch_p50 = _eager_p50_us(lambda: _torch_step(steps[0], lam, wl.gamma, s_c))
    del out32, out16

    torch.manual_seed(5)
    block = FieldBlock(dim, "triton", 32, 32, 64, 2752).to(device=dev, dtype=torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(batch, prompt, dim, device=dev, dtype=torch.bfloat16, generator=g)
    xt = torch.randn(32, batch, dim, device=dev, dtype=torch.bfloat16, generator=g)
    with torch.no_grad():
        _, bstate = block.prefill(x)
        params = block.mixer.transition()
        block_us = _graph_us_per_call([lambda t=t: block.step(xt[t], bstate, params) for t in range(32)])
        block_p50 = _eager_p50_us(lambda: block.step(xt[0], bstate, params), n=32)
        reforward = []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            block(x)
            torch.cuda.synchronize()
            reforward.append((time.perf_counter() - t0) * 1e6)
    ref_us = statistics.median(reforward)
    del x, block
    torch.cuda.empty_cache()
    bytes_step = batch * (3 * C * 2 + 2 * C * 4 * 2 + 4 * C * 2)
    return {
        "batch": batch,
        "kernel_norm_graph_us_per_step": norm_us,
        "kernel_norm_eager_p50_us": kernel_p50,
        "kernel_norm_bytes_per_step": bytes_step,
        "kernel_norm_graph_gbs": bytes_step / (norm_us * 1e-6) / 1e9,
        "kernel_plain_graph_us_per_step": plain_us,
        "block_step_graph_us_per_token": block_us,
        "block_step_graph_tokens_per_s": batch / (block_us * 1e-6),
        "block_step_eager_p50_us": block_p50,
        "reference_procedure_prefix_reforward_us": ref_us,
        "reference_procedure_prefix": prompt,
        "torch_eager_step_p50_us": torch_p50,
        "speedup_block_step_vs_reference_procedure": ref_us / block_us,
        "note": "block: FieldBlock(1024, ff_hidden 2752) bf16 weights, random init seed 5; "
                "reference procedure = full-prefix re-forward per token (prefix >= 2048), run "
                "with this package's kernels, so it is a lower bound of the reference's cost",
    }


def backward_timing(workload: str, steps: int = 50, warmup: int = 5, cold_only: bool = False):
    """fl_scan_backward on a workload (bf16 raw and bf16 grad_raw, fp32 read / grad_read):
    algorithmic bytes per token 3C*2 (raw) + 4C*4 (grad_read) + 3C*2 (grad_raw) + 2C*4/8 (the
    read's state at the row before each 8-step wave, from which the kernel recomputes s_{t-1})
    = 14,848 at C = 512."""
    import torch

    from fields_lm_amd import _native as nat
    from fields_lm_amd import field_scan
    from fields_lm_amd.workloads import make_scan_workload

    dev = torch.device("cuda:0")
    wl = make_scan_workload(workload, dev)
    B, T, C = wl.raw.shape[0], wl.raw.shape[1], wl.channels
    lib = nat.load()
    n = int(lib.fl_scan_backward_workspace_bytes(B, T, C))
    stream = torch.cuda.current_stream(dev)
    gen = torch.Generator(device=dev).manual_seed(4)

    class _Plan:
        device = dev

        def __init__(self, raw):
            self.raw = raw
            self.read = field_scan(raw, wl.tr, wl.ti, wl.gamma)
            self.gread = torch.randn(self.read.shape, device=dev, generator=gen)
            self.grad_raw = torch.empty(B, T, 3 * C, device=dev, dtype=torch.bfloat16)
            self.gp = [torch.empty(C, device=dev) for _ in range(3)]
            self.ws = torch.zeros(n, device=dev, dtype=torch.uint8)
            self.args = (nat.ptr(raw), nat.FL_DTYPE_BF16, B, T, C, raw.stride(0), raw.stride(1),
                         nat.ptr(wl.tr), nat.ptr(wl.ti), nat.ptr(wl.gamma), None, nat.ptr(self.read),
                         nat.ptr(self.gread), None, nat.ptr(self.grad_raw), nat.FL_DTYPE_BF16,
                         *[nat.ptr(x) for x in self.gp], None, nat.ptr(self.ws), n,
                         ctypes.c_void_p(stream.cuda_stream))

        def run(self, s=None):
            nat.check(lib.fl_scan_backward(*self.args), "fl_scan_backward")

        def nbytes(self):
            return sum(t.numel() * t.element_size() for t in (self.raw, self.read, self.gread,
                                                              self.grad_raw, self.ws))

    plans = [_Plan(wl.raw)]
    n_sets = cold_sets(plans[0].nbytes())
    plans += [_Plan(wl.raw.clone()) for _ in range(n_sets - 1)]
    _, ev = time_plan(plans, steps, warmup)
    hot = float("nan") if cold_only else time_plan(plans[0], steps, warmup)[1]
    nbytes = (3 * C * 2 + 4 * C * 4 + 3 * C * 2 + 2 * C * 4 // BWD_WAVE_ROWS) * B * T
    if any(nat.workspace_error(p.ws) != 0 for p in plans):
        raise RuntimeError("backward look-back wait gave up")
    del plans
    torch.cuda.empty_cache()
    return {"workload": workload, "us_per_step": ev * 1e3, "tokens_per_s": B * T / (ev * 1e-3),
            "bytes_per_token": nbytes // (B * T), "gbs": nbytes / (ev * 1e-3) / 1e9,
            "frac_hbm_peak": nbytes / (ev * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "hot_us_per_step": hot * 1e3, "hot_frac_hbm_peak": nbytes / (hot * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "cache": f"cold: {n_sets} rotated buffer sets; hot: one set replayed",
            "note": "two launches: the reverse scan, then the parameter-gradient reduction"}


def _promoted_model(dev):
    from fields_lm_amd.model import build_official_fields, cast_for_inference

    lm = build_official_fields(device=dev)
    return lm, cast_for_inference(lm.core_model).eval()


def model_prefill(batch: int = 4, length: int = 2048, steps: int = 10, warmup: int = 3):
    """Config 3: the promoted 18F/2M/4R model (random init, bf16 weights under bf16 autocast)
    prefilling B=4 x T=2048 uniform tokens (seed 2), logits of the last position as in v32:461-490;
    whole-model tokens/s, plus per-category device time from events around every block (the
    breakdown of v32:508-556) and the Field scan kernels' share from their own launch count."""
    import torch

    from fields_lm_amd.model import _kind

    dev = torch.device("cuda:0")
    lm, core = _promoted_model(dev)
    torch.manual_seed(2)
    tokens = torch.randint(0, 16384, (batch, length)).to(dev)
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        for _ in range(warmup):
            core.states_logits(tokens, last_only=True)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for _ in range(steps):
            core.states_logits(tokens, last_only=True)
        end.record()
        torch.cuda.synchronize()
        wall_ms = (time.perf_counter() - t0) * 1e3 / steps
        ev_ms = start.elapsed_time(end) / steps
        cats = {k: 0.0 for k in ("embedding", "field_blocks", "mamba_blocks", "refresh_blocks",
                                 "softpatch", "final_norm_head")}
        reps = 3
        for _ in range(reps):
            events = []

            def rec(cat, fn):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                out = fn()
                b.record()
                events.append((cat, a, b))
                return out

            h = rec("embedding", lambda: core.emb(tokens))
            for i, block in enumerate(core.blocks):
                cat = {"field": "field_blocks", "mamba": "mamba_blocks", "refresh": "refresh_blocks"}[_kind(block)]
                h = rec(cat, lambda blk=block, z=h: blk(z))
                if i == core.patch_position:
                    h = rec("softpatch", lambda z=h: core.softpatch(z, tokens))
            rec("final_norm_head", lambda z=h: core.lm_head(core.final_norm(z)[:, -1:]))
            torch.cuda.synchronize()
            for cat, a, b in events:
                cats[cat] += a.elapsed_time(b) / reps
        # the Field scan kernel alone, one launch per Field block, on a block's real raw
        fb = next(b for b in core.blocks if _kind(b) == "field")
        raw = fb.mixer.write_proj(core.emb(tokens))
        tr, ti, gamma = fb.mixer.transition()
        from fields_lm_amd import ScanPlan

        plan = ScanPlan(raw.contiguous(), tr, ti, gamma, read_dtype=torch.bfloat16,
                        norm_weight=fb.mixer.read_norm.weight.float())
        _, scan_ms = time_plan(plan, 50, 5)
    total = sum(cats.values())
    n_field = sum(1 for b in core.blocks if _kind(b) == "field")
    return {
        "batch": batch, "length": length, "tokens_per_s": batch * length / (wall_ms * 1e-3),
        "ms_per_prefill": wall_ms, "event_ms_per_prefill": ev_ms,
        "category_ms": cats, "category_pct": {k: 100.0 * v / max(total, 1e-9) for k, v in cats.items()},
        "field_scan_kernel_ms": scan_ms * n_field,
        "field_scan_kernel_pct": 100.0 * scan_ms * n_field / ev_ms,
        "params": sum(p.numel() for p in core.parameters()),
        "ff_hidden": lm.source_audit["ff_hidden"],
        "note": "random init (model seed 1234), bf16 weights + bf16 autocast; Field blocks run "
                "read_norm fused into the scan (fl_scan_norm_forward, bf16 out); refresh "
                "attention, Mamba-2 (PyTorch SSD), projections are stock PyTorch",
    }


def model_decode(batch: int = 64, prompt: int = 2048, new_tokens: int = 256):
    """Config 5: B=64 streams, a 2,048-token uniform prompt (seed 5), then 256 greedy tokens.
    Token 1 runs eagerly (warm-up); one decode step plus its argmax feedback is captured in a HIP
    graph and replayed for every further token, so the loop issues no host work per token."""
    import torch

    dev = torch.device("cuda:0")
    lm, core = _promoted_model(dev)
    torch.manual_seed(5)
    tokens = torch.randint(0, 16384, (batch, prompt)).to(dev)
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        core.states_logits(tokens[:, :256], last_only=True)  # warm-up of the prefill kernels
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits, cache = core.prefill(tokens, max_len=prompt + new_tokens)
        torch.cuda.synchronize()
        prefill_ms = (time.perf_counter() - t0) * 1e3
        tok = logits.argmax(-1)
        logits = core.step(tok, cache)  # token 1, eager
        tok.copy_(logits.argmax(-1))
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = core.step(tok, cache)
            tok.copy_(out.argmax(-1))
        # tokens 2..new_tokens: one replay each (positions stay below max_len); an event pair
        # around every replay gives the per-token device latency
        marks = [torch.cuda.Event(enable_timing=True) for _ in range(new_tokens)]
        torch.cuda.synchronize()
        marks[0].record()
        for i in range(1, new_tokens):
            graph.replay()
            marks[i].record()
        torch.cuda.synchronize()
        loop_ms = marks[0].elapsed_time(marks[-1])
        lat = [marks[i - 1].elapsed_time(marks[i]) * 1e3 for i in range(1, new_tokens)]
        end_pos = int(cache["pos"])
    if end_pos != prompt + new_tokens:
        raise RuntimeError(f"decode ended at position {end_pos}, expected {prompt + new_tokens}")
    per_token_ms = loop_ms / (new_tokens - 1)
    return {
        "batch": batch, "prompt": prompt, "new_tokens": new_tokens,
        "prefill_ms": prefill_ms,
        "graph_ms_per_token": per_token_ms,
        "tokens_per_s": batch / (per_token_ms * 1e-3),
        "p50_token_latency_us": statistics.median(lat),
        "p90_token_latency_us": sorted(lat)[int(0.9 * (len(lat) - 1))],
        "reference_procedure_ms_per_token": prefill_ms,
        "note": "reference procedure = re-running the whole model over the prefix for each new "
                "token (no incremental state), at least the 2,048-token prefill measured here",
    }


def cpu_backward(workload_name: str, runs: int = 3):
    """The reference CPU path's backward: torch autograd through the op-for-op restatement of
    reference_field_read (complex64, block 32) on the host cores, same workload, fp32 raw."""
    import torch

    import oracle  # noqa: F401  (checker package; timed CPU baseline only)
    from oracle import reference_path as ref
    from fields_lm_amd.workloads import make_scan_workload

    wl = make_scan_workload(workload_name, "cuda")
    raw = wl.raw.float().cpu().requires_grad_()
    tr, ti, gamma = (t.cpu().requires_grad_() for t in (wl.tr, wl.ti, wl.gamma))
    gread = torch.randn(raw.shape[0], raw.shape[1], 4 * wl.channels)
    times = []
    for i in range(runs + 1):
        read = ref.field_read(raw, tr, ti, gamma, 32)
        t0 = time.perf_counter()
        read.backward(gread)
        if i:
            times.append(time.perf_counter() - t0)
        raw.grad = None
    med = statistics.median(times)
    return {"value": wl.tokens / med, "unit": "tokens/s", "s_per_backward": med,
            "cores": len(os.sched_getaffinity(0)), "kind": "port",
            "sample": f"{workload_name}: autograd backward of the restated reference CPU path, median of {runs}"}


def cpu_decode_reforward(runs: int = 3):
    """Reference CPU path per-token cost of decode: one full-prefix re-forward of the Field block
    (oracle/reference_path.py, the reference's CPU path restated) at B=1, T=2048, fp32."""
    import torch

    import oracle  # noqa: F401  (checker package; timed CPU baseline only)
    from oracle import reference_path as ref
    from fields_lm_amd import FieldBlock

    torch.manual_seed(0)
    block = FieldBlock(1024, "triton", 32, 32, 64, 2752)
    sd = {k: v.detach() for k, v in block.state_dict().items()}
    x = torch.randn(1, 2048, 1024)
    with torch.no_grad():
        ref.block_forward(sd, x, field_chunk=32)
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            ref.block_forward(sd, x, field_chunk=32)
            times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"us_per_token_b1": med * 1e6, "batch": 1, "prefix": 2048, "dtype": "fp32",
            "config1_block_tokens_per_s": 2048 / med,
            "cores": len(os.sched_getaffinity(0)),
            "sample": f"FieldBlock(1024, ff_hidden 2752) seed 0, x ~ N(0,1) [1,2048,1024]; "
                      f"median of {runs} after 1 warm-up; at B=64 the re-forward is ~64x this"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="scan_b8_t2048_d1024")
    ap.add_argument("--variant", default="read_fp32", choices=list(VARIANTS))
    ap.add_argument("--algo", default="auto", choices=list(ALGOS),
                    help="scan algorithm of the timed step (auto: the library's default)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the B=64 decode comparison (kernel and block step in HIP graphs)")
    ap.add_argument("--backward-only", action="store_true",
                    help="only the backward scan (fl_scan_backward) on --workload")
    ap.add_argument("--model", choices=["prefill", "decode"],
                    help="only the whole-model run: prefill (config 3) or decode (config 5)")
    ap.add_argument("--cold-only", action="store_true",
                    help="time the headline scan cold only (no hot-cache replay): every launch of the "
                         "process then reads cold buffers, so a kernel trace's average is the cold time")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--copy-ceilings", action="store_true",
                    help="only time the copy kernels of the scan's access pattern (cold)")
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
    if args.decode_only:
        print(json.dumps({"decode_b64": decode_comparison()}), flush=True)
        return 0
    if args.copy_ceilings:
        wl = make_scan_workload(args.workload, dev)
        print(json.dumps({"copy_ceilings": copy_ceilings(wl, {"fp32_read": None, "bf16_read": None},
                                                         steps=args.steps, warmup=args.warmup)}),
              flush=True)
        return 0
    if args.backward_only:
        print(json.dumps({"backward": backward_timing(args.workload, steps=args.steps, warmup=args.warmup,
                                                      cold_only=args.cold_only)}), flush=True)
        return 0
    if args.model:
        fn = model_prefill if args.model == "prefill" else model_decode
        print(json.dumps({f"model_{args.model}": fn()}), flush=True)
        return 0
    log(f"[bench] device={torch.cuda.get_device_name(dev)} workload={args.workload} variant={args.variant}")
    wl = make_scan_workload(args.workload, dev)
    vkw, read_bytes, _ = VARIANTS[args.variant]
    kw = {}
    if vkw.get("read_dtype") == "bf16":
        kw["read_dtype"] = torch.bfloat16
    if vkw.get("norm"):
        kw["norm_weight"] = torch.ones(4 * wl.channels, device=dev)  # read_norm's init weight
    if not vkw.get("norm"):
        kw["algo"] = ALGOS[args.algo]
    # cold: rotated buffer sets, every launch reads its raw from HBM (the headline); hot: one
    # buffer set replayed, its working set resident in the Infinity Cache (reported beside)
    probe = ScanPlan(wl.raw, wl.tr, wl.ti, wl.gamma, **kw)
    n_sets = cold_sets(plan_set_bytes(probe))
    del probe
    plans = scan_plans(wl, n_sets, **kw)
    wall_ms, ev_ms = time_plan(plans, args.steps, args.warmup)
    hot_ev_ms = None if args.cold_only else time_plan(plans[0], args.steps, args.warmup)[1]
    out_dtype = plans[0].read.dtype
    bpt = scan_bytes_per_token(wl.channels, wl.raw.dtype, out_dtype.itemsize)
    alg_bytes = bpt * wl.tokens
    achieved = alg_bytes / (ev_ms * 1e-3) / 1e9
    log(f"[bench] {args.workload}: cold {ev_ms * 1e3:.1f} us/step (wall {wall_ms * 1e3:.1f}), "
        f"{achieved:.0f} GB/s; hot {hot_ev_ms * 1e3 if hot_ev_ms else float('nan'):.1f} us/step")

    result = {
        "metric": METRIC,
        "value": wl.tokens / (ev_ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ev_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype_name(torch.float32),  # the recurrence's state and arithmetic
        "data": "synthetic",
        "config": {
            "workload": args.workload, "variant": args.variant, "algo": args.algo,
            "B": wl.raw.shape[0], "T": wl.raw.shape[1], "d_model": 2 * wl.channels,
            "raw_dtype": dtype_name(wl.raw.dtype), "read_dtype": dtype_name(out_dtype),
            "state_dtype": dtype_name(plans[0].state_out.dtype), "read_norm_fused": bool(vkw.get("norm")),
            "bytes_per_token": bpt, "parallelism": "single-gpu",
            "cache": f"cold: {n_sets} rotated buffer sets of {plan_set_bytes(plans[0]) / 1e6:.0f} MB",
            "clock": "HIP events on the launch stream around the timed steps (value, ms_per_step, "
                     "achieved); wall_ms_per_step is the host clock around the same steps, "
                     f"including a {START_DELAY_US:.0f} us device delay queued ahead of the start "
                     "event so that the host's first enqueue stays out of the events",
            "start_delay": "queued" if _DELAY_LIB and _DELAY_LIB[0] is not None else "bench library absent",
            "wall_ms_per_step": wall_ms,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "fl_scan_lookback_kernel (one launch per step)",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(args.workload, args.variant),
            "algorithmic_bytes": alg_bytes,
            "event_us_per_launch": ev_ms * 1e3,
        },
    }
    if hot_ev_ms is not None:
        result["roofline"]["hot_cache"] = {
            "event_us_per_launch": hot_ev_ms * 1e3,
            "achieved": alg_bytes / (hot_ev_ms * 1e-3) / 1e9,
            "frac": alg_bytes / (hot_ev_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "note": "one buffer set replayed: its working set stays in the 256 MB Infinity Cache "
                    "between launches"}

    if not args.no_extras:
        extras = {}
        del plans
        torch.cuda.empty_cache()
        extras["device_copy"] = device_copy_ceiling(alg_bytes, achieved)
        # fp32 raw on the same shape
        wl32 = make_scan_workload(args.workload, dev, dtype=torch.float32)
        extras["fp32_raw"] = scan_timing(wl32, {}, 50, 5)
        del wl32
        torch.cuda.empty_cache()
        # config 4: long context
        wll = make_scan_workload("scan_b1_t65536_d1024", dev)
        extras["long_context_b1_t65536"] = scan_timing(wll, {}, 20, 3)
        del wll
        torch.cuda.empty_cache()
        # bf16 read, fused read_norm (bf16 / fp32 out), and the unfused sequence it replaces
        wl = make_scan_workload(args.workload, dev)
        C = wl.channels
        w = torch.ones(4 * C, device=dev)
        for key, kw in [("bf16_read", dict(read_dtype=torch.bfloat16)),
                        ("fused_read_norm_bf16_out", dict(read_dtype=torch.bfloat16, norm_weight=w)),
                        ("fused_read_norm_fp32_out", dict(norm_weight=w))]:
            extras[key] = scan_timing(wl, kw, 100, 10)
        extras["copy_ceilings"] = copy_ceilings(
            wl, {"fp32_read": ev_ms * 1e3 if args.variant == "read_fp32" else None,
                 "bf16_read": extras["bf16_read"]["us_per_step"]})
        wll = make_scan_workload("scan_b1_t65536_d1024", dev)
        extras["long_context_fused_read_norm_bf16_out"] = scan_timing(
            wll, dict(read_dtype=torch.bfloat16, norm_weight=torch.ones(4 * wll.channels, device=dev)), 20, 3)
        del wll
        torch.cuda.empty_cache()
        from fields_lm_amd import RMSNorm

        norm = RMSNorm(4 * C).to(dev)
        pp = ScanPlan(wl.raw, wl.tr, wl.ti, wl.gamma)  # hot cache, as the fused variants' hot figure

        class _Unfused:
            device = dev

            def run(self, stream=None):
                pp.run(stream)
                with torch.no_grad():
                    return norm(pp.read).to(torch.bfloat16)

        _, e = time_plan(_Unfused(), 50, 5)
        extras["unfused_scan_rmsnorm_cast"] = {"us_per_step": e * 1e3,
                                               "note": "fp32 read, then RMSNorm module, then bf16 cast"}
        del pp, wl, norm
        torch.cuda.empty_cache()
        extras["backward_b8_t2048"] = backward_timing("scan_b8_t2048_d1024")
        extras["backward_b1_t65536"] = backward_timing("scan_b1_t65536_d1024", steps=20, warmup=3)
        torch.cuda.empty_cache()
        extras["decode_b64"] = decode_comparison()
        torch.cuda.empty_cache()
        log("[bench] model prefill (config 3) ...")
        extras["model_prefill_b4_t2048"] = model_prefill()
        torch.cuda.empty_cache()
        log("[bench] model decode (config 5) ...")
        extras["model_decode_b64"] = model_decode()
        result["extras"] = extras

    if not args.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(args.workload)
        if not args.no_extras:
            log("[bench] cpu decode re-forward ...")
            result["cpu_baseline"]["decode_reforward"] = cpu_decode_reforward()
            log("[bench] cpu backward ...")
            result["cpu_baseline"]["backward"] = cpu_backward(args.workload)
            log("[bench] cpu baseline, config 4 ...")
            long_ctx = cpu_baseline("scan_b1_t65536_d1024", min_runs=3, budget_s=5.0)
            result["cpu_baseline"]["long_context_b1_t65536"] = {
                k: long_ctx[k] for k in ("value", "unit", "cores", "kind", "sample")}

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
