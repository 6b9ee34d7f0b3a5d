"""GPU: the block-order launches under contention.

Launches whose chains hold at most 64 chunks (every config-2 and config-3 scan) take ticket i in
block i with no atomic, which relies on the dispatcher issuing each XCD's blocks of a grid in
index order: then the lowest unfinished tile of a chain (or RMSNorm sibling group) is always
resident, since every block resident ahead of it on its XCD has a lower index
(fields_lm_amd/csrc/field_scan.hip, launch_lookback). The reference's serial carry
(src/fields_official/reference/field_only_v4_chunked_triton_wiki100.py:520-550, a launch of its
own) needs no such assumption.

Here another stream holds part of the chip while the scans run: ``fl_bench_occupy`` (the bench
library's measurement kernels) queues blocks of 1024 threads that each keep 112 KB of LDS, so no
scan block fits beside one on its CU, sleeping a bounded time on the wall clock. The default
config-2 scan (fp32 read), its bf16 read and the RMSNorm epilogue then run on the remaining CUs,
with the holders finishing in the middle of the scan or after it. Every output must equal the
uncontended call's bit for bit and every workspace's error word must stay 0; a wait that gave up
would have turned a dispatch out of order into NaN and a set error bit (never a hang: waits are
bounded). The test stops at the first failure.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from fields_lm_amd import _native

    _native.load()
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def bench_lib(dev):
    from fields_lm_amd.build import BENCH_LIB_PATH

    if not BENCH_LIB_PATH.exists():
        pytest.fail(f"{BENCH_LIB_PATH.name} not built (python -m fields_lm_amd.build)")
    lib = ctypes.CDLL(str(BENCH_LIB_PATH))
    lib.fl_bench_occupy.restype = ctypes.c_int
    lib.fl_bench_occupy.argtypes = [ctypes.c_int, ctypes.c_double, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def test_block_order_launches_under_contention(dev, bench_lib):
    from fields_lm_amd import ScanPlan
    from fields_lm_amd import _native as nat
    from fields_lm_amd.workloads import make_scan_workload

    wl = make_scan_workload("scan_b8_t2048_d1024", dev)
    w = 1.0 + 0.25 * torch.randn(4 * wl.channels, generator=torch.Generator().manual_seed(4)).to(dev)
    plans = {
        "fp32 read": ScanPlan(wl.raw, wl.tr, wl.ti, wl.gamma),
        "bf16 read": ScanPlan(wl.raw, wl.tr, wl.ti, wl.gamma, read_dtype=torch.bfloat16),
        "rmsnorm bf16": ScanPlan(wl.raw, wl.tr, wl.ti, wl.gamma, read_dtype=torch.bfloat16, norm_weight=w),
    }
    ref = {}
    for name, plan in plans.items():
        plan.run()
        torch.cuda.synchronize()
        ref[name] = (plan.read.clone(), plan.state_out.clone())
    sink = torch.zeros(1024, device=dev)
    side = torch.cuda.Stream(dev)
    main = torch.cuda.current_stream(dev)
    # (holding blocks, microseconds): a quarter to all but a few CUs, released during or after
    # the scan (a config-2 scan takes ~40 us)
    for blocks, us in [(64, 20.0), (128, 30.0), (192, 60.0), (240, 15.0), (250, 200.0)]:
        for name, plan in plans.items():
            print(f"[case] contention {name}: {blocks} holding blocks for {us} us", flush=True)
            plan.read.fill_(float("nan"))
            main.synchronize()
            side.wait_stream(main)
            assert bench_lib.fl_bench_occupy(blocks, us, ctypes.c_void_p(sink.data_ptr()),
                                             ctypes.c_void_p(side.cuda_stream)) == 0
            plan.run(main)
            torch.cuda.synchronize()
            assert nat.workspace_error(plan.workspace) == 0, (name, blocks, us)
            assert torch.equal(plan.read, ref[name][0]), (name, blocks, us)
            assert torch.equal(plan.state_out, ref[name][1]), (name, blocks, us)
