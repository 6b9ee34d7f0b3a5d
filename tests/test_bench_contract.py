"""bench.py's output contract: one JSON line whose headline figures follow from each other.

CPU: a request for more than one GPU is refused with a message (exit 2) before anything touches a
GPU, and a host without a ROCm device gets a message and exit 1.
GPU: a short run of the default workload (config 2: B=8, T=2048, C=512, bf16 raw, fp32 read; no
extras, no CPU baseline). Its last stdout line is one JSON object with the contract's keys, where
value = tokens / ms_per_step, roofline.achieved = algorithmic bytes / ms_per_step, frac =
achieved / peak, and the algorithmic bytes are config 2's 3C*2 + 4C*4 = 11,264 B per token.
"""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]


def _bench(args, timeout):
    return subprocess.run([sys.executable, str(REPO / "bench.py"), *args], capture_output=True,
                          text=True, timeout=timeout, cwd=REPO)


def test_more_than_one_gpu_is_refused():
    p = _bench(["--gpus", "2"], 120)
    assert p.returncode == 2
    assert "one GPU only" in p.stderr


def test_no_rocm_device_is_reported():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a ROCm device is present")
    p = _bench(["--steps", "1", "--warmup", "1"], 120)
    assert p.returncode == 1
    assert "needs a ROCm GPU" in p.stderr


@pytest.mark.gpu
def test_headline_line_follows_the_contract():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    print("[case] bench.py --steps 10 --warmup 2 --no-extras --no-cpu-baseline", flush=True)
    p = _bench(["--steps", "10", "--warmup", "2", "--no-extras", "--no-cpu-baseline"], 110)
    assert p.returncode == 0, p.stderr[-2000:]
    r = json.loads(p.stdout.strip().splitlines()[-1])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config", "roofline"):
        assert key in r, key
    assert (r["n_gpus"], r["steps"], r["warmup"]) == (1, 10, 2)
    assert r["unit"] == "tokens/s" and r["higher_is_better"] is True and r["data"] == "synthetic"
    assert r["dtype"] == "fp32" and r["config"]["workload"] == "scan_b8_t2048_d1024"
    assert (r["config"]["raw_dtype"], r["config"]["read_dtype"]) == ("bf16", "fp32")
    tokens = 8 * 2048
    seconds = r["ms_per_step"] * 1e-3
    assert r["value"] == pytest.approx(tokens / seconds, rel=1e-9)
    rf = r["roofline"]
    assert (rf["bound"], rf["unit"], rf["peak"]) == ("hbm", "GB/s", 8000.0)
    assert rf["algorithmic_bytes"] == 11264 * tokens
    assert rf["achieved"] == pytest.approx(rf["algorithmic_bytes"] / seconds / 1e9, rel=1e-9)
    assert rf["frac"] == pytest.approx(rf["achieved"] / rf["peak"], rel=1e-12)
    assert rf["event_us_per_launch"] == pytest.approx(r["ms_per_step"] * 1e3, rel=1e-9)
    # counters read at least the algorithmic bytes (or the figure is absent)
    assert rf["traffic"] is None or rf["traffic"] >= rf["algorithmic_bytes"]
    assert 0.2 < rf["frac"] < 1.0
