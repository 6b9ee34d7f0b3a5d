"""Synthetic inputs of the benchmark configurations (shared by bench.py and the GPU tests).

Config numbering follows the measured workloads of this path:
  2. scan in isolation: B=8, T=2048, d_model=1024, bf16 raw from a random-init Field mixer's
     write_proj (seed 1) applied to N(0,1) bf16 hidden states;
  4. long context: B=1, T=65,536, same construction with seed 3;
  decode: B=64 tokens of the same construction (seed 5) for the single-token step.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .field import IndependentVacancyField

SCAN_CONFIGS = {
    "scan_b8_t2048_d1024": dict(B=8, T=2048, dim=1024, seed=1),
    "scan_b1_t65536_d1024": dict(B=1, T=65536, dim=1024, seed=3),
}


@dataclass
class ScanWorkload:
    name: str
    raw: torch.Tensor  # [B,T,3C] bf16 (or fp32)
    tr: torch.Tensor
    ti: torch.Tensor
    gamma: torch.Tensor

    @property
    def tokens(self) -> int:
        return self.raw.shape[0] * self.raw.shape[1]

    @property
    def channels(self) -> int:
        return self.tr.numel()


def make_scan_workload(name: str, device, dtype: torch.dtype = torch.bfloat16,
                       batch: int | None = None, length: int | None = None) -> ScanWorkload:
    """raw = write_proj(x) of a seeded random-init mixer, x ~ N(0,1) in bf16, under bf16 autocast."""
    cfg = dict(SCAN_CONFIGS[name])
    if batch is not None:
        cfg["B"] = batch
    if length is not None:
        cfg["T"] = length
    torch.manual_seed(cfg["seed"])
    mixer = IndependentVacancyField(cfg["dim"], "triton", 32, 32, 64).to(device)
    g = torch.Generator(device=device).manual_seed(cfg["seed"])
    with torch.no_grad():
        x = torch.randn(cfg["B"], cfg["T"], cfg["dim"], device=device, dtype=torch.bfloat16, generator=g)
        with torch.autocast(device_type=torch.device(device).type, dtype=torch.bfloat16):
            raw = mixer.write_proj(x)
        raw = raw.to(dtype).contiguous()
        tr, ti, gamma = mixer.transition()
    return ScanWorkload(name, raw, tr.detach(), ti.detach(), gamma.detach())


def scan_bytes_per_token(channels: int, raw_dtype: torch.dtype, read_bytes: int = 4) -> int:
    """Algorithmic HBM bytes per token: raw read once (3C) + read written once (4C)."""
    raw_bytes = 2 if raw_dtype == torch.bfloat16 else 4
    return 3 * channels * raw_bytes + 4 * channels * read_bytes
