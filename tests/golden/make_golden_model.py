#!/usr/bin/env python3
"""Write golden fixtures of the promoted model's stock-PyTorch blocks from the reference's own
modules (CPU), for the pieces no closed form pins:

  * refresh block ``FusionRefreshBlockV21`` (field_fusion_system_smoke_v21.py:131-293) with its
    latent GQA landmark attention: dim 64, 4 query / 2 KV heads, latent 16, window 8, landmark
    chunk 4, FFN 96, full residual gate; B 2 x T 37 (several windows, padding, landmarks) and
    B 2 x T 6 (one window, no landmark);
  * softpatch ``FastBoundaryStateMixer`` (field_hybrid_speed_optimization_v6.py:293-338) as the
    token model builds it (vocabulary 16,384, so the lexical prior table is zero), learned
    boundary scorer: dim 64, rank 8, B 2 x T 41.

Weights that the reference initialises to zero (the residual gate's weight, the softpatch's up
and score weights) are set to small random values first, so that every term reaches the output.
Run in the build container only: python tests/golden/make_golden_model.py
"""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

import numpy as np
import torch

SRC = Path("/root/reference/src/fields_official/reference/official_source")
OUT = Path(__file__).resolve().parent / "model_blocks.npz"


def main() -> None:
    for p in (SRC, SRC.parent):
        if str(p) not in sys.path:
            sys.path.insert(0, str(p))
    v21 = importlib.import_module("field_fusion_system_smoke_v21")
    v3 = importlib.import_module("field_hybrid_attentionfree_qualification_v3")
    v6 = importlib.import_module("field_hybrid_speed_optimization_v6")
    arrays = {}

    torch.manual_seed(2024)
    blk = v21.FusionRefreshBlockV21(64, 4, 2, 16, 8, 4, 96, light_gate=False)
    with torch.no_grad():
        blk.residual_gate.weight.normal_(0.0, 0.05)
        blk.attn.global_mix_logit.fill_(0.25)
        blk.norm1.weight.uniform_(0.5, 1.5)
        blk.norm2.weight.uniform_(0.5, 1.5)
    for k, v in blk.state_dict().items():
        arrays[f"refresh::param::{k}"] = v.numpy()
    g = torch.Generator().manual_seed(7)
    for name, t in (("long", 37), ("short", 6)):
        x = torch.randn(2, t, 64, generator=g)
        with torch.no_grad():
            y = blk(x)
        arrays[f"refresh::{name}::x"] = x.numpy()
        arrays[f"refresh::{name}::y"] = y.numpy()

    v3.VOCAB = 16_384  # the token model's vocabulary (v18 patches the module the same way)
    v6.v3_global = v3  # the module-level binding its main() / the arena loader installs
    torch.manual_seed(2025)
    sp = v6.FastBoundaryStateMixer(64, 8, True, 0.16, v3)
    with torch.no_grad():
        sp.up.weight.normal_(0.0, 0.1)
        sp.score.weight.normal_(0.0, 0.2)
        sp.norm.weight.uniform_(0.5, 1.5)
    for k, v in sp.state_dict().items():
        arrays[f"softpatch::param::{k}"] = v.numpy()
    x = torch.randn(2, 41, 64, generator=g)
    tokens = torch.randint(0, 16_384, (2, 41), generator=g)
    with torch.no_grad():
        y = sp(x, tokens)
    arrays["softpatch::x"] = x.numpy()
    arrays["softpatch::tokens"] = tokens.numpy()
    arrays["softpatch::y"] = y.numpy()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
