#!/usr/bin/env python3
"""Write the golden fixtures of the Field block from the reference's own CPU path.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_golden.py

It imports ``field_only_v4_chunked_triton_wiki100`` from /root/reference (CPU, Triton absent,
``backend="reference"``) and records inputs and outputs of ``FieldBlock.forward``
(canon:1198-1221), whose transcription — RMSNorm eps, gate, residual, dtype casts, SwiGLU chunk
order, parameter construction order — no closed form pins. The scan output ``read`` is recorded
as the block's intermediate (the input of ``mixer.read_norm``). Only arrays are written: the
reference's code stays where it is.

Fixtures (float32 unless noted):
  selftest_block.npz   dim 64 (C = 32), B 2, T 37, field_chunk 8, ff_hidden 192, seed 7721
                        (the geometry of canon:1396-1420): state_dict, x, raw, read, mixer_out,
                        block_out.
  selftest_block_bf16.npz  the same block cast to bfloat16 and run under bf16 autocast
                        (bf16 values stored as float32).
  config1_block.npz    dim 1024, B 1, T 2048, field_chunk 32, ff_hidden 2752, seed 0, x ~ N(0,1)
                        drawn after construction: per-parameter checksums, x checksum, rows
                        ROWS of read / mixer_out / block_out, final complex state.
"""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

import numpy as np
import torch

REF_DIR = Path("/root/reference/src/fields_official/reference")
OUT_DIR = Path(__file__).resolve().parent
ROWS = (0, 1, 31, 32, 63, 64, 1023, 2047)


def load_canon():
    if str(REF_DIR) not in sys.path:
        sys.path.insert(0, str(REF_DIR))
    return importlib.import_module("field_only_v4_chunked_triton_wiki100")


def run_block(block, x):
    """Forward with hooks: returns raw, read, mixer_out, block_out."""
    rec = {}
    h1 = block.mixer.write_proj.register_forward_hook(lambda m, i, o: rec.__setitem__("raw", o.detach().clone()))
    h2 = block.mixer.read_norm.register_forward_pre_hook(lambda m, i: rec.__setitem__("read", i[0].detach().clone()))
    h3 = block.mixer.register_forward_hook(lambda m, i, o: rec.__setitem__("mixer_out", o.detach().clone()))
    with torch.no_grad():
        out = block(x)
    for h in (h1, h2, h3):
        h.remove()
    return rec["raw"], rec["read"], rec["mixer_out"], out.detach()


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().numpy()


def checksums(sd):
    keys = sorted(sd)
    return (np.array(keys),
            np.array([float(sd[k].double().sum()) for k in keys]),
            np.array([float(sd[k].double().abs().sum()) for k in keys]),
            np.stack([sd[k].flatten()[:8].float().numpy() for k in keys]))


def main() -> None:
    canon = load_canon()
    torch.set_num_threads(8)

    # (i) self-test geometry, fp32 and bf16
    torch.manual_seed(7721)
    block = canon.FieldBlock(64, "reference", 8, 8, 16, 192)
    x = torch.randn(2, 37, 64)
    raw, read, mix, out = run_block(block, x)
    sd = block.state_dict()
    payload = {f"param::{k}": f32(v) for k, v in sd.items()}
    payload.update(x=f32(x), raw=f32(raw), read=f32(read), mixer_out=f32(mix), block_out=f32(out))
    np.savez_compressed(OUT_DIR / "selftest_block.npz", **payload)

    # bf16 runs under autocast, as the reference's arenas and examples do (canon:128-133,
    # examples/inference.py:29-33); without it out_proj would see fp32 read and bf16 weights.
    block_bf = block.to(torch.bfloat16)
    xb = x.to(torch.bfloat16)
    with torch.autocast(device_type="cpu", dtype=torch.bfloat16):
        raw, read, mix, out = run_block(block_bf, xb)
    payload = dict(x=f32(xb), raw=f32(raw), read=f32(read), mixer_out=f32(mix), block_out=f32(out))
    np.savez_compressed(OUT_DIR / "selftest_block_bf16.npz", **payload)

    # (ii) config 1: promoted Field-block geometry, seed 0
    torch.manual_seed(0)
    block = canon.FieldBlock(1024, "reference", 32, 32, 64, 2752)
    x = torch.randn(1, 2048, 1024)
    raw, read, mix, out = run_block(block, x)
    keys, sums, abss, heads = checksums(block.state_dict())
    rows = np.array(ROWS)
    c = 512
    final = read[0, -1]
    np.savez_compressed(
        OUT_DIR / "config1_block.npz",
        param_keys=keys, param_sum=sums, param_abs=abss, param_head=heads,
        x_sum=np.array(float(x.double().sum())), x_head=f32(x.flatten()[:16]),
        rows=rows, read_rows=f32(read[0, rows]), mixer_rows=f32(mix[0, rows]),
        block_rows=f32(out[0, rows]), raw_rows=f32(raw[0, rows]),
        final_state=np.stack([f32(final[:c]), f32(final[c:2 * c])]),
        block_out_abs_max=np.array(float(out.abs().max())),
        read_abs_max=np.array(float(read.abs().max())),
    )
    for p in sorted(OUT_DIR.glob("*.npz")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
