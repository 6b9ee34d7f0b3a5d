"""The promoted Fields model (18F/2M/4R + PCAF) for inference, with the Field blocks on the HIP
kernels and every other block as stock PyTorch-ROCm ops.

Reference (paths relative to src/fields_official/):
  api  = fields_official.py                       FieldsConfig / FieldsForCausalLM / build_official_fields
  v20  = reference/official_source/field_fusion_300m_screen_v20.py   RMSNorm, SwiGLU, RoPE, GQA SDPA
  v21  = reference/official_source/field_fusion_system_smoke_v21.py  refresh block, token system
  v25  = reference/official_source/field_fusion_wiki100_mamba2_v25.py Mamba-2 residual block
  v29  = reference/official_source/field_fusion_delta_quality_ablation_v29.py  Mamba-2 placement
  r1   = reference/official_source/field_fusion_reengineering_r1_redundancy_map.py  18F/2M/4R arm
  v3/v6 = reference/official_source/field_hybrid_{attentionfree_qualification_v3,speed_optimization_v6}.py
         softpatch (BoundaryStateMixer) and the PCAF cache's parameters

Topology (api:72-91, r1:65-95, v21:586-616, v29:385-421): tied embedding (16,384 x 1,024);
24 blocks, Field blocks at every position except Mamba-2 at 10 and 22 and refresh attention at
5, 11, 17, 23 (windows 256, 512, 1024, 1024; landmark chunk 256; 16 query / 4 KV heads, latent
256); the softpatch after block 11; final RMSNorm; tied LM head. The FFN width is solved for 300M
parameters in steps of 32 (r1:263-321), and the first / last four Field blocks get -256 / +256
(r1:174-203). PCAF (v21:296-570) only changes ``loss_and_stats``; its parameters are kept so that
a reference state_dict loads with ``strict=True``, its loss routing is not rebuilt.

Decode: every block keeps a fixed-shape incremental state (Field: the complex state; refresh:
the current window's keys/values and the landmark keys/values plus the running latent sum of the
current landmark chunk; Mamba-2: convolution window and SSM state; softpatch: the boundary-scan
state), advanced by ``step`` with no shape that depends on the position, so one decode step can be
captured in a HIP graph and replayed token after token. The reference has no incremental decode:
it re-runs the whole prefix for every generated token.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Dict, List, Mapping, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .field import FieldBlock, RMSNorm, boundary_scan

# api:72-91
OFFICIAL_ARCHITECTURE: Mapping[str, Any] = {
    "name": "Fields 18F/2M/4R + PCAF",
    "vocabulary_size": 16_384,
    "target_parameters": 300_000_000,
    "model_dimension": 1_024,
    "block_count": 24,
    "native_field_positions": (0, 1, 2, 3, 4, 6, 7, 8, 9, 12, 13, 14, 15, 16, 18, 19, 20, 21),
    "mamba2_positions": (10, 22),
    "refresh_positions": (5, 11, 17, 23),
    "refresh_windows": (256, 512, 1024, 1024),
    "pcaf_enabled": True,
    "field_chunk": 32,
    "triton_channel_block": 32,
    "triton_time_chunk": 64,
}

# promoted hyper-parameters (oac:208-263, v25:455-468, v21:586-616, r1:174-203)
Q_HEADS, KV_HEADS, LATENT_DIM, LANDMARK_CHUNK = 16, 4, 256, 256
MAMBA = dict(d_state=128, d_conv=4, expand=2, headdim=64, ngroups=1, chunk_size=256)
SOFTPATCH_RANK = 64
FF_MULTIPLE = 32
LATE_FF_DELTA = 256


# ======================================================================================
# shared pieces (v20:94-163)
# ======================================================================================

class NativeRMSNorm(nn.Module):
    """v20:94-104: F.rms_norm with the weight cast to the input dtype (eps 1e-6)."""

    def __init__(self, dim: int, eps: float = 1.0e-6) -> None:
        super().__init__()
        self.dim = int(dim)
        self.eps = float(eps)
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.rms_norm(x, (self.dim,), self.weight.to(dtype=x.dtype), self.eps)


class GateUpSwiGLU(nn.Module):
    """v20:107-117 (``PackedSwiGLU`` of the refresh blocks and of the R1-resized Field FFNs):
    down(silu(gate) * up) with gate, up = gate_up(x).chunk(2)."""

    def __init__(self, dim: int, hidden: int) -> None:
        super().__init__()
        self.gate_up = nn.Linear(dim, 2 * hidden, bias=False)
        self.down = nn.Linear(hidden, dim, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = self.gate_up(x).chunk(2, dim=-1)
        return self.down(F.silu(gate) * up)


_ROPE: Dict[Tuple[str, int, torch.dtype, int], Tuple[torch.Tensor, torch.Tensor]] = {}


def rope_cos_sin(device, dtype: torch.dtype, length: int, head_dim: int):
    """Half-split RoPE tables, base 10,000, positions 0..length-1 (v20:121-137): [1,1,L,hd/2]."""
    key = (str(device), int(length), dtype, int(head_dim))
    hit = _ROPE.get(key)
    if hit is not None:
        return hit
    inv = 1.0 / (10000.0 ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    freq = torch.outer(torch.arange(length, device=device, dtype=torch.float32), inv)
    out = (freq.cos().to(dtype)[None, None], freq.sin().to(dtype)[None, None])
    _ROPE[key] = out
    return out


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """v20:140-144: rotate (first half, second half) pairs."""
    half = x.shape[-1] // 2
    a, b = x[..., :half], x[..., half:]
    return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)


def gqa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  allowed: Optional[torch.Tensor], causal: bool) -> torch.Tensor:
    """softmax(q k^T / sqrt(hd) + mask) v with grouped KV heads (query head h reads KV head
    h // (Hq / Hkv), the grouping of v20:147-163's ``enable_gqa``).

    q [N, Hq, Lq, hd], k/v [N, Hkv, Lk, hd]; ``allowed`` a bool mask broadcastable to
    [N, Hkv, Lq, Lk] (True = visible) or None; ``causal`` adds j <= i (Lq == Lk). The products run
    as plain matmuls on contiguous operands with an fp32 softmax.
    """
    n, hq, lq, hd = q.shape
    hkv, lk = k.shape[1], k.shape[2]
    rep = hq // hkv
    qg = q.reshape(n, hkv, rep * lq, hd)
    kt = k.transpose(-1, -2).contiguous()
    scores = torch.matmul(qg, kt).float().view(n, hkv, rep, lq, lk) * (hd ** -0.5)
    if causal:
        i = torch.arange(lq, device=q.device)
        mask = i[:, None] >= torch.arange(lk, device=q.device)[None, :]
        scores = scores.masked_fill(~mask, float("-inf"))
    if allowed is not None:
        scores = scores.masked_fill(~allowed.unsqueeze(-3), float("-inf"))
    p = torch.softmax(scores, dim=-1).to(v.dtype).view(n, hkv, rep * lq, lk)
    return torch.matmul(p, v.contiguous()).view(n, hq, lq, hd)


# ======================================================================================
# refresh block (v21:131-294)
# ======================================================================================

class LandmarkAttention(nn.Module):
    """Latent GQA attention with block-local windows and causal landmarks (v21:131-253).

    Local branch: tokens are split into consecutive windows of ``local_window``; a token attends
    causally inside its own window. Global branch: one landmark per completed chunk of
    ``landmark_chunk`` tokens, the chunk's mean latent lifted by ``kv_up`` (key rotated to the
    chunk's last position); a token in chunk c reads a null slot and the landmarks of chunks < c.
    out = out_proj(local + sigmoid(global_mix_logit) * global).
    """

    def __init__(self, dim: int, q_heads: int, kv_heads: int, latent_dim: int,
                 local_window: int, landmark_chunk: int) -> None:
        super().__init__()
        if dim % q_heads or q_heads % kv_heads:
            raise ValueError("dim % q_heads and q_heads % kv_heads must be 0")
        self.dim, self.q_heads, self.kv_heads = int(dim), int(q_heads), int(kv_heads)
        self.head_dim = dim // q_heads
        self.latent_dim = int(latent_dim)
        self.local_window = int(local_window)
        self.landmark_chunk = int(landmark_chunk)
        self.q_latent_proj = nn.Linear(dim, q_heads * self.head_dim + latent_dim, bias=False)
        self.kv_up = nn.Linear(latent_dim, 2 * kv_heads * self.head_dim, bias=False)
        self.out_proj = nn.Linear(dim, dim, bias=False)
        self.global_mix_logit = nn.Parameter(torch.tensor(-0.7))

    @property
    def q_width(self) -> int:
        return self.q_heads * self.head_dim

    def _heads(self, x: torch.Tensor, h: int) -> torch.Tensor:
        b, t, _ = x.shape
        return x.view(b, t, h, self.head_dim).transpose(1, 2)

    def _local(self, q, k, v) -> torch.Tensor:
        b, hq, length, hd = q.shape
        w = min(self.local_window, length)
        pad = (-length) % w
        if pad:
            q, k, v = (F.pad(t, (0, 0, 0, pad)) for t in (q, k, v))
        g = q.shape[2] // w

        def groups(t, h):
            return t.reshape(b, h, g, w, hd).permute(0, 2, 1, 3, 4).reshape(b * g, h, w, hd)

        y = gqa_attention(groups(q, hq), groups(k, self.kv_heads), groups(v, self.kv_heads), None, True)
        y = y.reshape(b, g, hq, w, hd).permute(0, 2, 1, 3, 4).reshape(b, hq, g * w, hd)
        return y[:, :, :length]

    def _landmarks(self, latent: torch.Tensor, full: int, cos, sin):
        """Keys / values of the first ``full`` landmarks: [B, Hkv, full, hd] each."""
        b = latent.shape[0]
        c = self.landmark_chunk
        mean = latent[:, : full * c].reshape(b, full, c, self.latent_dim).mean(dim=2)
        lk, lv = self.kv_up(mean).split(self.kv_heads * self.head_dim, dim=-1)
        lk, lv = self._heads(lk, self.kv_heads), self._heads(lv, self.kv_heads)
        pos = torch.arange(c - 1, full * c, c, device=latent.device)
        return apply_rope(lk, cos[:, :, pos], sin[:, :, pos]), lv

    def _global(self, q, latent, cos, sin) -> torch.Tensor:
        b, _, length, hd = q.shape
        c = self.landmark_chunk
        full = length // c
        if full == 0:
            return q.new_zeros(q.shape)
        lk, lv = self._landmarks(latent, full, cos, sin)
        zero = lk.new_zeros((b, self.kv_heads, 1, hd))
        lk, lv = torch.cat((zero, lk), 2), torch.cat((zero, lv), 2)
        chunk_of = torch.arange(length, device=q.device) // c
        allowed = torch.cat((torch.ones(length, 1, device=q.device, dtype=torch.bool),
                             torch.arange(full, device=q.device)[None, :] < chunk_of[:, None]), 1)
        return gqa_attention(q, lk, lv, allowed, False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        b, length, _ = x.shape
        qraw, latent = self.q_latent_proj(x).split((self.q_width, self.latent_dim), dim=-1)
        kraw, vraw = self.kv_up(latent).split(self.kv_heads * self.head_dim, dim=-1)
        q, k, v = self._heads(qraw, self.q_heads), self._heads(kraw, self.kv_heads), self._heads(vraw, self.kv_heads)
        cos, sin = rope_cos_sin(x.device, x.dtype, length, self.head_dim)
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        y = self._local(q, k, v)
        y = y + torch.sigmoid(self.global_mix_logit).to(y.dtype) * self._global(q, latent, cos, sin)
        return self.out_proj(y.transpose(1, 2).reshape(b, length, self.dim))

    # ---------------------------------------------------------------- incremental decode
    def new_state(self, batch: int, max_len: int, device, dtype) -> Dict[str, torch.Tensor]:
        self._rope_len = int(max_len)
        hd, h, w = self.head_dim, self.kv_heads, self.local_window
        # landmark slots: 0 is the null slot, slot k + 1 holds chunk k's landmark. The step at
        # position p writes its own chunk's running landmark to slot p // c + 1, so positions
        # below max_len use slots up to (max_len - 1) // c + 1 (with fewer, the last chunk's
        # running landmark would land on the one before it, which later tokens read)
        n_land = (max_len - 1) // self.landmark_chunk + 1
        return {
            "kt": torch.zeros(batch, h, hd, w, device=device, dtype=dtype),   # keys, transposed
            "v": torch.zeros(batch, h, w, hd, device=device, dtype=dtype),
            "lkt": torch.zeros(batch, h, hd, 1 + n_land, device=device, dtype=dtype),
            "lv": torch.zeros(batch, h, 1 + n_land, hd, device=device, dtype=dtype),
            "lat_sum": torch.zeros(batch, self.latent_dim, device=device, dtype=torch.float32),
        }

    def prefill(self, x: torch.Tensor, max_len: int) -> Tuple[torch.Tensor, Dict[str, torch.Tensor]]:
        """forward(x) plus the decode state after position T-1."""
        b, length, _ = x.shape
        if length + 1 > max_len:
            raise ValueError("max_len must exceed the prompt length")
        qraw, latent = self.q_latent_proj(x).split((self.q_width, self.latent_dim), dim=-1)
        kraw, vraw = self.kv_up(latent).split(self.kv_heads * self.head_dim, dim=-1)
        q, k, v = self._heads(qraw, self.q_heads), self._heads(kraw, self.kv_heads), self._heads(vraw, self.kv_heads)
        cos, sin = rope_cos_sin(x.device, x.dtype, max_len, self.head_dim)
        cl, sl = cos[:, :, :length], sin[:, :, :length]
        q, k = apply_rope(q, cl, sl), apply_rope(k, cl, sl)
        y = self._local(q, k, v)
        y = y + torch.sigmoid(self.global_mix_logit).to(y.dtype) * self._global(q, latent, cl, sl)
        out = self.out_proj(y.transpose(1, 2).reshape(b, length, self.dim))
        st = self.new_state(b, max_len, x.device, x.dtype)
        self._rope_len = int(max_len)
        w, c = self.local_window, self.landmark_chunk
        g0 = (length // w) * w  # the next token opens a window at g0 or continues it
        n = length - g0
        if n:
            st["kt"][..., :n] = k[:, :, g0:].transpose(-1, -2)
            st["v"][:, :, :n] = v[:, :, g0:]
        full = length // c
        if full:
            lk, lv = self._landmarks(latent, full, cos, sin)
            st["lkt"][..., 1:1 + full] = lk.transpose(-1, -2)
            st["lv"][:, :, 1:1 + full] = lv
        st["lat_sum"] = latent[:, full * c:].float().sum(1)
        return out, st

    def step(self, x_t: torch.Tensor, pos: torch.Tensor, st: Dict[str, torch.Tensor]) -> torch.Tensor:
        """One token at position ``pos`` (0-d int64 device tensor): x_t [B, dim] -> [B, dim].

        Static shapes only: the window slot, the landmark slot and the visibility masks are
        computed on the device from ``pos``. Positions must stay below the ``max_len`` given to
        :meth:`prefill` / :meth:`new_state`; every slot index is clamped into its buffer."""
        b = x_t.shape[0]
        hd, hq, hkv = self.head_dim, self.q_heads, self.kv_heads
        w, c = self.local_window, self.landmark_chunk
        qraw, latent = self.q_latent_proj(x_t).split((self.q_width, self.latent_dim), dim=-1)
        kraw, vraw = self.kv_up(latent).split(hkv * hd, dim=-1)
        cos, sin = rope_cos_sin(x_t.device, x_t.dtype, self._rope_len, hd)
        # gathered on the device (no host read of the position); clamped to the table, so a
        # position past the prefill's max_len reads the last row (and is not supported) instead
        # of reading out of bounds
        p1 = torch.clamp(pos, max=self._rope_len - 1).view(1)
        ct, stt = cos[0, 0].index_select(0, p1), sin[0, 0].index_select(0, p1)   # [1, hd/2]
        q = apply_rope(qraw.view(b, hq, hd), ct, stt)                  # [B,Hq,hd]
        k = apply_rope(kraw.view(b, hkv, hd), ct, stt)                 # [B,Hkv,hd]
        vv = vraw.view(b, hkv, hd)
        slot = torch.remainder(pos, w)
        st["kt"].index_copy_(3, slot.view(1), k.unsqueeze(-1))
        st["v"].index_copy_(2, slot.view(1), vv.unsqueeze(2))
        qg = q.view(b, hkv, hq // hkv, hd)
        local_ok = torch.arange(w, device=x_t.device) <= slot        # slots of this window so far
        s_loc = torch.matmul(qg, st["kt"]).float() * (hd ** -0.5)
        s_loc = s_loc.masked_fill(~local_ok, float("-inf"))
        y = torch.matmul(torch.softmax(s_loc, -1).to(vv.dtype), st["v"])
        # landmarks of completed chunks (slot 0 = null)
        chunk = torch.div(pos, c, rounding_mode="floor")
        n_slots = st["lv"].shape[2]
        land_ok = torch.arange(n_slots, device=x_t.device) <= chunk   # null + chunks < current
        s_g = torch.matmul(qg, st["lkt"]).float() * (hd ** -0.5)
        s_g = s_g.masked_fill(~land_ok, float("-inf"))
        g = torch.matmul(torch.softmax(s_g, -1).to(vv.dtype), st["lv"])
        y = y + torch.sigmoid(self.global_mix_logit).to(y.dtype) * g
        # running mean latent of the current chunk; its landmark is (re)written every step and
        # becomes visible once the chunk is complete (slot chunk+1 <= chunk of later tokens)
        fresh = (torch.remainder(pos, c) == 0).to(torch.float32)
        st["lat_sum"].mul_(1.0 - fresh).add_(latent.float())
        mean = (st["lat_sum"] / c).to(x_t.dtype)
        lk, lv = self.kv_up(mean).split(hkv * hd, dim=-1)
        lk = apply_rope(lk.view(b, hkv, hd), ct, stt)
        # (the clamp only keeps a position past max_len, which is not supported, in bounds)
        lslot = torch.clamp(chunk + 1, max=n_slots - 1).view(1)
        st["lkt"].index_copy_(3, lslot, lk.unsqueeze(-1))
        st["lv"].index_copy_(2, lslot, lv.view(b, hkv, 1, hd))
        return self.out_proj(y.reshape(b, self.dim))


class RefreshBlock(nn.Module):
    """v21:256-293 (``FusionRefreshBlockV21``, full residual gate): x + sigmoid(gate(z)) *
    attn(z) with z = norm1(x), then x + ff(norm2(x))."""

    def __init__(self, dim: int, q_heads: int, kv_heads: int, latent_dim: int, local_window: int,
                 landmark_chunk: int, ff_hidden: int, *, light_gate: bool = False) -> None:
        super().__init__()
        self.norm1 = NativeRMSNorm(dim)
        self.attn = LandmarkAttention(dim, q_heads, kv_heads, latent_dim, local_window, landmark_chunk)
        self.light_gate = bool(light_gate)
        init = math.log(0.25 / 0.75)
        if self.light_gate:
            self.residual_gate_logit = nn.Parameter(torch.full((dim,), init))
            self.residual_gate = None
        else:
            self.residual_gate = nn.Linear(dim, dim, bias=True)
            nn.init.zeros_(self.residual_gate.weight)
            nn.init.constant_(self.residual_gate.bias, init)
            self.register_parameter("residual_gate_logit", None)
        self.norm2 = NativeRMSNorm(dim)
        self.ff = GateUpSwiGLU(dim, ff_hidden)
        self.window = int(local_window)

    def _gate(self, z):
        if self.light_gate:
            return torch.sigmoid(self.residual_gate_logit).to(z.dtype)
        return torch.sigmoid(self.residual_gate(z))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        z = self.norm1(x)
        x = x + self._gate(z) * self.attn(z)
        return x + self.ff(self.norm2(x))

    def prefill(self, x: torch.Tensor, max_len: int):
        z = self.norm1(x)
        a, st = self.attn.prefill(z, max_len)
        x = x + self._gate(z) * a
        return x + self.ff(self.norm2(x)), st

    def step(self, x_t: torch.Tensor, pos: torch.Tensor, st) -> torch.Tensor:
        z = self.norm1(x_t)
        x_t = x_t + self._gate(z) * self.attn.step(z, pos, st)
        return x_t + self.ff(self.norm2(x_t))


# ======================================================================================
# Mamba-2 (v25:73-91; the mixer restates mamba_ssm 2.3.2's Mamba2 with its parameter layout)
# ======================================================================================

class GatedRMSNorm(nn.Module):
    """y = rmsnorm(x * silu(z)) * weight over the whole width (Mamba-2's output norm with
    norm_before_gate=False and one group), fp32 math, eps 1e-5."""

    def __init__(self, dim: int, eps: float = 1e-5) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = float(eps)

    def forward(self, x: torch.Tensor, z: torch.Tensor) -> torch.Tensor:
        y = x.float() * F.silu(z.float())
        y = y * torch.rsqrt(y.square().mean(-1, keepdim=True) + self.eps)
        return y * self.weight.float()


def ssd_chunked(x, dt, A, Bm, Cm, chunk: int, initial_state=None):
    """State-space-duality scan of Mamba-2 in fp32 (the chunked algorithm of Dao & Gu, 2024):

        h_t = exp(dt_t A) h_{t-1} + dt_t x_t B_t^T,   y_t = h_t C_t       (per head)

    x [b,l,h,p], dt [b,l,h] (after softplus), A [h] (negative), Bm/Cm [b,l,n] (one group).
    Within a chunk the output is a masked (C B^T ∘ decay) product; chunk states are carried by
    a short sequential loop. Returns (y [b,l,h,p], final state [b,h,p,n]).
    """
    b, l, h, p = x.shape
    n = Bm.shape[-1]
    pad = (-l) % chunk
    if pad:  # dt = 0 on padded steps: decay 1, input 0 (identity)
        x, dt, Bm, Cm = (F.pad(t, (0, 0) * (t.dim() - 2) + (0, pad)) for t in (x, dt, Bm, Cm))
    L = x.shape[1]
    c = L // chunk
    xdt = (x.float() * dt.float()[..., None]).view(b, c, chunk, h, p).permute(0, 3, 1, 2, 4).contiguous()
    adt = (dt.float() * A.float()).view(b, c, chunk, h).permute(0, 3, 1, 2)          # [b,h,c,s]
    acs = torch.cumsum(adt, -1)
    Bc = Bm.float().view(b, c, chunk, n)
    Cc = Cm.float().view(b, c, chunk, n)
    # intra-chunk: y_i = sum_{j<=i} (C_i.B_j) exp(acs_i - acs_j) xdt_j
    seg = acs[..., :, None] - acs[..., None, :]                                        # [b,h,c,s,s]
    causal = torch.ones(chunk, chunk, device=x.device, dtype=torch.bool).tril()
    decay = torch.exp(seg.masked_fill(~causal, float("-inf")))
    cb = torch.matmul(Cc, Bc.transpose(-1, -2).contiguous())                            # [b,c,s,s]
    y = torch.matmul(cb[:, None] * decay, xdt)                                          # [b,h,c,s,p]
    # chunk states from 0: sum_j exp(acs_end - acs_j) xdt_j B_j^T
    w_end = torch.exp(acs[..., -1:] - acs)                                              # [b,h,c,s]
    states = torch.matmul((xdt * w_end[..., None]).transpose(-1, -2).contiguous(), Bc[:, None])  # [b,h,c,p,n]
    chunk_decay = torch.exp(acs[..., -1])                                               # [b,h,c]
    s = (initial_state.float() if initial_state is not None
         else torch.zeros(b, h, p, n, device=x.device, dtype=torch.float32))
    carries = []
    for i in range(c):
        carries.append(s)
        s = s * chunk_decay[:, :, i, None, None] + states[:, :, i]
    carry = torch.stack(carries, 2)                                                     # [b,h,c,p,n]
    # inter-chunk: y_i += exp(acs_i) C_i carry
    y_off = torch.matmul(Cc[:, None], carry.transpose(-1, -2).contiguous())             # [b,h,c,s,p]
    y = y + y_off * torch.exp(acs)[..., None]
    y = y.permute(0, 2, 3, 1, 4).reshape(b, L, h, p)[:, :l]
    return y, s


class Mamba2Mixer(nn.Module):
    """Mamba-2 mixer in mamba_ssm 2.3.2's parameter layout (``in_proj``, ``conv1d``, ``dt_bias``,
    ``A_log``, ``D``, ``norm``, ``out_proj``; d_state 128, d_conv 4, expand 2, headdim 64, one
    group, chunk 256 — v25:455-468) and its initialisation ranges (dt in [1e-3, 0.1] log-uniform,
    floor 1e-4, stored as softplus^-1; A in [1, 16]; D = 1).

    in_proj(u) = [z | xBC | dt]; xBC = silu(causal depthwise conv(xBC)) = [x | B | C];
    dt = softplus(dt + dt_bias); y = SSD(x, dt, -exp(A_log), B, C) + D x; out_proj(norm(y, z)).
    """

    def __init__(self, d_model: int, d_state: int = 128, d_conv: int = 4, expand: int = 2,
                 headdim: int = 64, ngroups: int = 1, chunk_size: int = 256,
                 dt_min: float = 1e-3, dt_max: float = 0.1, dt_init_floor: float = 1e-4) -> None:
        super().__init__()
        if ngroups != 1:
            raise ValueError("one group (the promoted configuration)")
        self.d_model, self.d_state, self.d_conv = d_model, d_state, d_conv
        self.d_inner = expand * d_model
        self.headdim = headdim
        self.nheads = self.d_inner // headdim
        self.ngroups = ngroups
        self.chunk_size = chunk_size
        self.conv_dim = self.d_inner + 2 * ngroups * d_state
        d_in_proj = 2 * self.d_inner + 2 * ngroups * d_state + self.nheads
        self.in_proj = nn.Linear(d_model, d_in_proj, bias=False)
        self.conv1d = nn.Conv1d(self.conv_dim, self.conv_dim, d_conv, groups=self.conv_dim,
                                padding=d_conv - 1, bias=True)
        dt = torch.exp(torch.rand(self.nheads) * (math.log(dt_max) - math.log(dt_min)) + math.log(dt_min))
        dt = torch.clamp(dt, min=dt_init_floor)
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
        self.A_log = nn.Parameter(torch.log(torch.empty(self.nheads).uniform_(1.0, 16.0)))
        self.D = nn.Parameter(torch.ones(self.nheads))
        self.norm = GatedRMSNorm(self.d_inner)
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=False)

    def _split(self, zxbcdt):
        return zxbcdt.split((self.d_inner, self.conv_dim, self.nheads), dim=-1)

    def _ssm_in(self, xbc, dt):
        x, bm, cm = xbc.split((self.d_inner, self.d_state, self.d_state), dim=-1)
        dt = F.softplus(dt.float() + self.dt_bias.float())
        return x, bm, cm, dt

    def forward(self, u: torch.Tensor, return_state: bool = False):
        b, l, _ = u.shape
        z, xbc_raw, dt = self._split(self.in_proj(u))
        # causal depthwise convolution as d_conv shifted multiply-adds in the channel-last
        # layout: out[t] = bias + sum_k w[k] * in[t - (d_conv-1) + k]
        w = self.conv1d.weight.float()[:, 0]                                           # [C, K]
        xp = F.pad(xbc_raw.float(), (0, 0, self.d_conv - 1, 0))
        xbc = self.conv1d.bias.float() + xp[:, :l] * w[:, 0]
        for k in range(1, self.d_conv):
            xbc = torch.addcmul(xbc, xp[:, k:k + l], w[:, k])
        x, bm, cm, dt = self._ssm_in(F.silu(xbc), dt)
        A = -torch.exp(self.A_log.float())
        xh = x.reshape(b, l, self.nheads, self.headdim)
        y, state = ssd_chunked(xh, dt, A, bm, cm, self.chunk_size)
        y = y + self.D.float()[:, None] * xh
        out = self.out_proj(self.norm(y.reshape(b, l, self.d_inner), z).to(u.dtype))
        if not return_state:
            return out
        conv = xbc_raw.transpose(1, 2)[..., -self.d_conv:].float()
        if conv.shape[-1] < self.d_conv:
            conv = F.pad(conv, (self.d_conv - conv.shape[-1], 0))
        return out, {"conv": conv.contiguous(), "ssm": state.contiguous()}

    def new_state(self, batch: int, device) -> Dict[str, torch.Tensor]:
        return {"conv": torch.zeros(batch, self.conv_dim, self.d_conv, device=device),
                "ssm": torch.zeros(batch, self.nheads, self.headdim, self.d_state, device=device)}

    def step(self, u_t: torch.Tensor, st: Dict[str, torch.Tensor]) -> torch.Tensor:
        """One token: u_t [B, d_model] -> [B, d_model]; conv and SSM state advance in place."""
        b = u_t.shape[0]
        z, xbc_raw, dt = self._split(self.in_proj(u_t))
        conv = st["conv"]
        conv.copy_(torch.roll(conv, shifts=-1, dims=-1))
        conv[..., -1] = xbc_raw.float()
        xbc = (conv * self.conv1d.weight.float()[:, 0]).sum(-1) + self.conv1d.bias.float()
        x, bm, cm, dt = self._ssm_in(F.silu(xbc), dt)
        A = -torch.exp(self.A_log.float())
        xh = x.view(b, self.nheads, self.headdim)
        decay = torch.exp(dt * A)                                                       # [B,H]
        ssm = st["ssm"]
        ssm.mul_(decay[:, :, None, None]).add_((xh * dt[..., None])[..., None] * bm[:, None, None, :])
        y = torch.matmul(ssm, cm[:, None, :, None]).squeeze(-1) + self.D.float()[:, None] * xh
        return self.out_proj(self.norm(y.reshape(b, self.d_inner), z).to(u_t.dtype))


class FastRMSNorm(NativeRMSNorm):
    """v25:63-70: F.rms_norm, eps 1e-5, weight as stored."""

    def __init__(self, dim: int, eps: float = 1.0e-5) -> None:
        super().__init__(dim, eps)


class Mamba2ResidualBlock(nn.Module):
    """v25:73-91: x + mixer(norm(x))."""

    def __init__(self, dim: int, **mamba) -> None:
        super().__init__()
        self.norm = FastRMSNorm(dim)
        self.mixer = Mamba2Mixer(dim, **(mamba or MAMBA))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return x + self.mixer(self.norm(x))

    def prefill(self, x: torch.Tensor, max_len: int):
        y, st = self.mixer(self.norm(x), return_state=True)
        return x + y, st

    def step(self, x_t: torch.Tensor, pos: torch.Tensor, st) -> torch.Tensor:
        return x_t + self.mixer.step(self.norm(x_t), st)


# ======================================================================================
# softpatch (v3:425-462, v6 FastBoundaryStateMixer) and the PCAF parameters (v3:524-570)
# ======================================================================================

class BoundaryStateMixer(nn.Module):
    """x + up([z | s]) with h = norm(x), z = down(h), boundary = clamp(sigmoid(score(h) +
    1.5 prior), 0.01, 0.99), s_t = (1 - boundary_t) s_{t-1} + boundary_t z_t (the boundary scan
    runs in ``fl_boundary_scan``). The lexical prior is zero for a 16,384-token vocabulary
    (v6: the 256-entry byte table applies to byte models only)."""

    def __init__(self, dim: int, rank: int = 64, learned: bool = True, target_rate: float = 0.16,
                 vocab: int = 16_384) -> None:
        super().__init__()
        self.learned, self.target_rate = bool(learned), float(target_rate)
        self.norm = RMSNorm(dim)
        self.down = nn.Linear(dim, rank, bias=False)
        self.score = nn.Linear(dim, 1, bias=True) if learned else None
        if self.score is not None:
            nn.init.zeros_(self.score.weight)
            nn.init.constant_(self.score.bias, math.log(target_rate / (1.0 - target_rate)))
        self.up = nn.Linear(2 * rank, dim, bias=False)
        nn.init.zeros_(self.up.weight)
        self.register_buffer("_boundary_lut", torch.zeros(vocab), persistent=False)
        self.last_aux = torch.tensor(0.0)

    def _boundary(self, h, tokens):
        prior = self._boundary_lut[tokens]
        if not self.learned:
            raise NotImplementedError("only the learned boundary scorer of the promoted model")
        return torch.sigmoid(self.score(h).float().squeeze(-1) + 1.5 * prior).clamp(0.01, 0.99)

    def forward(self, x: torch.Tensor, tokens: torch.Tensor, return_state: bool = False):
        h = self.norm(x)
        z = self.down(h).float()
        boundary = self._boundary(h, tokens)
        state, last = boundary_scan((1.0 - boundary).contiguous(), (boundary[..., None] * z).contiguous(),
                                    return_state=True)
        out = x + self.up(torch.cat((z, state), dim=-1).to(x.dtype))
        return (out, last) if return_state else out

    def step(self, x_t: torch.Tensor, token_t: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
        h = self.norm(x_t)
        z = self.down(h).float()
        boundary = self._boundary(h, token_t)[:, None]
        s.mul_(1.0 - boundary).add_(boundary * z)
        return x_t + self.up(torch.cat((z, s), dim=-1).to(x_t.dtype))


class SuccessorCacheParams(nn.Module):
    """Parameters of the PCAF successor cache (v3:524-570 with the "confidence" router, as
    mirrored by v6's FastSuccessorCacheV5), under the same names. PCAF acts only in
    ``loss_and_stats`` (v21:296-570); the inference path does not use these weights."""

    FEATURE_DIM = 15

    def __init__(self, state_dim: int, memory_dim: int = 64, num_buckets: int = 16_384,
                 order: int = 4, top_k: int = 4) -> None:
        super().__init__()
        self.state_dim, self.memory_dim = state_dim, memory_dim
        self.num_buckets, self.order, self.top_k = num_buckets, order, top_k
        self.router_mode = "confidence"
        self.shared_weight = nn.Parameter(torch.empty(memory_dim, state_dim))
        nn.init.kaiming_uniform_(self.shared_weight, a=math.sqrt(5))
        self.state_gate = nn.Sequential(RMSNorm(state_dim), nn.Linear(state_dim, 1))
        self.router = nn.Sequential(nn.LayerNorm(self.FEATURE_DIM), nn.Linear(self.FEATURE_DIM, 64), nn.SiLU(),
                                    nn.Linear(64, 32), nn.SiLU(), nn.Linear(32, 1))
        nn.init.zeros_(self.router[-1].weight)
        nn.init.zeros_(self.router[-1].bias)
        self.evidence_gain = nn.Parameter(torch.tensor(0.50))
        self.evidence_bias = nn.Parameter(torch.tensor(-0.75))
        self.recency_scale = nn.Parameter(torch.tensor(1.0))
        self.enabled = True


# ======================================================================================
# token system (v21:580-637 with the v29 / r1 patches)
# ======================================================================================

def _kind(block: nn.Module) -> str:
    if isinstance(block, Mamba2ResidualBlock):
        return "mamba"
    if isinstance(block, RefreshBlock):
        return "refresh"
    return "field"


class FieldTokenSystem(nn.Module):
    """Embedding, 24 blocks, softpatch after block ``patch_position``, final norm, tied head."""

    def __init__(self, *, vocab: int, dim: int, ff_hidden: int, refresh_windows=(256, 512, 1024, 1024),
                 mamba_positions=(10, 22), field_chunk: int = 32, triton_block_c: int = 32,
                 triton_chunk_t: int = 64, layers: int = 24, q_heads: int = Q_HEADS,
                 kv_heads: int = KV_HEADS, latent_dim: int = LATENT_DIM,
                 landmark_chunk: int = LANDMARK_CHUNK, softpatch_rank: int = SOFTPATCH_RANK,
                 mamba: Optional[Mapping[str, int]] = None, mamba_seed: Optional[int] = None,
                 late_ff_delta: int = LATE_FF_DELTA) -> None:
        super().__init__()
        if layers != 6 * len(refresh_windows):
            raise ValueError("layers must equal 6 * number of refresh windows (v21:586-587)")
        self.emb = nn.Embedding(vocab, dim)
        blocks: List[nn.Module] = []
        for window in refresh_windows:
            for _ in range(5):
                blocks.append(FieldBlock(dim, "triton", field_chunk, triton_block_c, triton_chunk_t, ff_hidden))
            blocks.append(RefreshBlock(dim, q_heads, kv_heads, latent_dim, int(window), landmark_chunk, ff_hidden))
        self.blocks = nn.ModuleList(blocks)
        self.final_norm = RMSNorm(dim)
        self.lm_head = nn.Linear(dim, vocab, bias=False)
        self.cache = SuccessorCacheParams(dim)
        self.softpatch = BoundaryStateMixer(dim, softpatch_rank, learned=True, vocab=vocab)
        self.patch_position = max(0, layers // 2 - 1)
        self.locals = nn.ModuleDict()
        self.multiscales = nn.ModuleDict()
        if mamba_seed is not None and mamba_positions:  # v29:397-400
            torch.manual_seed(int(mamba_seed))
        for index in mamba_positions:  # v29:401-405
            if _kind(self.blocks[index]) == "refresh":
                raise ValueError(f"cannot replace refresh block {index}")
            self.blocks[index] = Mamba2ResidualBlock(dim, **dict(mamba or MAMBA))
        native = [i for i, b in enumerate(self.blocks) if _kind(b) == "field"]
        if late_ff_delta:
            for i in native[:4]:  # r1:174-203
                self.blocks[i].ff = GateUpSwiGLU(dim, ff_hidden - late_ff_delta)
            for i in native[-4:]:
                self.blocks[i].ff = GateUpSwiGLU(dim, ff_hidden + late_ff_delta)
        self.lm_head.weight = self.emb.weight  # tied (v18:142-157)

    def kinds(self) -> List[str]:
        return [_kind(b) for b in self.blocks]

    def states_logits(self, tokens: torch.Tensor, last_only: bool = False):
        """v21:620-627 / v29:353-381 (inference): hidden states and logits (of the last position
        only when ``last_only``, as v32:461-490's prefill benchmark)."""
        x = self.emb(tokens)
        for i, block in enumerate(self.blocks):
            x = block(x)
            if i == self.patch_position:
                x = self.softpatch(x, tokens)
        h = self.final_norm(x)
        return x, self.lm_head(h[:, -1:] if last_only else h)

    # ---------------------------------------------------------------- incremental decode
    def prefill(self, tokens: torch.Tensor, max_len: int):
        """Logits of the last prompt position and the decode state after it."""
        x = self.emb(tokens)
        states: List[Any] = []
        soft = None
        for i, block in enumerate(self.blocks):
            kind = _kind(block)
            if kind == "field":
                x, st = block.prefill(x)
            else:
                x, st = block.prefill(x, max_len)
            states.append(st)
            if i == self.patch_position:
                x, soft = self.softpatch(x, tokens, return_state=True)
        logits = self.lm_head(self.final_norm(x[:, -1]))
        pos = torch.tensor(tokens.shape[1], device=tokens.device, dtype=torch.long)
        return logits, {"blocks": states, "softpatch": soft.contiguous(), "pos": pos,
                        "params": [b.mixer.decode_params() if _kind(b) == "field" else None for b in self.blocks]}

    def step(self, token_t: torch.Tensor, cache: Dict[str, Any]) -> torch.Tensor:
        """One decode token for every sequence: token_t [B] (int64) -> logits [B, vocab]; the
        cache (including its position counter) advances in place."""
        x = self.emb(token_t)
        pos = cache["pos"]
        for i, block in enumerate(self.blocks):
            st = cache["blocks"][i]
            if _kind(block) == "field":
                x = block.step(x, st, cache["params"][i])
            else:
                x = block.step(x, pos, st)
            if i == self.patch_position:
                x = self.softpatch.step(x, token_t, cache["softpatch"])
        pos.add_(1)
        return self.lm_head(self.final_norm(x))


# ======================================================================================
# public API (api:98-422)
# ======================================================================================

@dataclass(frozen=True)
class FieldsConfig:
    """api:98-150. The architecture is fixed; these fields control initialisation and
    placement. ``source_root`` / ``canonical_source`` / ``cache_dir`` / ``output_dir`` are kept for
    call compatibility: this build carries its own implementation and reads no reference files."""

    source_root: Optional[Path] = None
    canonical_source: Optional[Path] = None
    cache_dir: Path = Path.home() / "field_lab" / "hf_cache"
    output_dir: Path = Path.home() / "pcaf_runs" / "fields_official_api"
    model_seed: int = 1234
    embedding_seed: int = 314159
    pcaf_enabled: bool = True
    amp: str = "bf16"


@dataclass
class FieldsForwardOutput:
    """api:153-166."""

    loss: Optional[torch.Tensor] = None
    primary_loss: Optional[torch.Tensor] = None
    logits: Optional[torch.Tensor] = None
    states: Optional[torch.Tensor] = None
    stats: Optional[Mapping[str, Any]] = None


class FieldsForCausalLM(nn.Module):
    """api:229-318: the public module around the token system."""

    def __init__(self, core_model: FieldTokenSystem, *, backend_name: str,
                 source_audit: Mapping[str, Any], topology_audit: Mapping[str, Any]) -> None:
        super().__init__()
        self.core_model = core_model
        self.backend_name = str(backend_name)
        self.source_audit = dict(source_audit)
        self.topology_audit = dict(topology_audit)

    @property
    def pcaf_enabled(self) -> bool:
        return bool(getattr(self.core_model.cache, "enabled", False))

    @property
    def config_dict(self) -> Dict[str, Any]:
        return {**dict(OFFICIAL_ARCHITECTURE), "pcaf_enabled": self.pcaf_enabled,
                "backend_name": self.backend_name, "topology_audit": self.topology_audit}

    def set_pcaf_enabled(self, enabled: bool) -> None:
        self.core_model.cache.enabled = bool(enabled)

    def forward(self, input_ids: torch.Tensor, labels: Optional[torch.Tensor] = None, *,
                compute_metrics: bool = False, return_states: bool = False) -> FieldsForwardOutput:
        if input_ids.ndim != 2 or input_ids.dtype != torch.long:
            raise TypeError("input_ids must be a rank-2 torch.long tensor [batch, time]")
        if labels is None:
            states, logits = self.core_model.states_logits(input_ids)
            return FieldsForwardOutput(logits=logits, states=states if return_states else None)
        if labels.shape != input_ids.shape or labels.dtype != torch.long:
            raise TypeError("labels must match input_ids shape and use torch.long")
        raise NotImplementedError(
            "loss_and_stats (PCAF routing, training) is not rebuilt: this build is inference only")

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor, max_len: int):
        return self.core_model.prefill(input_ids, max_len)

    @torch.no_grad()
    def step(self, token_t: torch.Tensor, cache) -> torch.Tensor:
        return self.core_model.step(token_t, cache)


def solve_ff_hidden(dim: int = 1024, vocab: int = 16_384, target: int = 300_000_000) -> int:
    """FFN width of the parameter-matched promoted model (r1:263-321): params are affine in the
    width (slope 3 * dim * 22 FFN-carrying blocks); round to a multiple of 32."""
    with torch.device("meta"):
        probe = FieldTokenSystem(vocab=vocab, dim=dim, ff_hidden=2048)
    total = sum(p.numel() for p in probe.parameters())
    ff_blocks = sum(1 for k in probe.kinds() if k != "mamba")
    slope = 3 * dim * ff_blocks
    fixed = total - slope * 2048
    raw = (target - fixed) / slope
    return int(round(raw / FF_MULTIPLE) * FF_MULTIPLE)


def tied_embedding_init(model: FieldTokenSystem, seed: int, std: float = 0.02) -> None:
    """v20:440-447: N(0, 0.02) from a CPU generator seeded with ``seed``, shared with the head."""
    g = torch.Generator(device="cpu").manual_seed(int(seed))
    w = torch.empty(tuple(model.emb.weight.shape), dtype=torch.float32).normal_(0.0, std, generator=g)
    with torch.no_grad():
        model.emb.weight.copy_(w.to(model.emb.weight.device, model.emb.weight.dtype))
    model.lm_head.weight = model.emb.weight


def cast_for_inference(model: nn.Module, dtype: torch.dtype = torch.bfloat16) -> nn.Module:
    """Store the GEMM weights in ``dtype`` (what bf16 autocast computes with) and keep in fp32
    the parameters that the reference always reads in fp32: the Field transition parameters
    (radius_logit, theta) and Mamba-2's A_log, dt_bias, D."""
    keep = ("radius_logit", "theta", "A_log", "dt_bias", ".D")
    for name, p in model.named_parameters():
        if not name.endswith(keep) and p.is_floating_point():
            p.data = p.data.to(dtype)
    return model


def topology_audit(core: FieldTokenSystem) -> Dict[str, Any]:
    """oac:369-400: 24 blocks, 18 Field / 2 Mamba-2 / 4 refresh at the promoted positions."""
    kinds = core.kinds()
    audit = {
        "field": kinds.count("field"), "mamba": kinds.count("mamba"), "refresh": kinds.count("refresh"),
        "mamba_positions": [i for i, k in enumerate(kinds) if k == "mamba"],
        "refresh_positions": [i for i, k in enumerate(kinds) if k == "refresh"],
        "sequence": kinds,
    }
    if (audit["field"], audit["mamba"], audit["refresh"]) != (18, 2, 4) or \
            tuple(audit["mamba_positions"]) != OFFICIAL_ARCHITECTURE["mamba2_positions"] or \
            tuple(audit["refresh_positions"]) != OFFICIAL_ARCHITECTURE["refresh_positions"]:
        raise AssertionError(f"topology mismatch: {audit}")
    return audit


def build_official_fields(config: Optional[FieldsConfig] = None, *,
                          device: Optional[torch.device | str] = None) -> FieldsForCausalLM:
    """api:374-422: the promoted 18F/2M/4R + PCAF model from scratch (random init from the
    config's seeds), topology-audited. Mamba-2 blocks are initialised from their own seed
    offset (v29:397-400), the R1-resized FFNs after them."""
    cfg = config or FieldsConfig()
    dev = torch.device(device if device is not None else ("cuda" if torch.cuda.is_available() else "cpu"))
    ff = solve_ff_hidden()
    torch.manual_seed(int(cfg.model_seed))
    core = FieldTokenSystem(vocab=OFFICIAL_ARCHITECTURE["vocabulary_size"],
                            dim=OFFICIAL_ARCHITECTURE["model_dimension"], ff_hidden=ff,
                            refresh_windows=OFFICIAL_ARCHITECTURE["refresh_windows"],
                            mamba_positions=OFFICIAL_ARCHITECTURE["mamba2_positions"],
                            mamba_seed=int(cfg.model_seed) + 290_400)
    tied_embedding_init(core, cfg.embedding_seed)
    core.cache.enabled = bool(cfg.pcaf_enabled)
    core = core.to(dev)
    audit = topology_audit(core)
    return FieldsForCausalLM(core, backend_name="fields_lm_amd-hip-gfx950", source_audit={"ff_hidden": ff},
                             topology_audit=audit)
