"""TEST INFRASTRUCTURE ONLY — torch restatement of the reference's CPU Field path.

Used by the tests as a second, independent checker (hierarchical complex64 scan vs the
sequential float64 C oracle) and by ``bench.py`` as the timed CPU baseline (``kind: "port"``).
Never imported by the product package.

Each function restates, in its own code, the operation sequence of
src/fields_official/reference/field_only_v4_chunked_triton_wiki100.py (``canon``):

* :func:`doubling_scan`     — ``assoc_scan``           canon:333-344
* :func:`blocked_scan`      — ``hierarchical_scan``    canon:347-389
* :func:`field_read`        — ``reference_field_read`` canon:392-416
* :func:`transition_params` — parameter transform in ``IndependentVacancyField.forward`` canon:1169-1173
* :func:`rms_norm`          — ``RMSNorm.forward``      canon:306-309
* :func:`mixer_forward`     — ``IndependentVacancyField.forward`` canon:1167-1195 (reference backend)
* :func:`block_forward`     — ``FieldBlock.forward``   canon:1219-1221 with ``PackedSwiGLU`` canon:323-325
"""
from __future__ import annotations

import math
from typing import Mapping, Tuple

import torch
import torch.nn.functional as F

VACANCY_MAX = 0.90  # canon:68


def _shift_right(x: torch.Tensor, step: int, fill: float) -> torch.Tensor:
    """x shifted by ``step`` along dim 1, the vacated front filled with ``fill``."""
    out = torch.full_like(x, fill)
    out[:, step:] = x[:, :-step]
    return out


def doubling_scan(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Inclusive scan of s_t = a_t*s_{t-1} + b_t (s_{-1} = 0) along dim 1 by recursive doubling.

    After the pass with shift d, (a_t, b_t) holds the composition of the maps t-2d+1 .. t.
    """
    a = a.clone()
    b = b.clone()
    n = a.shape[1]
    step = 1
    while step < n:
        a_prev = _shift_right(a, step, 1.0)
        b_prev = _shift_right(b, step, 0.0)
        b = a * b_prev + b
        a = a * a_prev
        step *= 2
    return b


def blocked_scan(a: torch.Tensor, b: torch.Tensor, block: int = 32) -> torch.Tensor:
    """Two-level scan: doubling inside blocks of ``block`` steps, then across block tails.

    a, b: complex [B, T, C]. Padding steps are identity maps (a = 1, b = 0).
    """
    if block < 1 or block > 64:
        raise ValueError("field_chunk must be in [1, 64]")
    bsz, length, ch = a.shape
    pad = (-length) % block
    if pad:
        a = torch.cat((a, torch.ones((bsz, pad, ch), dtype=a.dtype)), dim=1)
        b = torch.cat((b, torch.zeros((bsz, pad, ch), dtype=b.dtype)), dim=1)
    groups = a.shape[1] // block
    la = a.reshape(bsz * groups, block, ch).clone()
    lb = b.reshape(bsz * groups, block, ch).clone()
    step = 1
    while step < block:
        a_prev = _shift_right(la, step, 1.0)
        b_prev = _shift_right(lb, step, 0.0)
        lb = la * b_prev + lb
        la = la * a_prev
        step *= 2
    la = la.reshape(bsz, groups, block, ch)
    lb = lb.reshape(bsz, groups, block, ch)
    tail_state = doubling_scan(la[:, :, -1], lb[:, :, -1])  # state after each block
    carry = torch.zeros_like(tail_state)
    carry[:, 1:] = tail_state[:, :-1]
    states = la * carry[:, :, None, :] + lb
    return states.reshape(bsz, groups * block, ch)[:, :length]


def field_read(raw: torch.Tensor, tr: torch.Tensor, ti: torch.Tensor, gamma: torch.Tensor,
               field_chunk: int = 32) -> torch.Tensor:
    """raw fp32 [B,T,3C] -> read fp32 [B,T,4C] = [Re s | Im s | Re disp | Im disp]."""
    ch = tr.numel()
    inj = torch.complex(torch.tanh(raw[..., :ch]), torch.tanh(raw[..., ch:2 * ch]))
    vac = torch.sigmoid(raw[..., 2 * ch:]) * VACANCY_MAX
    lam = torch.complex(tr, ti)
    vac_c = vac.to(torch.complex64)
    a = (1.0 - vac).to(torch.complex64) * lam
    b = gamma.to(torch.complex64) * vac_c * inj
    states = blocked_scan(a, b, field_chunk)
    prev = torch.zeros_like(states)
    prev[:, 1:] = states[:, :-1]
    disp = vac_c * (lam * prev)
    return torch.cat((states.real, states.imag, disp.real, disp.imag), dim=-1)


def transition_params(radius_logit: torch.Tensor, theta: torch.Tensor
                      ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(tr, ti, gamma) from the mixer parameters, in the parameters' dtype then fp32."""
    radius = torch.sigmoid(radius_logit).clamp(0.50, 0.99995).float()
    th = theta.float()
    tr = radius * torch.cos(th)
    ti = radius * torch.sin(th)
    gamma = torch.sqrt((1.0 - radius.square()).clamp_min(1e-4))
    return tr, ti, gamma


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    xf = x.float()
    y = xf * torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return (y * weight.float()).to(x.dtype)


def mixer_forward(p: Mapping[str, torch.Tensor], x: torch.Tensor, prefix: str = "mixer.",
                  field_chunk: int = 32, return_read: bool = False):
    """Field mixer forward from a state_dict ``p`` (keys ``{prefix}write_proj.weight`` ...)."""
    g = lambda k: p[prefix + k]  # noqa: E731
    raw = F.linear(x, g("write_proj.weight"), g("write_proj.bias")).contiguous().float()
    tr, ti, gamma = transition_params(g("radius_logit"), g("theta"))
    read = field_read(raw, tr, ti, gamma, field_chunk)
    out = F.linear(rms_norm(read, g("read_norm.weight")), g("out_proj.weight"), g("out_proj.bias"))
    gate = torch.sigmoid(F.linear(x, g("gate_proj.weight"), g("gate_proj.bias")))
    y = x + (out * gate).to(x.dtype)
    return (y, read) if return_read else y


def block_forward(p: Mapping[str, torch.Tensor], x: torch.Tensor, field_chunk: int = 32,
                  return_read: bool = False):
    """FieldBlock forward: mixer (with its own residual), then x + SwiGLU(RMSNorm(x))."""
    x, read = mixer_forward(p, x, "mixer.", field_chunk, return_read=True)
    h = rms_norm(x, p["ff_norm.weight"])
    gate, value = F.linear(h, p["ff.w12.weight"]).chunk(2, dim=-1)
    y = x + F.linear(F.silu(gate) * value, p["ff.w3.weight"])
    return (y, read) if return_read else y


def init_radius_theta(channels: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Deterministic mixer init (canon:1156-1160)."""
    ring = torch.linspace(0.85, 0.999, channels)
    return torch.log(ring / (1.0 - ring)), torch.linspace(0.03, math.pi * 0.97, channels)
