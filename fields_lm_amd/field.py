"""Field recurrence ops and the drop-in Field mixer / block modules (HIP path only).

Reference: src/fields_official/reference/field_only_v4_chunked_triton_wiki100.py ("canon").

* :func:`fused_field_read`      — same call as canon:1108-1123; runs ``fl_scan_forward``.
* :func:`field_scan_norm`       — the scan with the mixer's read_norm fused in (canon:1176-1193
  then canon:300-309), ``fl_scan_norm_forward``.
* :func:`field_decode_step`     — single-token step (no reference counterpart), ``fl_decode_step``;
  :func:`field_decode_norm_step` the same with read_norm fused, ``fl_decode_norm_step``.
* :class:`IndependentVacancyField`, :class:`FieldBlock`, :class:`RMSNorm`,
  :class:`PackedSwiGLU` — same constructor signatures, parameter names, initialisation order
  and forward maths as canon:1131-1221 and canon:300-325, so a reference state_dict loads
  with ``strict=True`` and a seeded construction yields identical parameters.

The scan runs only on a ROCm device through ``libfields_amd.so``. There is no CPU path and no
fallback: a CPU tensor or a missing library raises, as the reference's Triton path does
(canon:923-926).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _native as nat

VAC_MAX = 0.90  # canon:68
BACKENDS = ("reference", "triton", "hip")


# ======================================================================================
# scan ops
# ======================================================================================

def _check_scan_inputs(raw: torch.Tensor, tr: torch.Tensor):
    """Argument checks of canon:923-938, in the same order and with the same exception types."""
    if not raw.is_cuda:
        raise RuntimeError("Chunked Field kernel requires a ROCm (cuda) device")
    if raw.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"raw must be float32 or bfloat16, got {raw.dtype}")
    if raw.ndim != 3:
        raise ValueError(raw.shape)
    batch, length, three_channels = raw.shape
    if three_channels % 3:
        raise ValueError(raw.shape)
    channels = three_channels // 3
    if tr.numel() != channels:
        raise ValueError((raw.shape, tr.shape))
    return batch, length, channels


def _read_code(read_dtype: torch.dtype) -> int:
    if read_dtype == torch.float32:
        return nat.FL_DTYPE_F32
    if read_dtype == torch.bfloat16:
        return nat.FL_DTYPE_BF16
    raise TypeError(f"read must be float32 or bfloat16, got {read_dtype}")


def _scan_call(raw, transition_r, transition_i, gamma, state_in, return_state, out_dtype, launch):
    """Shared argument handling of the scan entry points; ``launch(lib, args)`` makes the call.

    args = (raw, batch, length, channels, tr, ti, gm, sin, sout, out, workspace)."""
    lib = nat.load()
    batch, length, channels = _check_scan_inputs(raw, transition_r)
    if raw.stride(2) != 1:
        raw = raw.contiguous()
    dev = raw.device
    tr = transition_r.detach().to(device=dev, dtype=torch.float32).contiguous()
    ti = transition_i.detach().to(device=dev, dtype=torch.float32).contiguous()
    gm = gamma.detach().to(device=dev, dtype=torch.float32).contiguous()
    if ti.numel() != channels or gm.numel() != channels:
        raise ValueError((raw.shape, transition_i.shape, gamma.shape))
    _read_code(out_dtype)
    out = torch.empty((batch, length, 4 * channels), device=dev, dtype=out_dtype)
    sin = None
    if state_in is not None:
        if state_in.shape != (batch, 2 * channels):
            raise ValueError(f"state_in must be [B, 2C] = {(batch, 2 * channels)}, got {tuple(state_in.shape)}")
        sin = state_in.detach().to(device=dev, dtype=torch.float32).contiguous()
    sout = torch.empty((batch, 2 * channels), device=dev, dtype=torch.float32) if return_state else None
    if batch == 0 or length == 0 or channels == 0:
        if sout is not None:
            sout.copy_(sin if sin is not None else torch.zeros_like(sout))
        return (out, sout) if return_state else out
    ws_bytes = int(lib.fl_scan_workspace_bytes(batch, length, channels))
    workspace = nat.scan_workspace(dev, ws_bytes)
    nat.before_call(workspace, "field scan")
    launch(lib, (raw, batch, length, channels, tr, ti, gm, sin, sout, out, workspace))
    return (out, sout) if return_state else out


def field_scan(raw: torch.Tensor, transition_r: torch.Tensor, transition_i: torch.Tensor,
               gamma: torch.Tensor, state_in: Optional[torch.Tensor] = None,
               return_state: bool = False, algo: int = nat.FL_ALGO_AUTO,
               read_dtype: torch.dtype = torch.float32):
    """Run the HIP scan. Returns ``read`` [B,T,4C] (and the final planar state [B,2C], fp32).

    raw: fp32 or bf16 [B,T,3C] on a ROCm device, channel stride 1 (other strides are passed
    through). state_in: fp32 [B,2C] planar (re | im) or None for the zero state.
    read_dtype: fp32 (the reference's output) or bf16 (the fp32 values rounded to nearest even).
    """
    def launch(lib, a):
        raw_, batch, length, channels, tr, ti, gm, sin, sout, read, ws = a
        code = lib.fl_scan_forward_ex(
            nat.ptr(raw_), nat.dtype_code(raw_.dtype), batch, length, channels,
            raw_.stride(0), raw_.stride(1), nat.ptr(tr), nat.ptr(ti), nat.ptr(gm), nat.ptr(sin),
            nat.ptr(sout), nat.ptr(read), _read_code(read.dtype), nat.ptr(ws), ws.numel(), algo,
            nat.stream_handle(raw_.device))
        nat.check(code, "fl_scan_forward")
        nat.check_waits(ws, "fl_scan_forward")

    return _scan_call(raw, transition_r, transition_i, gamma, state_in, return_state, read_dtype,
                      launch)


def _norm_weight(weight: torch.Tensor, channels: int, device) -> torch.Tensor:
    w = weight.detach().to(device=device, dtype=torch.float32).contiguous()
    if w.numel() != 4 * channels:
        raise ValueError(f"norm weight must have 4C = {4 * channels} entries, got {w.numel()}")
    return w


def field_scan_norm(raw: torch.Tensor, transition_r: torch.Tensor, transition_i: torch.Tensor,
                    gamma: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                    state_in: Optional[torch.Tensor] = None, return_state: bool = False,
                    out_dtype: torch.dtype = torch.float32):
    """``RMSNorm(read)`` of the scan in one launch (canon:1176-1193 then canon:300-309):
    out[b,t,:] = read * rsqrt(mean(read^2) + eps) * weight, with read in fp32 as
    :func:`field_scan` computes it; ``read`` itself is never written to memory.

    weight: [4C] (the mixer's ``read_norm.weight``). out_dtype fp32, or bf16 (the fp32 value
    rounded to nearest even, as bf16 autocast hands it to out_proj). C <= 4096.
    """
    def launch(lib, a):
        raw_, batch, length, channels, tr, ti, gm, sin, sout, out, ws = a
        w = _norm_weight(weight, channels, raw_.device)
        code = lib.fl_scan_norm_forward(
            nat.ptr(raw_), nat.dtype_code(raw_.dtype), batch, length, channels,
            raw_.stride(0), raw_.stride(1), nat.ptr(tr), nat.ptr(ti), nat.ptr(gm), nat.ptr(sin),
            nat.ptr(sout), nat.ptr(w), ctypes.c_float(float(eps)), nat.ptr(out),
            _read_code(out.dtype), nat.ptr(ws), ws.numel(), nat.stream_handle(raw_.device))
        nat.check(code, "fl_scan_norm_forward")
        nat.check_waits(ws, "fl_scan_norm_forward")

    if raw.is_cuda:
        _norm_weight(weight, raw.shape[-1] // 3, raw.device)  # shape check before any launch
    return _scan_call(raw, transition_r, transition_i, gamma, state_in, return_state, out_dtype,
                      launch)


def field_scan_backward(raw: torch.Tensor, transition_r: torch.Tensor, transition_i: torch.Tensor,
                        gamma: torch.Tensor, read: torch.Tensor, grad_read: torch.Tensor,
                        state_in: Optional[torch.Tensor] = None,
                        grad_state_out: Optional[torch.Tensor] = None,
                        return_state_grad: bool = False):
    """Gradients of :func:`field_scan` (``fl_scan_backward``; canon:1020-1105): given the forward's
    fp32 ``read`` and dL/dread (and dL/dstate_out), returns (grad_raw in raw's dtype, grad_tr,
    grad_ti, grad_gamma [C] fp32[, grad_state_in [B,2C]])."""
    lib = nat.load()
    batch, length, channels = _check_scan_inputs(raw, transition_r)
    if raw.stride(2) != 1:
        raw = raw.contiguous()
    dev = raw.device
    if read.shape != (batch, length, 4 * channels) or read.dtype != torch.float32:
        raise ValueError("read must be the forward's fp32 [B, T, 4C] output")
    if grad_read.shape != read.shape:
        raise ValueError("grad_read must match read")
    tr, ti, gm = (t.detach().to(device=dev, dtype=torch.float32).contiguous()
                  for t in (transition_r, transition_i, gamma))
    read = read.detach().contiguous()
    grad_read = grad_read.detach().to(dtype=torch.float32).contiguous()
    sin = None if state_in is None else state_in.detach().to(device=dev, dtype=torch.float32).contiguous()
    gso = None if grad_state_out is None else grad_state_out.detach().to(device=dev, dtype=torch.float32).contiguous()
    for name, t in (("state_in", sin), ("grad_state_out", gso)):
        if t is not None and t.shape != (batch, 2 * channels):
            raise ValueError(f"{name} must be [B, 2C]")
    grad_raw = torch.empty((batch, length, 3 * channels), device=dev, dtype=raw.dtype)
    work = bool(batch and length and channels)
    # the kernels write every element of the parameter gradients and of grad_state_in; zeros only
    # where there is nothing to scan
    alloc = torch.empty if work else torch.zeros
    g_tr, g_ti, g_gm = (alloc(channels, device=dev, dtype=torch.float32) for _ in range(3))
    g_sin = alloc((batch, 2 * channels), device=dev, dtype=torch.float32) if return_state_grad else None
    if work:
        ws_bytes = int(lib.fl_scan_backward_workspace_bytes(batch, length, channels))
        ws = nat.scan_workspace(dev, ws_bytes, "backward")
        nat.before_call(ws, "fl_scan_backward")
        code = lib.fl_scan_backward(
            nat.ptr(raw), nat.dtype_code(raw.dtype), batch, length, channels, raw.stride(0),
            raw.stride(1), nat.ptr(tr), nat.ptr(ti), nat.ptr(gm), nat.ptr(sin), nat.ptr(read),
            nat.ptr(grad_read), nat.ptr(gso), nat.ptr(grad_raw), nat.dtype_code(grad_raw.dtype),
            nat.ptr(g_tr), nat.ptr(g_ti), nat.ptr(g_gm), nat.ptr(g_sin), nat.ptr(ws), ws.numel(),
            nat.stream_handle(dev))
        nat.check(code, "fl_scan_backward")
        nat.check_waits(ws, "fl_scan_backward")
    elif g_sin is not None and gso is not None:
        g_sin.copy_(gso)
    out = (grad_raw, g_tr, g_ti, g_gm)
    return (*out, g_sin) if return_state_grad else out


class _FieldReadFunction(torch.autograd.Function):
    """canon:912-1105 on the HIP path: forward ``fl_scan_forward``, backward ``fl_scan_backward``.

    When a gradient is needed the fp32 ``read`` is what gets saved (the backward reads the states
    in fp32); a bf16 ``read_dtype`` then returns its rounded copy."""

    @staticmethod
    def forward(ctx, raw, transition_r, transition_i, gamma, block_c, chunk_t,
                read_dtype=torch.float32):
        if not any(ctx.needs_input_grad[:4]):
            return field_scan(raw, transition_r, transition_i, gamma, read_dtype=read_dtype)
        read = field_scan(raw, transition_r, transition_i, gamma)
        ctx.save_for_backward(raw, transition_r, transition_i, gamma, read)
        return read if read_dtype == torch.float32 else read.to(read_dtype)

    @staticmethod
    def backward(ctx, grad_read):
        raw, tr, ti, gamma, read = ctx.saved_tensors
        grad_raw, g_tr, g_ti, g_gm = field_scan_backward(raw, tr, ti, gamma, read, grad_read)
        return grad_raw, g_tr.to(tr.dtype), g_ti.to(ti.dtype), g_gm.to(gamma.dtype), None, None, None


class _FieldNormReadFunction(torch.autograd.Function):
    """Forward of read_norm(fused_field_read(...)) on the HIP path, for inference: the fused
    epilogue never writes ``read``, so there is nothing to differentiate through (the modules
    take the unfused path whenever a gradient is needed)."""

    @staticmethod
    def forward(ctx, raw, transition_r, transition_i, gamma, weight, eps, out_dtype):
        return field_scan_norm(raw, transition_r, transition_i, gamma, weight, eps,
                               out_dtype=out_dtype)

    @staticmethod
    def backward(ctx, *grad_outputs):
        raise NotImplementedError(
            "the fused read_norm scan never writes read, so it has no backward: with gradients "
            "enabled the modules run fused_field_read (backward fl_scan_backward) and the RMSNorm "
            "module instead")


def fused_field_read(raw: torch.Tensor, transition_r: torch.Tensor, transition_i: torch.Tensor,
                     gamma: torch.Tensor, block_c: int = 32, chunk_t: int = 64, *,
                     read_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Drop-in for canon:1108-1123 ``fused_field_read``.

    ``block_c`` / ``chunk_t`` are the Triton kernels' tile sizes; they do not change the result
    and are accepted for call compatibility. The HIP kernels choose their own tiling.
    Unlike the reference, bf16 ``raw`` is accepted as well (upcast in-register, exactly), and
    ``read_dtype=torch.bfloat16`` returns the same values rounded to bf16.
    """
    return _FieldReadFunction.apply(raw, transition_r, transition_i, gamma, block_c, chunk_t,
                                    read_dtype)


def field_decode_step(raw_t: torch.Tensor, transition_r: torch.Tensor, transition_i: torch.Tensor,
                      gamma: torch.Tensor, state: torch.Tensor,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One recurrent step: ``state`` (fp32 [B,2C] planar) is updated in place; returns read_t
    fp32 [B,4C]. Equal to row t of :func:`field_scan` when ``state`` holds s[t-1].

    Static shapes, no host synchronisation: capturable in a HIP graph.
    """
    lib = nat.load()
    if not raw_t.is_cuda:
        raise RuntimeError("Field decode step requires a ROCm (cuda) device")
    if raw_t.ndim != 2 or raw_t.shape[1] % 3:
        raise ValueError(raw_t.shape)
    batch, channels = raw_t.shape[0], raw_t.shape[1] // 3
    if transition_r.numel() != channels:
        raise ValueError((raw_t.shape, transition_r.shape))
    if raw_t.stride(1) != 1:
        raw_t = raw_t.contiguous()
    if state.shape != (batch, 2 * channels) or state.dtype != torch.float32 or not state.is_contiguous():
        raise ValueError("state must be a contiguous fp32 [B, 2C] tensor")
    for p in (transition_r, transition_i, gamma):
        if p.dtype != torch.float32 or not p.is_contiguous() or p.device != raw_t.device:
            raise ValueError("transition_r/transition_i/gamma must be contiguous fp32 on the raw device")
    if out is None:
        out = torch.empty((batch, 4 * channels), device=raw_t.device, dtype=torch.float32)
    code = lib.fl_decode_step(nat.ptr(raw_t), nat.dtype_code(raw_t.dtype), batch, channels,
                              raw_t.stride(0), nat.ptr(transition_r), nat.ptr(transition_i),
                              nat.ptr(gamma), nat.ptr(state), nat.ptr(out), nat.FL_DTYPE_F32,
                              nat.stream_handle(raw_t.device))
    nat.check(code, "fl_decode_step")
    return out


def field_decode_norm_step(raw_t: torch.Tensor, transition_r: torch.Tensor,
                           transition_i: torch.Tensor, gamma: torch.Tensor, state: torch.Tensor,
                           weight: torch.Tensor, eps: float = 1e-6,
                           out: Optional[torch.Tensor] = None,
                           out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """:func:`field_decode_step` with read_norm fused: ``state`` advances in place and the
    result is RMSNorm(read_t) [B,4C] (``weight`` [4C] fp32 on the device). Capturable."""
    lib = nat.load()
    if not raw_t.is_cuda:
        raise RuntimeError("Field decode step requires a ROCm (cuda) device")
    if raw_t.ndim != 2 or raw_t.shape[1] % 3:
        raise ValueError(raw_t.shape)
    batch, channels = raw_t.shape[0], raw_t.shape[1] // 3
    if transition_r.numel() != channels:
        raise ValueError((raw_t.shape, transition_r.shape))
    if raw_t.stride(1) != 1:
        raw_t = raw_t.contiguous()
    if state.shape != (batch, 2 * channels) or state.dtype != torch.float32 or not state.is_contiguous():
        raise ValueError("state must be a contiguous fp32 [B, 2C] tensor")
    for p in (transition_r, transition_i, gamma, weight):
        if p.dtype != torch.float32 or not p.is_contiguous() or p.device != raw_t.device:
            raise ValueError("transition_r/transition_i/gamma/weight must be contiguous fp32 on the raw device")
    if weight.numel() != 4 * channels:
        raise ValueError(f"norm weight must have 4C = {4 * channels} entries, got {weight.numel()}")
    if out is None:
        out = torch.empty((batch, 4 * channels), device=raw_t.device, dtype=out_dtype)
    if out.shape != (batch, 4 * channels) or not out.is_contiguous():
        raise ValueError("out must be a contiguous [B, 4C] tensor")
    code = lib.fl_decode_norm_step(nat.ptr(raw_t), nat.dtype_code(raw_t.dtype), batch, channels,
                                   raw_t.stride(0), nat.ptr(transition_r), nat.ptr(transition_i),
                                   nat.ptr(gamma), nat.ptr(state), nat.ptr(weight),
                                   ctypes.c_float(float(eps)), nat.ptr(out), _read_code(out.dtype),
                                   nat.stream_handle(raw_t.device))
    nat.check(code, "fl_decode_norm_step")
    return out


def boundary_scan(a: torch.Tensor, drive: torch.Tensor, state_in: Optional[torch.Tensor] = None,
                  return_state: bool = False):
    """Softpatch boundary scan on the HIP path: s[b,t,:] = a[b,t] * s[b,t-1,:] + drive[b,t,:]
    (``hierarchical_scan(a, drive, 32)`` of v3:458-460 with ``a`` one value per token).

    a [B,T] fp32, drive [B,T,R] fp32, state_in [B,R] or None. Returns s [B,T,R] (and s[:,T-1]).
    """
    lib = nat.load()
    if not (a.is_cuda and drive.is_cuda):
        raise RuntimeError("the boundary scan requires a ROCm (cuda) device")
    if drive.ndim != 3 or a.shape != drive.shape[:2]:
        raise ValueError((tuple(a.shape), tuple(drive.shape)))
    if a.dtype != torch.float32 or drive.dtype != torch.float32:
        raise TypeError("a and drive must be float32")
    a, drive = a.contiguous(), drive.contiguous()
    batch, length, rank = drive.shape
    out = torch.empty_like(drive)
    sout = torch.empty((batch, rank), device=drive.device, dtype=torch.float32) if return_state else None
    sin = None
    if state_in is not None:
        if state_in.shape != (batch, rank):
            raise ValueError(f"state_in must be [B, R] = {(batch, rank)}")
        sin = state_in.detach().to(device=drive.device, dtype=torch.float32).contiguous()
    if batch == 0 or length == 0 or rank == 0:
        if sout is not None:
            sout.copy_(sin if sin is not None else torch.zeros_like(sout))
        return (out, sout) if return_state else out
    code = lib.fl_boundary_scan(nat.ptr(a), nat.ptr(drive), batch, length, rank, nat.ptr(sin),
                                nat.ptr(sout), nat.ptr(out), nat.stream_handle(drive.device))
    nat.check(code, "fl_boundary_scan")
    return (out, sout) if return_state else out


def _row_stride(t: torch.Tensor) -> Optional[int]:
    """Element distance between consecutive rows of ``t`` viewed as [rows, t.shape[-1]] when its
    last dimension is unit-stride and every leading dimension steps whole rows (a column slice of
    a contiguous tensor); None otherwise."""
    if t.ndim == 0 or t.stride(-1) != 1:
        return None
    if t.ndim == 1:
        return t.shape[-1]
    rs = t.stride(-2)
    if rs < t.shape[-1]:
        return None
    step = rs
    for i in range(t.ndim - 2, 0, -1):
        step *= t.shape[i]
        if t.shape[i - 1] > 1 and t.stride(i - 1) != step:
            return None
    return rs


def gate_residual_norm(x: torch.Tensor, out: torch.Tensor, gate_pre: torch.Tensor,
                       weight: torch.Tensor, eps: float = 1e-6) -> Tuple[torch.Tensor, torch.Tensor]:
    """``x + out * sigmoid(gate_pre)`` and its RMSNorm (``fl_gate_residual_norm``): the mixer's
    gated residual (canon:1193-1195) and the block's ``ff_norm`` (canon:1219-1221) in one launch,
    rounded as the stock ops round. x: residual stream (fp32 / bf16); out, gate_pre: the out_proj /
    gate_proj outputs; all [..., dim] on one device. ``gate_pre`` may be a column slice of a wider
    GEMM output (rows a fixed stride apart); the others are made contiguous. Returns (x_new,
    normed) in x's dtype."""
    lib = nat.load()
    if not x.is_cuda:
        raise RuntimeError("gate_residual_norm requires a ROCm (cuda) device")
    if out.shape != x.shape or gate_pre.shape != x.shape or out.dtype != gate_pre.dtype:
        raise ValueError("x, out and gate_pre must have one shape; out and gate_pre one dtype")
    dim = x.shape[-1]
    if weight.numel() != dim:
        raise ValueError("weight must have dim entries")
    x, out = x.contiguous(), out.contiguous()
    gate_stride = _row_stride(gate_pre)
    if gate_stride is None:
        gate_pre = gate_pre.contiguous()
        gate_stride = dim
    w = weight.detach().to(device=x.device, dtype=torch.float32).contiguous()
    x_new, normed = torch.empty_like(x), torch.empty_like(x)
    rows = x.numel() // dim if dim else 0
    if rows == 0:
        return x_new, normed
    code = lib.fl_gate_residual_norm(nat.ptr(x), nat.dtype_code(x.dtype), nat.ptr(out), nat.ptr(gate_pre),
                                     nat.dtype_code(out.dtype), rows, dim, gate_stride, nat.ptr(w),
                                     ctypes.c_float(float(eps)), nat.ptr(x_new), nat.ptr(normed),
                                     nat.stream_handle(x.device))
    nat.check(code, "fl_gate_residual_norm")
    return x_new, normed


def swiglu(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up with [gate | up] = gate_up [..., 2H] (``fl_swiglu``; canon:323-325)."""
    lib = nat.load()
    if not gate_up.is_cuda:
        raise RuntimeError("swiglu requires a ROCm (cuda) device")
    if gate_up.shape[-1] % 2:
        raise ValueError("the last dimension must be even")
    gate_up = gate_up.contiguous()
    hidden = gate_up.shape[-1] // 2
    out = torch.empty((*gate_up.shape[:-1], hidden), device=gate_up.device, dtype=gate_up.dtype)
    rows = gate_up.numel() // (2 * hidden) if hidden else 0
    if rows == 0:
        return out
    code = lib.fl_swiglu(nat.ptr(gate_up), nat.dtype_code(gate_up.dtype), rows, hidden, nat.ptr(out),
                         nat.stream_handle(gate_up.device))
    nat.check(code, "fl_swiglu")
    return out


def state_to_complex(state: torch.Tensor) -> torch.Tensor:
    """Planar [B,2C] fp32 state -> complex64 [B,C]."""
    c = state.shape[-1] // 2
    return torch.complex(state[..., :c], state[..., c:])


# ======================================================================================
# modules (canon:300-325, 1131-1221)
# ======================================================================================

class RMSNorm(nn.Module):
    """canon:300-309: fp32 normalisation, result cast back to the input dtype."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        y = xf * torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


class PackedSwiGLU(nn.Module):
    """canon:312-325: w12 packs (gate, value); out = w3(silu(gate) * value)."""

    def __init__(self, dim: int, hidden: Optional[int] = None):
        super().__init__()
        self.hidden = int(hidden) if hidden is not None else ((int(8 * dim / 3) + 63) // 64) * 64
        self.w12 = nn.Linear(dim, 2 * self.hidden, bias=False)
        self.w3 = nn.Linear(self.hidden, dim, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, value = self.w12(x).chunk(2, dim=-1)
        return self.w3(F.silu(gate) * value)


class IndependentVacancyField(nn.Module):
    """Zero-attention Field mixer with independent vacancy and displaced readout (canon:1131-1195).

    Every backend name of the reference is accepted ("reference", "triton"; plus "hip"); all
    of them run the HIP scan, the one implementation this package has.
    """

    def __init__(self, dim: int, backend: str, field_chunk: int, triton_block_c: int,
                 triton_chunk_t: int):
        super().__init__()
        if dim % 2:
            raise ValueError("Field dim must be even")
        if backend not in BACKENDS:
            raise ValueError(backend)
        self.dim = dim
        self.channels = dim // 2
        self.backend = backend
        self.field_chunk = int(field_chunk)
        self.triton_block_c = int(triton_block_c)
        self.triton_chunk_t = int(triton_chunk_t)
        # parameter creation order fixes the RNG stream: write_proj, out_proj, gate_proj
        self.write_proj = nn.Linear(dim, dim + self.channels)
        ring = torch.linspace(0.85, 0.999, self.channels)
        self.radius_logit = nn.Parameter(torch.log(ring / (1.0 - ring)))
        self.theta = nn.Parameter(torch.linspace(0.03, math.pi * 0.97, self.channels))
        self.read_norm = RMSNorm(2 * dim)
        self.out_proj = nn.Linear(2 * dim, dim)
        self.gate_proj = nn.Linear(dim, dim)
        # dtype of what the fused scan hands to out_proj. "auto": bf16 when raw is bf16 (bf16
        # autocast, whose out_proj casts its input to bf16 anyway), else fp32; or a fixed torch
        # dtype. The unfused path (and every path that needs a gradient) keeps read in fp32 under
        # "auto", as the reference does (canon:1168, 1193). Not a parameter or buffer:
        # state_dict is unchanged.
        self.read_dtype = "auto"
        # True: read_norm runs inside the scan kernel (fl_scan_norm_forward /
        # fl_decode_norm_step) and the fp32 read never reaches memory; False: the scan writes
        # read and read_norm runs as a separate module call, as in the reference.
        self.fuse_read_norm = True
        # True: without gradients, write_proj and gate_proj run as one GEMM (in_proj). Not a
        # parameter or buffer: state_dict is unchanged.
        self.fuse_in_proj = True
        self._packed = None  # (key, weight, bias) of the stacked projections

    def transition(self) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(tr, ti, gamma) fp32 [C] (canon:1169-1173), computed in the parameters' dtype."""
        radius = torch.sigmoid(self.radius_logit).clamp(0.50, 0.99995).float()
        theta = self.theta.float()
        tr = radius * torch.cos(theta)
        ti = radius * torch.sin(theta)
        gamma = torch.sqrt((1.0 - radius.square()).clamp_min(1e-4))
        return tr.contiguous(), ti.contiguous(), gamma.contiguous()

    def _raw(self, x: torch.Tensor, raw: Optional[torch.Tensor] = None) -> torch.Tensor:
        # bf16 (autocast) and fp32 raw go to the kernel as they are; the kernel's upcast of
        # bf16 is exact, so this equals the reference's `.contiguous().float()` copy.
        if raw is None:
            raw = self.write_proj(x)
        if raw.dtype not in (torch.float32, torch.bfloat16):
            raw = raw.float()
        return raw

    def _no_grad(self, x: torch.Tensor) -> bool:
        return not (torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())))

    def in_proj(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """(raw, gate_pre) = (write_proj(x), gate_proj(x)). Without gradients the two run as one
        GEMM over their weights stacked ([write_proj; gate_proj], a packed copy rebuilt whenever a
        weight or bias changes): raw and gate_pre are column slices of its output, which the scan,
        the decode step and the fused tail read in place (row stride dim + C + dim)."""
        if not (self.fuse_in_proj and self._no_grad(x)) or self.write_proj.bias is None \
                or self.gate_proj.bias is None:
            return self.write_proj(x), self.gate_proj(x)
        w, b = self._packed_in_proj()
        y = F.linear(x, w, b)
        n = self.write_proj.out_features
        return y[..., :n], y[..., n:]

    def _packed_in_proj(self) -> Tuple[torch.Tensor, torch.Tensor]:
        srcs = (self.write_proj.weight, self.write_proj.bias, self.gate_proj.weight, self.gate_proj.bias)
        key = tuple((id(t), t.data_ptr(), t._version, t.dtype, t.device) for t in srcs)
        if self._packed is None or self._packed[0] != key:
            with torch.no_grad():
                w = torch.cat([srcs[0], srcs[2]], 0)
                b = torch.cat([srcs[1], srcs[3]], 0)
            self._packed = (key, w, b)
        return self._packed[1], self._packed[2]

    def _project(self, x: torch.Tensor, normed: torch.Tensor) -> torch.Tensor:
        out = self.out_proj(normed)
        gate = torch.sigmoid(self.gate_proj(x))
        return x + (out * gate).to(x.dtype)

    def _fused(self, x: Optional[torch.Tensor] = None) -> bool:
        """read_norm inside the scan kernel: inference only (no gradient needed), the reference's
        RMSNorm module, C <= 4096."""
        if not (self.fuse_read_norm and type(self.read_norm) is RMSNorm and self.channels <= 4096):
            return False
        if torch.is_grad_enabled() and ((x is not None and x.requires_grad)
                                        or any(p.requires_grad for p in self.parameters())):
            return False
        return True

    def _read_dtype(self, raw: torch.Tensor) -> torch.dtype:
        """Output dtype of the fused scan + read_norm."""
        if self.read_dtype == "auto":
            return torch.bfloat16 if raw.dtype == torch.bfloat16 else torch.float32
        return self.read_dtype

    def _unfused_read_dtype(self) -> torch.dtype:
        """dtype of ``read`` when read_norm runs as a separate module: fp32 under "auto" (the
        reference's read, canon:1168-1193), so RMSNorm normalises, and its backward
        differentiates, the fp32 values."""
        return torch.float32 if self.read_dtype == "auto" else self.read_dtype

    def normed_read(self, x: torch.Tensor, raw: Optional[torch.Tensor] = None) -> torch.Tensor:
        """read_norm(read) of the scan of x: what out_proj consumes (``raw`` = write_proj(x) when
        already computed)."""
        tr, ti, gamma = self.transition()
        raw = self._raw(x, raw)
        if self._fused(x):
            return _FieldNormReadFunction.apply(raw, tr, ti, gamma, self.read_norm.weight,
                                                self.read_norm.eps, self._read_dtype(raw))
        read = fused_field_read(raw, tr, ti, gamma, self.triton_block_c, self.triton_chunk_t,
                                read_dtype=self._unfused_read_dtype())
        return self.read_norm(read)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self._project(x, self.normed_read(x))

    def normed_prefill(self, x: torch.Tensor, state: Optional[torch.Tensor] = None,
                       raw: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """read_norm(read) over [B,T,dim] and the recurrent state s[T-1] (fp32 [B,2C])."""
        tr, ti, gamma = self.transition()
        raw = self._raw(x, raw)
        if self._fused(x):
            return field_scan_norm(raw, tr, ti, gamma, self.read_norm.weight, self.read_norm.eps,
                                   state_in=state, return_state=True, out_dtype=self._read_dtype(raw))
        read, new_state = field_scan(raw, tr, ti, gamma, state_in=state, return_state=True,
                                     read_dtype=self._unfused_read_dtype())
        return self.read_norm(read), new_state

    def prefill(self, x: torch.Tensor, state: Optional[torch.Tensor] = None
                ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Forward over [B,T,dim] that also returns the recurrent state s[T-1] (fp32 [B,2C]).

        ``state`` continues a previous segment (state_in); None starts from zero as forward does.
        """
        normed, new_state = self.normed_prefill(x, state)
        return self._project(x, normed), new_state

    def decode_params(self) -> Tuple[torch.Tensor, ...]:
        """(tr, ti, gamma, read_norm weight in fp32): what :meth:`step` reads, cached once per
        decode loop."""
        return (*self.transition(), self.read_norm.weight.detach().float().contiguous())

    def step(self, x_t: torch.Tensor, state: torch.Tensor,
             params: Optional[Tuple[torch.Tensor, ...]] = None) -> torch.Tensor:
        """One decode token: x_t [B,dim] -> [B,dim]; ``state`` [B,2C] fp32 is advanced in place.

        ``params`` = a cached ``self.transition()`` or ``self.decode_params()`` (recomputed when
        None).
        """
        return self._project(x_t, self.normed_step(x_t, state, params))

    def normed_step(self, x_t: torch.Tensor, state: torch.Tensor,
                    params: Optional[Tuple[torch.Tensor, ...]] = None,
                    raw_t: Optional[torch.Tensor] = None) -> torch.Tensor:
        """read_norm(read_t) of one decode token; ``state`` advances in place."""
        params = params if params is not None else self.decode_params()
        tr, ti, gamma = params[:3]
        raw_t = self._raw(x_t, raw_t)
        if self._fused(x_t):
            w = params[3] if len(params) > 3 else self.read_norm.weight.detach().float().contiguous()
            return field_decode_norm_step(raw_t, tr, ti, gamma, state, w, self.read_norm.eps,
                                          out_dtype=self._read_dtype(raw_t))
        return self.read_norm(field_decode_step(raw_t, tr, ti, gamma, state))

    def new_state(self, batch: int, device=None) -> torch.Tensor:
        return torch.zeros((batch, 2 * self.channels), device=device, dtype=torch.float32)


class FieldBlock(nn.Module):
    """canon:1198-1221: x = mixer(x) (residual inside); x + ff(ff_norm(x))."""

    def __init__(self, dim: int, backend: str, field_chunk: int, triton_block_c: int,
                 triton_chunk_t: int, ff_hidden: int):
        super().__init__()
        self.mixer = IndependentVacancyField(dim, backend, field_chunk, triton_block_c, triton_chunk_t)
        self.ff_norm = RMSNorm(dim)
        self.ff = PackedSwiGLU(dim, hidden=ff_hidden)
        # True: the elementwise tail runs fused (fl_gate_residual_norm, fl_swiglu) when no
        # gradient is needed. Not a parameter or buffer: state_dict is unchanged.
        self.fuse_tail = True

    # The elementwise tail (gated residual, ff_norm, SwiGLU activation) runs in two fused launches
    # on the inference path (no gradient needed); the GEMMs stay stock.
    def _fused_tail(self, x: torch.Tensor) -> bool:
        if not self.fuse_tail or type(self.ff_norm) is not RMSNorm:
            return False
        if not (hasattr(self.ff, "w12") or hasattr(self.ff, "gate_up")):
            return False
        return not (torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())))

    def _tail(self, x: torch.Tensor, normed: torch.Tensor, gate_pre: torch.Tensor) -> torch.Tensor:
        m = self.mixer
        x1, h = gate_residual_norm(x, m.out_proj(normed), gate_pre, self.ff_norm.weight, self.ff_norm.eps)
        first, second = (self.ff.w12, self.ff.w3) if hasattr(self.ff, "w12") else (self.ff.gate_up, self.ff.down)
        return x1 + second(swiglu(first(h)))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._fused_tail(x):
            raw, gate_pre = self.mixer.in_proj(x)
            return self._tail(x, self.mixer.normed_read(x, raw), gate_pre)
        x = self.mixer(x)
        return x + self.ff(self.ff_norm(x))

    def prefill(self, x: torch.Tensor, state: Optional[torch.Tensor] = None
                ) -> Tuple[torch.Tensor, torch.Tensor]:
        if self._fused_tail(x):
            raw, gate_pre = self.mixer.in_proj(x)
            normed, state = self.mixer.normed_prefill(x, state, raw)
            return self._tail(x, normed, gate_pre), state
        x, state = self.mixer.prefill(x, state)
        return x + self.ff(self.ff_norm(x)), state

    def step(self, x_t: torch.Tensor, state: torch.Tensor, params=None) -> torch.Tensor:
        if self._fused_tail(x_t):
            raw_t, gate_pre = self.mixer.in_proj(x_t)
            return self._tail(x_t, self.mixer.normed_step(x_t, state, params, raw_t), gate_pre)
        x_t = self.mixer.step(x_t, state, params)
        return x_t + self.ff(self.ff_norm(x_t))


class ScanPlan:
    """Pre-bound ``fl_scan_forward`` call for a fixed raw tensor: output, state and workspace are
    allocated once, so :meth:`run` is one C call (no allocation; capturable in a HIP graph).

    ``raw`` may be refilled in place between runs; ``read`` and ``state_out`` are overwritten.
    With ``norm_weight`` [4C], ``read`` receives RMSNorm(read) (``fl_scan_norm_forward``).
    """

    def __init__(self, raw: torch.Tensor, transition_r: torch.Tensor, transition_i: torch.Tensor,
                 gamma: torch.Tensor, state_in: Optional[torch.Tensor] = None,
                 algo: int = nat.FL_ALGO_AUTO, read_dtype: torch.dtype = torch.float32,
                 norm_weight: Optional[torch.Tensor] = None, eps: float = 1e-6):
        self.algo = algo
        self.lib = nat.load()
        batch, length, channels = _check_scan_inputs(raw, transition_r)
        if raw.stride(2) != 1:
            raise ValueError("raw must have channel stride 1")
        if batch == 0 or length == 0 or channels == 0:
            raise ValueError("ScanPlan needs a non-empty raw tensor")
        dev = raw.device
        self.raw = raw
        self.params = [t.detach().to(device=dev, dtype=torch.float32).contiguous()
                       for t in (transition_r, transition_i, gamma)]
        self.state_in = None if state_in is None else state_in.detach().float().contiguous()
        self.read = torch.empty((batch, length, 4 * channels), device=dev, dtype=read_dtype)
        self.state_out = torch.empty((batch, 2 * channels), device=dev, dtype=torch.float32)
        self.ws_bytes = int(self.lib.fl_scan_workspace_bytes(batch, length, channels))
        self.workspace = torch.zeros(self.ws_bytes, device=dev, dtype=torch.uint8)  # zero-filled once
        nat.guard_workspace(self.workspace, fresh=True)
        head = (nat.ptr(raw), nat.dtype_code(raw.dtype), batch, length, channels, raw.stride(0),
                raw.stride(1), *[nat.ptr(p) for p in self.params], nat.ptr(self.state_in),
                nat.ptr(self.state_out))
        if norm_weight is None:
            self.norm_weight = None
            self.fn, self.name = self.lib.fl_scan_forward_ex, "fl_scan_forward"
            self.args = head + (nat.ptr(self.read), _read_code(read_dtype), nat.ptr(self.workspace),
                                self.ws_bytes, algo)
        else:
            self.norm_weight = _norm_weight(norm_weight, channels, dev)
            self.fn, self.name = self.lib.fl_scan_norm_forward, "fl_scan_norm_forward"
            self.args = head + (nat.ptr(self.norm_weight), ctypes.c_float(float(eps)),
                                nat.ptr(self.read), _read_code(read_dtype), nat.ptr(self.workspace),
                                self.ws_bytes)
        self.device = dev

    def run(self, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        nat.before_call(self.workspace, self.name)
        code = self.fn(*self.args, ctypes.c_void_p(s.cuda_stream))
        nat.check(code, self.name)
        nat.check_waits(self.workspace, self.name)
        return self.read
