"""TEST INFRASTRUCTURE ONLY — the CPU oracle of the Field recurrence.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker (or the timed CPU baseline), never as the measured or
shipped path. The product (``fields_lm_amd``) never imports it.

Contents
--------
* :func:`scan_f64` / :func:`decode_step_f64` — float64 sequential recurrence in plain C
  (``field_oracle.c``), following ``reference_field_read``
  (src/fields_official/reference/field_only_v4_chunked_triton_wiki100.py:392-416).
* :func:`rms_norm_f64` — float64 ``RMSNorm`` (same file, 300-309), the mixer's ``read_norm``
  applied to ``read`` (1193): the checker of the fused scan epilogue.
* :func:`scan_f64_autograd` — the same recurrence as differentiable float64 torch ops
  (complex128 doubling scan), whose autograd gradients are the checker of the backward scan
  (``_ChunkedFieldReadFunction.backward``, same file 1020-1105).
* :mod:`oracle.reference_path` — op-for-op torch restatement of the reference's CPU path
  (``assoc_scan`` / ``hierarchical_scan`` / ``reference_field_read``, same file 333-416) and of
  the Field mixer / block forward (1131-1221, 300-325). Also the timed CPU baseline.

Pinning (tests/test_oracle.py): closed forms (T = 1, scipy.signal.lfilter for constant
vacancy, geometric series), invariants (chunk-size independence, state continuation,
``s_t + disp_t = lam*s_{t-1} + b_t``, causality), the two restatements against each other, and
the golden fixtures of tests/golden/ written from the reference's own CPU path.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Optional, Tuple

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
C_SOURCE = ORACLE_DIR / "field_oracle.c"
LIB_PATH = ORACLE_DIR / "_build" / "libfield_oracle.so"

_lib = None


def build() -> Path:
    """Compile field_oracle.c with gcc into oracle/_build/libfield_oracle.so."""
    LIB_PATH.parent.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fno-fast-math", str(C_SOURCE), "-o", str(tmp), "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"gcc failed:\n{proc.stdout}\n{proc.stderr}")
    tmp.replace(LIB_PATH)
    return LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < C_SOURCE.stat().st_mtime:
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    dp = ctypes.POINTER(ctypes.c_double)
    i64 = ctypes.c_int64
    lib.fo_scan_f64.argtypes = [dp, i64, i64, i64, i64, i64, dp, dp, dp, dp, dp, dp]
    lib.fo_scan_f64.restype = None
    lib.fo_decode_step_f64.argtypes = [dp, i64, i64, i64, dp, dp, dp, dp, dp]
    lib.fo_decode_step_f64.restype = None
    _lib = lib
    return lib


def _ptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _f64(a) -> np.ndarray:
    if hasattr(a, "detach"):  # torch tensor
        a = a.detach().to("cpu").double().numpy()
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def scan_f64(raw, tr, ti, gamma, state_in=None) -> Tuple[np.ndarray, np.ndarray]:
    """Sequential float64 Field scan.

    raw [B,T,3C]; tr/ti/gamma [C]; state_in [B,2C] planar (re | im) or None.
    Returns (read [B,T,4C], state_out [B,2C]) as float64 arrays.
    """
    lib = _load()
    raw = _f64(raw)
    if raw.ndim != 3 or raw.shape[2] % 3:
        raise ValueError(f"raw must be [B,T,3C], got {raw.shape}")
    B, T, C3 = raw.shape
    C = C3 // 3
    tr, ti, gamma = _f64(tr), _f64(ti), _f64(gamma)
    if tr.shape != (C,) or ti.shape != (C,) or gamma.shape != (C,):
        raise ValueError("tr/ti/gamma must be [C]")
    sin = None if state_in is None else _f64(state_in).reshape(B, 2 * C)
    read = np.empty((B, T, 4 * C), dtype=np.float64)
    sout = np.empty((B, 2 * C), dtype=np.float64)
    lib.fo_scan_f64(_ptr(raw), B, T, C, T * C3, C3, _ptr(tr), _ptr(ti), _ptr(gamma), _ptr(sin),
                    _ptr(sout), _ptr(read))
    return read, sout


def decode_step_f64(raw_t, tr, ti, gamma, state) -> Tuple[np.ndarray, np.ndarray]:
    """One float64 decode step. raw_t [B,3C], state [B,2C] planar. Returns (read_t, new_state)."""
    lib = _load()
    raw_t = _f64(raw_t)
    B, C3 = raw_t.shape
    C = C3 // 3
    st = _f64(state).reshape(B, 2 * C).copy()
    out = np.empty((B, 4 * C), dtype=np.float64)
    lib.fo_decode_step_f64(_ptr(raw_t), B, C, C3, _ptr(_f64(tr)), _ptr(_f64(ti)), _ptr(_f64(gamma)),
                           _ptr(st), _ptr(out))
    return out, st


def rms_norm_f64(x, weight, eps: float = 1e-6) -> np.ndarray:
    """float64 RMSNorm over the last axis: x * (mean(x^2) + eps)^(-1/2) * weight.

    Follows ``RMSNorm.forward`` (field_only_v4_chunked_triton_wiki100.py:306-309): the mean of
    squares over the last dimension, eps added inside the root, then the weight."""
    x = _f64(x)
    w = _f64(weight)
    if w.shape != x.shape[-1:]:
        raise ValueError(f"weight must be [{x.shape[-1]}], got {w.shape}")
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * w


def scan_f64_autograd(raw, tr, ti, gamma, state_in=None):
    """Differentiable float64 Field scan (torch complex128), for gradient checks.

    raw [B,T,3C], tr/ti/gamma [C], state_in [B,2C] planar or None, all float64 torch tensors
    (requires_grad as needed). Returns (read [B,T,4C], state_out [B,2C]). Same formulas as
    ``reference_field_read`` (canon:392-416): inj = tanh + i tanh, v = 0.9 sigmoid,
    a = (1-v) lam, b = gamma v inj, s_t = a_t s_{t-1} + b_t, disp = v lam s_{t-1}; the scan is a
    recursive doubling with out-of-place shifts so that autograd differentiates every step.
    """
    import torch

    c = tr.numel()
    inj = torch.complex(torch.tanh(raw[..., :c]), torch.tanh(raw[..., c:2 * c]))
    v = 0.9 * torch.sigmoid(raw[..., 2 * c:])
    lam = torch.complex(tr, ti)
    a = (1.0 - v) * lam
    b = gamma * v * inj
    b_len, t_len = raw.shape[0], raw.shape[1]
    s0 = (torch.zeros((b_len, c), dtype=a.dtype) if state_in is None
          else torch.complex(state_in[:, :c], state_in[:, c:]))
    b = torch.cat((b[:, :1] + a[:, :1] * s0[:, None], b[:, 1:]), dim=1)
    step = 1
    while step < t_len:
        a_prev = torch.cat((torch.ones_like(a[:, :step]), a[:, :-step]), dim=1)
        b_prev = torch.cat((torch.zeros_like(b[:, :step]), b[:, :-step]), dim=1)
        b = a * b_prev + b
        a = a * a_prev
        step *= 2
    prev = torch.cat((s0[:, None], b[:, :-1]), dim=1)
    disp = v * lam * prev
    read = torch.cat((b.real, b.imag, disp.real, disp.imag), dim=-1)
    return read, torch.cat((b[:, -1].real, b[:, -1].imag), dim=-1)


def rel_err(actual, expected) -> float:
    """Norm-wise relative error max|actual - expected| / max|expected| (the parity metric)."""
    a = _f64(actual)
    e = _f64(expected)
    denom = float(np.max(np.abs(e))) if e.size else 0.0
    diff = float(np.max(np.abs(a - e))) if e.size else 0.0
    return diff / max(denom, 1e-30)


def rel_err_rows(actual, expected, planes: int = 1) -> float:
    """Row-wise relative error: the last axis is split into ``planes`` equal planes (``read``'s
    ``[Re s | Im s | Re disp | Im disp]``, ``grad_raw``'s three gate planes), every (row, plane)
    is normalised by its own max|expected|, and the worst one is returned. An error confined to
    small-magnitude rows or to one plane, which :func:`rel_err` divides by the tensor's largest
    value, shows here. A (row, plane) whose expected values are all zero is compared absolutely."""
    a = _f64(actual)
    e = _f64(expected)
    if a.shape != e.shape:
        raise ValueError(f"shape mismatch {a.shape} vs {e.shape}")
    if e.size == 0:
        return 0.0
    n = e.shape[-1]
    if n % planes:
        raise ValueError(f"last axis {n} does not split into {planes} planes")
    a = a.reshape(-1, planes, n // planes)
    e = e.reshape(-1, planes, n // planes)
    diff = np.max(np.abs(a - e), axis=-1)
    den = np.max(np.abs(e), axis=-1)
    return float(np.max(diff / np.where(den > 0.0, den, 1.0)))
