"""ctypes binding of ``libfields_amd.so`` (the C ABI declared in include/fields_amd.h).

PyTorch-ROCm is imported before the library is opened: the library names the HIP runtime by
SONAME (``libamdhip64.so.7``) and the dynamic loader then binds it to the runtime PyTorch has
already loaded, so PyTorch's streams and device pointers are valid in the library.

There is no fallback: if the library is missing, every entry point raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library; see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libfields_amd.so"

FL_DTYPE_F32 = 0
FL_DTYPE_BF16 = 1
FL_ALGO_AUTO = 0
FL_ALGO_CHUNKED3 = 1
FL_ALGO_LOOKBACK = 2
FL_OK = 0
FL_ERR_INVALID_ARGUMENT = 1
FL_ERR_DTYPE = 2
FL_ERR_WORKSPACE = 3
FL_ERR_HIP_BASE = 1000

# every extern "C" symbol of include/fields_amd.h, with (restype, argtypes)
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t
SIGNATURES = {
    "fl_scan_forward": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp,
                               _vp, _int, _vp, _sz, _vp]),
    "fl_scan_forward_ex": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                                  _vp, _vp, _int, _vp, _sz, _int, _vp]),
    "fl_scan_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "fl_scan_norm_forward": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                                    _vp, _vp, ctypes.c_float, _vp, _int, _vp, _sz, _vp]),
    "fl_decode_step": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _int, _vp]),
    "fl_decode_norm_step": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp,
                                   ctypes.c_float, _vp, _int, _vp]),
    "fl_scan_backward": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp,
                                _vp, _vp, _vp, _int, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "fl_scan_backward_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "fl_gate_residual_norm": (_int, [_vp, _int, _vp, _vp, _int, _i64, _i64, _i64, _vp, ctypes.c_float,
                                     _vp, _vp, _vp]),
    "fl_swiglu": (_int, [_vp, _int, _i64, _i64, _vp, _vp]),
    "fl_boundary_scan": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "fl_version": (ctypes.c_char_p, []),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Open libfields_amd.so (once) and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"HIP extension not built: {LIB_PATH} is missing "
                "(run `python -m fields_lm_amd.build` or __graft_entry__.build())")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def check(code: int, what: str) -> None:
    """Map a C-ABI return code to the exception type the reference raises for that failure."""
    if code == FL_OK:
        return
    if code == FL_ERR_INVALID_ARGUMENT:
        raise ValueError(f"{what}: invalid shape, stride or pointer")
    if code == FL_ERR_DTYPE:
        raise TypeError(f"{what}: unsupported dtype")
    if code == FL_ERR_WORKSPACE:
        raise RuntimeError(f"{what}: workspace missing or too small")
    if code >= FL_ERR_HIP_BASE:
        raise RuntimeError(f"{what}: HIP error {code - FL_ERR_HIP_BASE}")
    raise RuntimeError(f"{what}: error code {code}")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return FL_DTYPE_F32
    if dtype == torch.bfloat16:
        return FL_DTYPE_BF16
    raise TypeError(f"raw must be float32 or bfloat16, got {dtype}")


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


# Scan workspaces, one per (device, stream): zero-filled when allocated, then reused as is
# (the library keeps launch counters in the first 2 KiB and re-arms them after every call).
_workspaces: dict = {}


def scan_workspace(device: torch.device, nbytes: int, kind: str = "forward") -> torch.Tensor:
    """Zero-filled, 256-byte aligned workspace of at least ``nbytes`` for the current stream.

    ``kind`` keeps the forward and backward scans' workspaces apart (their layouts differ)."""
    stream = torch.cuda.current_stream(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream.cuda_stream, kind)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), device=device, dtype=torch.uint8)
        _workspaces[key] = ws
    return ws


def workspace_error(ws: torch.Tensor) -> int:
    """Error word of a scan workspace header (0 = every look-back wait completed).

    Header: bytes 0..3 tiles done, 128..131 error bits, 256..263 epoch and ticket counter."""
    return int(ws[128:132].view(torch.int32).item())


# FIELDS_AMD_CHECK=1: every scan, RMSNorm-epilogue scan and backward call synchronizes its stream
# and raises if one of its look-back waits gave up (not usable under HIP graph capture).
CHECK_WAITS = os.environ.get("FIELDS_AMD_CHECK", "0") not in ("", "0")


def check_waits(ws: torch.Tensor, what: str) -> None:
    """With CHECK_WAITS: raise RuntimeError if the workspace's error word is set (bit 0: a wait
    gave up after its spin limit, so a tile went on without its carry or its partner tiles'
    values; bit 1: a ticket beyond the launch's tiles), then clear the word so that later calls
    are checked afresh."""
    if not CHECK_WAITS:
        return
    err = workspace_error(ws)
    if err:
        ws[128:132].zero_()
        raise RuntimeError(f"{what}: a look-back wait gave up (workspace error word {err:#x}); "
                           "the results of this call are invalid")
