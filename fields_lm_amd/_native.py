"""ctypes binding of ``libfields_amd.so`` (the C ABI declared in include/fields_amd.h).

PyTorch-ROCm is imported before the library is opened: the library names the HIP runtime by
SONAME (``libamdhip64.so.7``) and the dynamic loader then binds it to the runtime PyTorch has
already loaded, so PyTorch's streams and device pointers are valid in the library.

There is no fallback: if the library is missing, every entry point raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import weakref
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
FL_ERR_CAPTURE = 4
FL_ERR_HIP_BASE = 1000
FL_STATIC_MAX_TILES = 12288
FL_STATIC_SCRATCH_BYTES = 31508480

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
    "fl_scan_forward_static": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp,
                                      _vp, _vp, _int, _vp]),
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
    if code == FL_ERR_CAPTURE:
        raise RuntimeError(f"{what}: the first call on a device sets up its static scratch and "
                           "must not be made under stream capture")
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


# Workspace header (the C ABI, include/fields_amd.h): bytes 128..131 the error word, 384..387 the
# spin limit of the kernels' bounded waits (0: 2^20 polls), 392..399 the address of a host-visible
# 32-bit word that the kernels also set when they set the error word (0: none).
ERROR_OFFSET = 128
SPIN_LIMIT_OFFSET = 384
HOST_ERROR_OFFSET = 392
# Published words carry 30 bits of a launch epoch that every launch advances; the launch that
# brings those 30 bits back to zero has its last block zero-fill the buffer after the header, so
# no caller (graph replays and the static-scratch entry included) has to re-zero a workspace.


class _HostWords:
    """Pinned host int32 words for the workspaces' failure reports, handed out from pages that are
    never freed: a kernel that outlives its workspace can only ever write into a word of this pool
    (whose next owner then sees a spurious failure), never into memory reused for other data."""

    PAGE = 1024

    def __init__(self):
        self.pages = []
        self.free = []

    def take(self) -> torch.Tensor:
        if not self.free:
            page = torch.zeros(self.PAGE, dtype=torch.int32, pin_memory=True)
            self.pages.append(page)
            self.free.extend(page[i:i + 1] for i in range(self.PAGE - 1, -1, -1))
        word = self.free.pop()
        word.zero_()
        return word

    def give(self, word: torch.Tensor) -> None:
        self.free.append(word)


_host_words = _HostWords()


class WorkspaceGuard:
    """Host side of one workspace: a pinned host word whose address sits in the header (the
    kernels set it when a bounded wait gives up, so no device read is needed to see it)."""

    def __init__(self, ws: torch.Tensor):
        self.host_error = _host_words.take()
        self.arm(ws)

    def arm(self, ws: torch.Tensor) -> None:
        addr = torch.tensor([self.host_error.data_ptr()], dtype=torch.int64).view(torch.uint8)
        ws[HOST_ERROR_OFFSET:HOST_ERROR_OFFSET + 8].copy_(addr)

    def before_call(self, ws: torch.Tensor, what: str) -> None:
        """Raise RuntimeError if an earlier call on this workspace had a wait give up (its outputs
        hold NaN where a value was missing) or blocks that found the ticket counter out of range
        (their tiles were not computed; the parameter gradients of a backward are NaN)."""
        if int(self.host_error[0]) != 0:
            self.host_error.zero_()
            ws[ERROR_OFFSET:ERROR_OFFSET + 4].zero_()
            raise RuntimeError(
                f"{what}: an earlier call on this workspace had a look-back wait give up or a "
                "ticket out of range; the outputs of that call are invalid (NaN where a carry or a "
                "partner value was missing, not written where a tile was refused)")


# Guards by (device, address) of their workspace tensor; an entry leaves with its tensor, so a
# workspace later allocated at the same address gets a guard (and a header) of its own.
_guards: dict = {}


def _drop_guard(key, guard: WorkspaceGuard) -> None:
    if _guards.get(key) is guard:
        del _guards[key]
    _host_words.give(guard.host_error)


def guard_workspace(ws: torch.Tensor, fresh: bool = False) -> WorkspaceGuard:
    """The guard of a workspace tensor, created (and its host word's address written into the
    header) on first use. ``fresh``: a newly zero-filled workspace, which always gets a new guard."""
    key = (ws.device.index, ws.data_ptr())
    g = _guards.get(key)
    if g is None or fresh:
        g = WorkspaceGuard(ws)
        _guards[key] = g
        weakref.finalize(ws, _drop_guard, key, g)
    return g


def before_call(ws: torch.Tensor, what: str) -> None:
    guard_workspace(ws).before_call(ws, what)


def set_spin_limit(ws: torch.Tensor, polls: int) -> None:
    """Polls a bounded wait of the kernels makes on this workspace before it gives up (0: the
    default 2^20). A small limit makes waits give up on purpose (tests of the failure path)."""
    ws[SPIN_LIMIT_OFFSET:SPIN_LIMIT_OFFSET + 4].copy_(torch.tensor([polls], dtype=torch.int32).view(torch.uint8))


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
        guard_workspace(ws, fresh=True)
    return ws


def workspace_error(ws: torch.Tensor) -> int:
    """Error word of a scan workspace header (0 = every look-back wait completed); reads device
    memory, so it waits for the stream's work."""
    return int(ws[ERROR_OFFSET:ERROR_OFFSET + 4].view(torch.int32).item())


# FIELDS_AMD_CHECK=1: every scan, RMSNorm-epilogue scan and backward call synchronizes its stream
# and raises if one of its look-back waits gave up (skipped while the stream is capturing a HIP
# graph, which cannot synchronize). Without it, and for graph replays, a wait that gave up is
# reported at the next call on the workspace (before_call).
CHECK_WAITS = os.environ.get("FIELDS_AMD_CHECK", "0") not in ("", "0")


def check_waits(ws: torch.Tensor, what: str) -> None:
    """With CHECK_WAITS: raise RuntimeError if the workspace's error word is set (bit 0: a wait
    gave up after its spin limit, so a tile went on without its carry or its partner tiles'
    values; bit 1: a ticket beyond the launch's tiles), then clear the word (and the host word)
    so that later calls are checked afresh. A no-op while the current stream is capturing."""
    if not CHECK_WAITS or (ws.is_cuda and torch.cuda.is_current_stream_capturing()):
        return
    err = workspace_error(ws)
    if err:
        ws[ERROR_OFFSET:ERROR_OFFSET + 4].zero_()
        g = _guards.get((ws.device.index, ws.data_ptr()))
        if g is not None:
            g.host_error.zero_()
        raise RuntimeError(f"{what}: a look-back wait gave up (workspace error word {err:#x}); "
                           "the results of this call are invalid")
