"""C-ABI library: loads, exports every symbol include/fields_amd.h declares, host-side checks.

No kernel is launched here (no GPU in the build container): only host functions and argument
validation paths that return before any HIP call.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from fields_lm_amd import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "fields_amd.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fl_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not nat.LIB_PATH.exists():
        from fields_lm_amd import build

        build.build()
    return nat.load()


def test_header_declares_expected_entry_points():
    names = _declared_functions()
    assert {"fl_scan_forward", "fl_scan_forward_ex", "fl_scan_workspace_bytes",
            "fl_scan_norm_forward", "fl_decode_step", "fl_decode_norm_step",
            "fl_version"} <= set(names)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name
        assert name in nat.SIGNATURES, name


def test_no_kernel_launch_stub_left_undefined(lib):
    """Every kernel launch in the library has its host stub: hipcc once linked a library whose
    launches of four look-back instances referred to stubs it never emitted, and loading it
    failed. build() refuses such a library."""
    from fields_lm_amd import build

    assert build.unresolved_kernel_stubs(nat.LIB_PATH) == []


def test_header_constants_match_binding():
    text = HEADER.read_text()
    consts = dict(re.findall(r"#define (FL_[A-Z0-9_]+) (\d+)", text))
    for name, value in consts.items():
        assert getattr(nat, name) == int(value), name


def test_version_and_workspace_size(lib):
    assert lib.fl_version().decode().startswith("fields_amd")
    # header + look-back status/data regions + the three-phase buffers (20 B per channel-chunk)
    for B, T, C in [(8, 2048, 512), (1, 65536, 512), (2, 37, 5)]:
        n = lib.fl_scan_workspace_bytes(B, T, C)
        chunked3 = B * ((T + 63) // 64) * C * 20
        lookback = B * ((T + 255) // 256) * ((C + 63) // 64) * 64 * 40  # tiles of <= 256 steps
        assert n >= 2048 + chunked3 + lookback, (B, T, C, n)
        assert n % 4 == 0
    assert lib.fl_scan_workspace_bytes(0, 2048, 512) == 0
    assert lib.fl_scan_workspace_bytes(8, 4096, 512) > lib.fl_scan_workspace_bytes(8, 2048, 512)


def _scan(lib, **kw):
    a = dict(raw=256, raw_dtype=0, B=1, T=4, C=8, sb=4 * 24, st=24, tr=256, ti=256, gamma=256,
             state_in=None, state_out=None, read=256, read_dtype=0, ws=256, ws_bytes=1 << 20,
             algo=0, stream=None)
    a.update(kw)
    return lib.fl_scan_forward_ex(a["raw"], a["raw_dtype"], a["B"], a["T"], a["C"], a["sb"], a["st"],
                                  a["tr"], a["ti"], a["gamma"], a["state_in"], a["state_out"], a["read"],
                                  a["read_dtype"], a["ws"], a["ws_bytes"], a["algo"], a["stream"])


def test_argument_validation_returns_before_launch(lib):
    # fake (never dereferenced) pointers: every case below fails validation first
    assert _scan(lib, raw_dtype=7) == nat.FL_ERR_DTYPE
    assert _scan(lib, read_dtype=7) == nat.FL_ERR_DTYPE
    assert _scan(lib, B=0) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan(lib, T=-1) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan(lib, st=23) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan(lib, B=2, sb=24) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan(lib, raw=None) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan(lib, read=None) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan(lib, algo=9) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan(lib, algo=nat.FL_ALGO_LOOKBACK | (99 << 8)) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan(lib, ws=None) == nat.FL_ERR_WORKSPACE
    assert _scan(lib, ws_bytes=10) == nat.FL_ERR_WORKSPACE
    assert _scan(lib, raw=257) == nat.FL_ERR_INVALID_ARGUMENT  # misaligned bf16/f32 pointer
    assert _scan(lib, ws=264) == nat.FL_ERR_INVALID_ARGUMENT  # workspace not 256-byte aligned
    assert lib.fl_decode_step(16, 3, 1, 8, 24, 16, 16, 16, 16, 16, 0, None) == nat.FL_ERR_DTYPE
    assert lib.fl_decode_step(16, 0, 0, 8, 24, 16, 16, 16, 16, 16, 0, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert lib.fl_decode_step(16, 0, 1, 8, 23, 16, 16, 16, 16, 16, 0, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert lib.fl_decode_step(None, 0, 1, 8, 24, 16, 16, 16, 16, 16, 0, None) == nat.FL_ERR_INVALID_ARGUMENT


def _scan_norm(lib, **kw):
    a = dict(raw=256, raw_dtype=0, B=1, T=4, C=8, sb=4 * 24, st=24, tr=256, ti=256, gamma=256,
             state_in=None, state_out=None, w=256, eps=1e-6, out=256, out_dtype=0, ws=256,
             ws_bytes=1 << 40, stream=None)
    a.update(kw)
    return lib.fl_scan_norm_forward(a["raw"], a["raw_dtype"], a["B"], a["T"], a["C"], a["sb"], a["st"],
                                    a["tr"], a["ti"], a["gamma"], a["state_in"], a["state_out"],
                                    a["w"], a["eps"], a["out"], a["out_dtype"], a["ws"],
                                    a["ws_bytes"], a["stream"])


def test_norm_argument_validation_returns_before_launch(lib):
    assert _scan_norm(lib, w=None) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan_norm(lib, w=258) == nat.FL_ERR_INVALID_ARGUMENT  # misaligned weight
    assert _scan_norm(lib, eps=-1.0) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan_norm(lib, eps=float("nan")) == nat.FL_ERR_INVALID_ARGUMENT
    assert _scan_norm(lib, out_dtype=7) == nat.FL_ERR_DTYPE
    assert _scan_norm(lib, ws_bytes=10) == nat.FL_ERR_WORKSPACE
    # 65 channel tiles of 64: above the cap of tiles resident together
    assert _scan_norm(lib, C=4160, st=3 * 4160, sb=4 * 3 * 4160) == nat.FL_ERR_INVALID_ARGUMENT
    dn = lib.fl_decode_norm_step
    assert dn(16, 0, 1, 8, 24, 16, 16, 16, 16, 16, 1e-6, 16, 7, None) == nat.FL_ERR_DTYPE
    assert dn(16, 5, 1, 8, 24, 16, 16, 16, 16, 16, 1e-6, 16, 0, None) == nat.FL_ERR_DTYPE
    assert dn(16, 0, 0, 8, 24, 16, 16, 16, 16, 16, 1e-6, 16, 0, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert dn(16, 0, 1, 8, 23, 16, 16, 16, 16, 16, 1e-6, 16, 0, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert dn(16, 0, 1, 8, 24, 16, 16, 16, 16, None, 1e-6, 16, 0, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert dn(16, 0, 1, 8, 24, 16, 16, 16, 16, 16, -1.0, 16, 0, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert dn(16, 0, 1, 8, 24, 16, 16, 16, 16, 18, 1e-6, 16, 0, None) == nat.FL_ERR_INVALID_ARGUMENT


def test_boundary_scan_validation_returns_before_launch(lib):
    bs = lib.fl_boundary_scan
    assert bs(256, 256, 0, 4, 8, None, None, 256, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert bs(256, 256, 1, 0, 8, None, None, 256, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert bs(256, 256, 1, 4, 0, None, None, 256, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert bs(None, 256, 1, 4, 8, None, None, 256, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert bs(256, 256, 1, 4, 8, None, None, None, None) == nat.FL_ERR_INVALID_ARGUMENT
    assert bs(258, 256, 1, 4, 8, None, None, 256, None) == nat.FL_ERR_INVALID_ARGUMENT  # misaligned


def test_error_mapping():
    nat.check(nat.FL_OK, "x")
    with pytest.raises(ValueError):
        nat.check(nat.FL_ERR_INVALID_ARGUMENT, "x")
    with pytest.raises(TypeError):
        nat.check(nat.FL_ERR_DTYPE, "x")
    with pytest.raises(RuntimeError):
        nat.check(nat.FL_ERR_WORKSPACE, "x")
    with pytest.raises(RuntimeError, match="HIP error 2"):
        nat.check(nat.FL_ERR_HIP_BASE + 2, "x")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(nat, "_lib", None)
    monkeypatch.setattr(nat, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(RuntimeError, match="not built"):
        nat.load()


def test_wait_check_raises_on_error_word(monkeypatch):
    """FIELDS_AMD_CHECK: a set error word in the workspace header raises RuntimeError and is
    cleared; a clear word passes; with the check off nothing is read."""
    import torch

    ws = torch.zeros(4096, dtype=torch.uint8)
    monkeypatch.setattr(nat, "CHECK_WAITS", True)
    nat.check_waits(ws, "fl_scan_forward")
    ws[128] = 1
    with pytest.raises(RuntimeError, match="look-back wait gave up"):
        nat.check_waits(ws, "fl_scan_forward")
    assert nat.workspace_error(ws) == 0
    monkeypatch.setattr(nat, "CHECK_WAITS", False)
    ws[128] = 1
    nat.check_waits(ws, "fl_scan_forward")
    assert nat.workspace_error(ws) == 1


def test_bench_library_exports():
    """bench.py's measurement library (copy kernels of the scan's access pattern, the device delay)
    loads and exports its three entry points; its argument checks refuse shapes outside the
    pattern and delays outside 0..10 ms."""
    from fields_lm_amd import build

    if not build.BENCH_LIB_PATH.exists():
        build.build_bench()
    blib = ctypes.CDLL(str(build.BENCH_LIB_PATH))
    for name in ("fl_bench_tile_copy", "fl_bench_stream_copy", "fl_bench_device_delay"):
        assert hasattr(blib, name), name
    blib.fl_bench_device_delay.restype = ctypes.c_int
    blib.fl_bench_device_delay.argtypes = [ctypes.c_double, ctypes.c_void_p]
    assert blib.fl_bench_device_delay(-1.0, None) == 1      # refused before any HIP call
    assert blib.fl_bench_device_delay(20000.0, None) == 1   # beyond 10 ms
    blib.fl_bench_tile_copy.restype = ctypes.c_int
    blib.fl_bench_tile_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 3 + \
        [ctypes.c_int, ctypes.c_void_p]
    assert blib.fl_bench_tile_copy(None, None, 1, 100, 64, 4, None) == 1  # T % 128 != 0
    assert blib.fl_bench_tile_copy(None, None, 1, 128, 65, 4, None) == 1  # C % 64 != 0
