"""GPU: ``fl_scan_forward_static``, the entry point that allocates nothing (its look-back state
lives in the library's file-scope device array), against ``fl_scan_forward`` with a
caller-provided workspace, through the C ABI. The two run the same kernels, so their outputs
must agree bit for bit; the calls come in a row, each smaller than the one before, on the shared
array that keeps the previous call's contents. Shapes past the array's capacity are refused on
the host before any launch.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

import oracle
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _inputs(B, T, C, raw_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(raw_dtype)
    rl, th = ref.init_radius_theta(C)
    tr, ti, gamma = ref.transition_params(rl + 0.5 * torch.randn(C, generator=g),
                                          th + 0.3 * torch.randn(C, generator=g))
    sin = torch.randn(B, 2 * C, generator=g)
    return raw, tr, ti, gamma, sin


# each call smaller than the one before: config 2, a ragged shape with fp32 raw and bf16 read, a
# short one with a partial channel tile
CASES = [(8, 2048, 512, torch.bfloat16, torch.float32),
         (3, 700, 200, torch.float32, torch.bfloat16),
         (2, 37, 32, torch.bfloat16, torch.float32)]


def test_static_entry_point_equals_workspace_entry_point(dev):
    from fields_lm_amd import _native as nat

    lib = nat.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    for i, (B, T, C, rdt, odt) in enumerate(CASES):
        print(f"[case] static scan call {i}: B={B} T={T} C={C} raw={rdt} read={odt}", flush=True)
        raw, tr, ti, gamma, sin = _inputs(B, T, C, rdt, seed=100 + i)
        raw, tr, ti, gamma, sin = (t.to(dev).contiguous() for t in (raw, tr, ti, gamma, sin))
        st_in = sin if i == 1 else None
        outs = []
        for static in (False, True):
            read = torch.full((B, T, 4 * C), float("nan"), device=dev, dtype=odt)
            sout = torch.full((B, 2 * C), float("nan"), device=dev)
            head = (_p(raw), nat.dtype_code(rdt), B, T, C, raw.stride(0), raw.stride(1), _p(tr), _p(ti),
                    _p(gamma), _p(st_in), _p(sout), _p(read), nat.dtype_code(odt))
            if static:
                rc = lib.fl_scan_forward_static(*head, stream)
            else:
                n = int(lib.fl_scan_workspace_bytes(B, T, C))
                ws = torch.zeros(n, device=dev, dtype=torch.uint8)
                rc = lib.fl_scan_forward(*head, _p(ws), n, stream)
            assert rc == nat.FL_OK, (static, rc)
            torch.cuda.synchronize()
            outs.append((read, sout))
        (r0, s0), (r1, s1) = outs
        assert torch.equal(r0, r1), i  # same kernels: bit for bit
        assert torch.equal(s0, s1), i
        exp, exp_state = oracle.scan_f64(raw.float().cpu(), tr.cpu(), ti.cpu(), gamma.cpu(),
                                         None if st_in is None else st_in.cpu())
        assert oracle.rel_err(r1.float().cpu(), exp) <= (1e-4 if odt == torch.float32 else 1e-2)
        assert oracle.rel_err(s1.cpu(), exp_state) <= 1e-4


def test_static_entry_point_refuses_oversized_shapes(dev):
    from fields_lm_amd import _native as nat

    lib = nat.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    # 64 x 8 channel tiles x 25 chunks = 12,800 tiles > FL_STATIC_MAX_TILES: refused before any
    # launch or pointer use (the pointers are never read)
    B, T, C = 64, 25 * 128, 512
    assert B * (C // 64) * (T // 128) > nat.FL_STATIC_MAX_TILES
    dummy = torch.empty(16, device=dev)
    rc = lib.fl_scan_forward_static(_p(dummy), nat.FL_DTYPE_BF16, B, T, C, T * 3 * C, 3 * C, _p(dummy),
                                    _p(dummy), _p(dummy), None, None, _p(dummy), nat.FL_DTYPE_F32, stream)
    assert rc == nat.FL_ERR_WORKSPACE
