"""GPU: seeded random shapes against the float64 oracle.

Each case draws B, T and C (C from 1 to 700, so every path is hit: partial channel tiles,
register I/O, the LDS-staged path where C % 64 == 0), a padded row stride for raw, raw and read
dtypes, a state_in or none, and the algorithm (look-back or three-phase), then checks read and
state_out against ``oracle.scan_f64`` (canon:392-416) at 1e-4 (bf16 read: the fp32 result rounded
to nearest even, 1e-2). Every fifth case also runs the fused RMSNorm epilogue against
``rms_norm_f64`` at 1e-4, and every seventh the backward, on a row prefix of the case (at most 60k
token-channels), against the float64 autograd oracle at 1e-4 (bf16 grad_raw, the rounded fp32
value, at 1e-2). Separate cases draw decode steps (24), backward calls (16, some with long
chains of counter tickets) and RMSNorm-epilogue scans (12, up to 64 channel tiles of siblings). The draws are fixed by the seed, so a failure names a reproducible case.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

N_CASES = 48


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from fields_lm_amd import _native

    _native.load()
    return torch.device("cuda:0")


def _draw(i):
    rng = np.random.default_rng(1000 + i)
    C = int(rng.choice([int(rng.integers(1, 64)), 64 * int(rng.integers(1, 9)),
                        int(rng.integers(65, 700))]))
    B = int(rng.integers(1, 6))
    t_max = max(1, min(3000, 600_000 // (B * C)))
    T = int(rng.integers(1, t_max + 1))
    pad = int(rng.choice([0, 0, 8, int(rng.integers(1, 17))]))
    return dict(B=B, T=T, C=C, pad=pad, raw_bf16=bool(rng.integers(0, 2)),
                read_bf16=bool(rng.integers(0, 4) == 0), state=bool(rng.integers(0, 2)),
                chunked3=bool(rng.integers(0, 5) == 0), seed=int(rng.integers(0, 1 << 30)),
                eps=float(rng.choice([1e-6, 0.05])))


def _inputs(case, dev):
    B, T, C, pad = case["B"], case["T"], case["C"], case["pad"]
    g = torch.Generator().manual_seed(case["seed"])
    full = torch.randn(B, T, 3 * C + pad, generator=g) * 2
    raw_cpu = full[..., :3 * C]
    if case["raw_bf16"]:
        full = full.to(torch.bfloat16)
        raw_cpu = full[..., :3 * C].float()
    rl, th = ref.init_radius_theta(C)
    tr, ti, gamma = ref.transition_params(rl + 0.5 * torch.randn(C, generator=g),
                                          th + 0.3 * torch.randn(C, generator=g))
    sin = torch.randn(B, 2 * C, generator=g) if case["state"] else None
    raw = full.to(dev)[..., :3 * C]  # row stride 3C + pad
    return raw, raw_cpu, tr, ti, gamma, sin


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_shape_against_oracle(dev, i):
    from fields_lm_amd import _native as nat
    from fields_lm_amd import field_scan, field_scan_backward, field_scan_norm

    case = _draw(i)
    print(f"[case] fuzz {i}: {case}", flush=True)
    raw, raw_cpu, tr, ti, gamma, sin = _inputs(case, dev)
    B, T, C = case["B"], case["T"], case["C"]
    d = [t.to(dev) for t in (tr, ti, gamma)]
    sin_d = None if sin is None else sin.to(dev)
    algo = nat.FL_ALGO_CHUNKED3 if case["chunked3"] else nat.FL_ALGO_AUTO
    read_dtype = torch.bfloat16 if case["read_bf16"] else torch.float32
    read, state = field_scan(raw, *d, state_in=sin_d, return_state=True, algo=algo,
                             read_dtype=read_dtype)
    exp_read, exp_state = oracle.scan_f64(raw_cpu, tr, ti, gamma, sin)
    tol = 1e-2 if case["read_bf16"] else 1e-4
    assert oracle.rel_err(read.float().cpu(), exp_read) <= tol
    assert oracle.rel_err(state.cpu(), exp_state) <= 1e-4
    if i % 5 == 0 and C <= 4096:
        w = torch.rand(4 * C, generator=torch.Generator().manual_seed(i)) + 0.5
        out, st2 = field_scan_norm(raw, *d, w.to(dev), case["eps"], state_in=sin_d,
                                   return_state=True)
        exp = oracle.rms_norm_f64(exp_read, w, case["eps"])
        assert oracle.rel_err(out.cpu(), exp) <= 1e-4
        assert oracle.rel_err(st2.cpu(), exp_state) <= 1e-4
    if i % 7 == 0:
        # the backward on a row prefix of the case (same strides), at most 60k token-channels
        tb = max(1, min(T, 60_000 // (B * C)))
        raw_b = raw[:, :tb]
        read32 = field_scan(raw_b, *d, state_in=sin_d)
        gread = torch.randn(B, tb, 4 * C, generator=torch.Generator().manual_seed(i + 1))
        gso = torch.randn(B, 2 * C, generator=torch.Generator().manual_seed(i + 2))
        g_raw, g_tr, g_ti, g_gm, g_sin = field_scan_backward(
            raw_b, *d, read32, gread.to(dev), state_in=sin_d, grad_state_out=gso.to(dev),
            return_state_grad=True)
        r = raw_cpu[:, :tb].double().requires_grad_()
        p = [t.double().requires_grad_() for t in (tr, ti, gamma)]
        s0 = None if sin is None else sin.double().requires_grad_()
        out64, st64 = oracle.scan_f64_autograd(r, *p, s0)
        ((out64 * gread.double()).sum() + (st64 * gso.double()).sum()).backward()
        tol_raw = 1e-2 if case["raw_bf16"] else 1e-4  # bf16 grad_raw is the rounded fp32 value
        assert oracle.rel_err(g_raw.float().cpu(), r.grad) <= tol_raw
        assert oracle.rel_err(g_tr.cpu(), p[0].grad) <= 1e-4
        assert oracle.rel_err(g_ti.cpu(), p[1].grad) <= 1e-4
        assert oracle.rel_err(g_gm.cpu(), p[2].grad) <= 1e-4
        if s0 is not None:
            assert oracle.rel_err(g_sin.cpu(), s0.grad) <= 1e-4


@pytest.mark.parametrize("i", range(24))
def test_random_decode_step_against_oracle(dev, i):
    """Random B (1..300), C (1..1200), raw dtype, padded raw_t rows and output dtype: two chained
    steps of ``field_decode_step`` and of ``field_decode_norm_step`` against ``decode_step_f64``
    (+ ``rms_norm_f64``), state included, at 1e-4 (bf16 output: 1e-2)."""
    from fields_lm_amd import field_decode_norm_step, field_decode_step

    rng = np.random.default_rng(5000 + i)
    B, C = int(rng.integers(1, 301)), int(rng.integers(1, 1201))
    pad = int(rng.choice([0, 8, int(rng.integers(1, 17))]))
    raw_bf16, out_bf16 = bool(rng.integers(0, 2)), bool(rng.integers(0, 3) == 0)
    eps = float(rng.choice([1e-6, 0.05]))
    print(f"[case] decode fuzz {i}: B={B} C={C} pad={pad} raw_bf16={raw_bf16} out_bf16={out_bf16}",
          flush=True)
    g = torch.Generator().manual_seed(int(rng.integers(0, 1 << 30)))
    rl, th = ref.init_radius_theta(C)
    tr, ti, gamma = ref.transition_params(rl + 0.5 * torch.randn(C, generator=g),
                                          th + 0.3 * torch.randn(C, generator=g))
    w = torch.rand(4 * C, generator=g) + 0.5
    state0 = torch.randn(B, 2 * C, generator=g)
    d = [t.to(dev) for t in (tr, ti, gamma)]
    st_plain, st_norm = state0.to(dev), state0.to(dev)
    exp_state = state0.double().numpy()
    for step in range(2):
        full = torch.randn(B, 3 * C + pad, generator=g) * 2
        if raw_bf16:
            full = full.to(torch.bfloat16)
        raw_cpu = full[:, :3 * C].float()
        raw_t = full.to(dev)[:, :3 * C]  # row stride 3C + pad
        read_t = field_decode_step(raw_t, *d, st_plain)
        normed = field_decode_norm_step(raw_t, *d, st_norm, w.to(dev), eps,
                                        out_dtype=torch.bfloat16 if out_bf16 else torch.float32)
        exp_read, exp_state = oracle.decode_step_f64(raw_cpu, tr, ti, gamma, exp_state)
        assert oracle.rel_err(read_t.cpu(), exp_read) <= 1e-4, step
        exp_norm = oracle.rms_norm_f64(exp_read, w, eps)
        assert oracle.rel_err(normed.float().cpu(), exp_norm) <= (1e-2 if out_bf16 else 1e-4), step
        assert oracle.rel_err(st_plain.cpu(), exp_state) <= 1e-4, step
        assert torch.equal(st_plain, st_norm), step  # the same state update in both kernels


@pytest.mark.parametrize("i", range(16))
def test_random_backward_against_oracle(dev, i):
    """Random B (1..6), C (1..300, multiples of 64 every third case), T up to 70,000 // (B * C) with
    every fourth case past 64 tiles of 64 steps (counter tickets), a padded raw row stride, raw
    dtype, state_in and dL/dstate_out present or not: ``field_scan_backward`` against the float64
    autograd oracle (canon:1020-1105) at 1e-4 (bf16 grad_raw: the rounded fp32 value, 1e-2),
    parameter gradients and grad_state_in (of the zero state when state_in is absent) included."""
    from fields_lm_amd import field_scan, field_scan_backward

    rng = np.random.default_rng(7000 + i)
    C = 64 * int(rng.integers(1, 5)) if i % 3 == 0 else int(rng.integers(1, 301))
    B = int(rng.integers(1, 7))
    if i % 4 == 1:
        B, C = 1, int(rng.integers(1, 9))
        T = int(rng.integers(64 * 64 + 1, 64 * 90))
    else:
        T = int(rng.integers(1, max(2, 70_000 // (B * C))))
    pad = int(rng.choice([0, 8, int(rng.integers(1, 17))]))
    raw_bf16, with_state, with_gso = (bool(rng.integers(0, 2)) for _ in range(3))
    print(f"[case] backward fuzz {i}: B={B} T={T} C={C} pad={pad} raw_bf16={raw_bf16} "
          f"state={with_state} gso={with_gso}", flush=True)
    g = torch.Generator().manual_seed(int(rng.integers(0, 1 << 30)))
    full = torch.randn(B, T, 3 * C + pad, generator=g) * 2
    if raw_bf16:
        full = full.to(torch.bfloat16)
    raw_cpu = full[..., :3 * C].float()
    rl, th = ref.init_radius_theta(C)
    tr, ti, gamma = ref.transition_params(rl + 0.5 * torch.randn(C, generator=g),
                                          th + 0.3 * torch.randn(C, generator=g))
    sin = torch.randn(B, 2 * C, generator=g) if with_state else None
    gso = torch.randn(B, 2 * C, generator=g) if with_gso else None
    gread = torch.randn(B, T, 4 * C, generator=g)
    raw = full.to(dev)[..., :3 * C]  # row stride 3C + pad
    d = [t.to(dev) for t in (tr, ti, gamma)]
    sin_d = None if sin is None else sin.to(dev)
    read = field_scan(raw, *d, state_in=sin_d)
    g_raw, g_tr, g_ti, g_gm, g_sin = field_scan_backward(
        raw, *d, read, gread.to(dev), state_in=sin_d,
        grad_state_out=None if gso is None else gso.to(dev), return_state_grad=True)
    r = raw_cpu.double().requires_grad_()
    p = [t.double().requires_grad_() for t in (tr, ti, gamma)]
    # without state_in the scan starts from zero: the gradient reaching it is dL/d(zero state)
    s0 = (sin if sin is not None else torch.zeros(B, 2 * C)).double().requires_grad_()
    out64, st64 = oracle.scan_f64_autograd(r, *p, s0)
    loss = (out64 * gread.double()).sum()
    if gso is not None:
        loss = loss + (st64 * gso.double()).sum()
    loss.backward()
    assert oracle.rel_err(g_raw.float().cpu(), r.grad) <= (1e-2 if raw_bf16 else 1e-4)
    assert oracle.rel_err(g_tr.cpu(), p[0].grad) <= 1e-4
    assert oracle.rel_err(g_ti.cpu(), p[1].grad) <= 1e-4
    assert oracle.rel_err(g_gm.cpu(), p[2].grad) <= 1e-4
    assert oracle.rel_err(g_sin.cpu(), s0.grad) <= 1e-4


@pytest.mark.parametrize("i", range(12))
def test_random_norm_epilogue_against_oracle(dev, i):
    """The fused RMSNorm epilogue on random shapes with up to 64 channel tiles of siblings:
    C from 1 to 4,096 (the epilogue's limit; multiples of 64 every other case, so the LDS-staged
    path runs too), B 1..4, T up to 400,000 // (B * C) with every fourth case past 64 chunks
    (counter tickets), a padded raw row stride, raw dtype, fp32 or bf16 output, state_in or none:
    ``field_scan_norm`` against ``rms_norm_f64(scan_f64(...))`` (canon:300-309 on canon:392-416's
    read) at 1e-4 (bf16 output: 1e-2), state_out against the oracle state at 1e-4."""
    from fields_lm_amd import field_scan_norm

    rng = np.random.default_rng(9000 + i)
    C = 64 * int(rng.integers(1, 65)) if i % 2 == 0 else int(rng.integers(1, 4097))
    B = int(rng.integers(1, 5))
    if i % 4 == 3:  # counter tickets with sibling groups of up to 8 channel tiles
        B, C = 1, 64 * int(rng.integers(1, 9)) - int(rng.integers(0, 2)) * int(rng.integers(1, 64))
        T = int(rng.integers(128 * 64 + 1, 128 * 80))
    else:
        T = int(rng.integers(1, max(2, 400_000 // (B * C))))
    pad = int(rng.choice([0, 8, int(rng.integers(1, 17))]))
    raw_bf16, out_bf16, with_state = (bool(rng.integers(0, 2)) for _ in range(3))
    eps = float(rng.choice([1e-6, 0.05]))
    print(f"[case] norm fuzz {i}: B={B} T={T} C={C} pad={pad} raw_bf16={raw_bf16} "
          f"out_bf16={out_bf16} state={with_state}", flush=True)
    g = torch.Generator().manual_seed(int(rng.integers(0, 1 << 30)))
    full = torch.randn(B, T, 3 * C + pad, generator=g) * 2
    if raw_bf16:
        full = full.to(torch.bfloat16)
    raw_cpu = full[..., :3 * C].float()
    rl, th = ref.init_radius_theta(C)
    tr, ti, gamma = ref.transition_params(rl + 0.5 * torch.randn(C, generator=g),
                                          th + 0.3 * torch.randn(C, generator=g))
    sin = torch.randn(B, 2 * C, generator=g) if with_state else None
    w = torch.rand(4 * C, generator=g) + 0.5
    raw = full.to(dev)[..., :3 * C]  # row stride 3C + pad
    d = [t.to(dev) for t in (tr, ti, gamma)]
    out, st = field_scan_norm(raw, *d, w.to(dev), eps, state_in=None if sin is None else sin.to(dev),
                              return_state=True,
                              out_dtype=torch.bfloat16 if out_bf16 else torch.float32)
    exp_read, exp_state = oracle.scan_f64(raw_cpu, tr, ti, gamma, sin)
    exp = oracle.rms_norm_f64(exp_read, w, eps)
    assert oracle.rel_err(out.float().cpu(), exp) <= (1e-2 if out_bf16 else 1e-4)
    assert oracle.rel_err(st.cpu(), exp_state) <= 1e-4

