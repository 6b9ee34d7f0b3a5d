"""GPU parity of the scan / decode step with the read_norm RMSNorm fused into the epilogue
(fl_scan_norm_forward, fl_decode_norm_step) against the float64 oracle.

Tolerances: norm-wise relative error <= 1e-4 for fp32 output (the bar of the scan itself);
bf16 output must equal the fp32 output rounded to nearest even, bit for bit; the fused and
unfused module paths agree to 1e-5 (fp32) since they differ only in summation order.
"""
from __future__ import annotations

import pytest
import torch

import oracle
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from fields_lm_amd import _native

    _native.load()
    return torch.device("cuda:0")


def _params(C, seed):
    rl, th = ref.init_radius_theta(C)
    g = torch.Generator().manual_seed(seed)
    rl = rl + 0.5 * torch.randn(C, generator=g)
    th = th + 0.3 * torch.randn(C, generator=g)
    return ref.transition_params(rl, th)


def _weight(C, seed):
    g = torch.Generator().manual_seed(seed + 17)
    return 1.0 + 0.5 * torch.randn(4 * C, generator=g)


def _to(dev, *ts):
    return [t.to(dev).contiguous() for t in ts]


# C = 48, 6, 5: one partial channel tile; 512: 8 tiles; 1024: 16; 4096: 64 (the maximum);
# (16, 1000, 512), (24, 700, 200): more tiles than one round of resident blocks; (2, 9000, 200):
# more than 64 chunks per chain, tickets from the counter instead of in block order
SHAPES = [(2, 37, 32), (1, 1, 32), (3, 64, 48), (2, 100, 6), (2, 65, 5), (1, 130, 512),
          (4, 257, 512), (2, 1000, 1024), (1, 300, 4096), (16, 1000, 512), (24, 700, 200),
          (2, 9000, 200)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_scan_norm_matches_oracle(dev, shape, dtype):
    from fields_lm_amd import field_scan_norm

    B, T, C = shape
    print(f"[case] scan_norm shape={shape} dtype={dtype}", flush=True)
    g = torch.Generator().manual_seed(B * 1000 + T + C)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dtype)
    sin = torch.randn(B, 2 * C, generator=g) * 0.3
    tr, ti, gamma = _params(C, seed=C)
    w = _weight(C, C)
    for eps in (1e-6, 0.05):
        out, state = field_scan_norm(*_to(dev, raw, tr, ti, gamma, w), eps=eps,
                                     state_in=sin.to(dev), return_state=True)
        torch.cuda.synchronize()
        exp_read, exp_state = oracle.scan_f64(raw.float(), tr, ti, gamma, state_in=sin)
        exp = oracle.rms_norm_f64(exp_read, w, eps)
        assert out.dtype == torch.float32
        assert oracle.rel_err(out.cpu(), exp) <= TOL, eps
        assert oracle.rel_err(state.cpu(), exp_state) <= TOL
        # every row is normalised on its own: check the worst row too
        got = out.cpu().double().numpy()
        row_err = abs(got - exp).max(axis=-1) / abs(exp).max(axis=-1).clip(1e-30)
        assert float(row_err.max()) <= 1e-3, float(row_err.max())


def test_norm_bf16_out_is_rounded_fp32_out(dev):
    """bf16 output = fp32 output rounded to nearest even; state_out equals the plain scan's."""
    from fields_lm_amd import field_scan, field_scan_norm

    print("[case] scan_norm bf16 out", flush=True)
    for (B, T, C, dtype) in [(2, 37, 32, torch.float32), (3, 1000, 512, torch.bfloat16),
                             (2, 130, 7, torch.bfloat16), (1, 4099, 64, torch.float32)]:
        g = torch.Generator().manual_seed(B + T + C)
        raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dtype)
        sin = torch.randn(B, 2 * C, generator=g) * 0.2
        draw, tr, ti, gamma, w = _to(dev, raw, *_params(C, seed=C), _weight(C, C))
        o32, s32 = field_scan_norm(draw, tr, ti, gamma, w, state_in=sin.to(dev), return_state=True)
        o16, s16 = field_scan_norm(draw, tr, ti, gamma, w, state_in=sin.to(dev), return_state=True,
                                   out_dtype=torch.bfloat16)
        _, s_plain = field_scan(draw, tr, ti, gamma, state_in=sin.to(dev), return_state=True)
        assert o16.dtype == torch.bfloat16
        torch.testing.assert_close(o16, o32.to(torch.bfloat16), rtol=0, atol=0)
        torch.testing.assert_close(s16, s32, rtol=0, atol=0)
        torch.testing.assert_close(s32, s_plain, rtol=0, atol=0)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_norm_lds_staged_equals_register_io(dev, out_dtype):
    """The epilogue's LDS-staged 16-byte loads and stores (bf16 raw with 16-byte aligned rows,
    C % 64 == 0) give the register path's output bit for bit: the same values in raw rows with
    an odd stride take the register loads and stores. Ragged T, B > 1, the maximum channel count
    and a chain of more than 64 chunks."""
    from fields_lm_amd import field_scan_norm

    for (B, T, C) in [(3, 1000, 512), (2, 77, 128), (1, 300, 4096), (2, 9000, 64)]:
        print(f"[case] scan_norm lds staged B={B} T={T} C={C} {out_dtype}", flush=True)
        g = torch.Generator().manual_seed(B + T + C + 5)
        raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16)
        sin = torch.randn(B, 2 * C, generator=g) * 0.2
        draw, tr, ti, gamma, w = _to(dev, raw, *_params(C, seed=C), _weight(C, C))
        odd = torch.zeros(B, T, 3 * C + 1, device=dev, dtype=torch.bfloat16)[..., :3 * C]
        odd.copy_(draw)
        a, sa = field_scan_norm(draw, tr, ti, gamma, w, state_in=sin.to(dev), return_state=True,
                                out_dtype=out_dtype)
        b, sb = field_scan_norm(odd, tr, ti, gamma, w, state_in=sin.to(dev), return_state=True,
                                out_dtype=out_dtype)
        torch.cuda.synchronize()
        assert torch.equal(a, b) and torch.equal(sa, sb), (B, T, C)
        exp_read, _ = oracle.scan_f64(raw.float(), *_params(C, seed=C), state_in=sin)
        exp = oracle.rms_norm_f64(exp_read, _weight(C, C), 1e-6)
        assert oracle.rel_err(a.float().cpu(), exp) <= (TOL if out_dtype == torch.float32 else 4e-3)


def test_norm_equals_rmsnorm_module_of_read(dev):
    """Fused epilogue == the package's RMSNorm module applied to the plain scan's fp32 read."""
    from fields_lm_amd import RMSNorm, field_scan, field_scan_norm

    print("[case] scan_norm vs RMSNorm(read)", flush=True)
    B, T, C = 3, 777, 512
    g = torch.Generator().manual_seed(9)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16)
    draw, tr, ti, gamma, w = _to(dev, raw, *_params(C, seed=9), _weight(C, 9))
    norm = RMSNorm(4 * C).to(dev)
    with torch.no_grad():
        norm.weight.copy_(w)
        expect = norm(field_scan(draw, tr, ti, gamma))
    got = field_scan_norm(draw, tr, ti, gamma, w)
    assert oracle.rel_err(got.cpu(), expect.cpu()) <= 1e-5


def test_norm_state_continuation(dev):
    from fields_lm_amd import field_scan_norm

    print("[case] scan_norm continuation", flush=True)
    B, T, C, cut = 2, 700, 256, 333
    g = torch.Generator().manual_seed(11)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16)
    draw, tr, ti, gamma, w = _to(dev, raw, *_params(C, seed=11), _weight(C, 11))
    full, s_full = field_scan_norm(draw, tr, ti, gamma, w, return_state=True)
    a, s_a = field_scan_norm(draw[:, :cut], tr, ti, gamma, w, return_state=True)
    b, s_b = field_scan_norm(draw[:, cut:], tr, ti, gamma, w, state_in=s_a, return_state=True)
    assert oracle.rel_err(torch.cat([a, b], 1).cpu(), full.cpu()) <= TOL
    assert oracle.rel_err(s_b.cpu(), s_full.cpu()) <= TOL


def test_norm_and_plain_calls_share_a_workspace(dev):
    """Plain and fused launches alternate on one workspace (one stream) without interference."""
    from fields_lm_amd import ScanPlan
    from fields_lm_amd import _native as nat

    print("[case] scan_norm workspace sharing", flush=True)
    B, T, C = 2, 900, 512
    g = torch.Generator().manual_seed(12)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16)
    tr, ti, gamma = _params(C, seed=12)
    w = _weight(C, 12)
    draw, dtr, dti, dgm, dw = _to(dev, raw, tr, ti, gamma, w)
    plain = ScanPlan(draw, dtr, dti, dgm)
    fused = ScanPlan(draw, dtr, dti, dgm, norm_weight=dw)
    fused.workspace = plain.workspace  # same bytes, same size
    fused.args = fused.args[:-2] + (nat.ptr(plain.workspace), plain.ws_bytes)
    exp_read, _ = oracle.scan_f64(raw.float(), tr, ti, gamma)
    exp_norm = oracle.rms_norm_f64(exp_read, w, 1e-6)
    for _ in range(3):
        plain.run()
        fused.run()
        torch.cuda.synchronize()
        assert oracle.rel_err(plain.read.cpu(), exp_read) <= TOL
        assert oracle.rel_err(fused.read.cpu(), exp_norm) <= TOL
    assert nat.workspace_error(plain.workspace) == 0


def test_norm_plan_graph_replays(dev):
    from fields_lm_amd import ScanPlan, field_scan_norm
    from fields_lm_amd import _native as nat

    print("[case] scan_norm graph", flush=True)
    B, T, C = 2, 600, 512
    tr, ti, gamma, w = _to(dev, *_params(C, 3), _weight(C, 3))
    raw = torch.zeros(B, T, 3 * C, device=dev, dtype=torch.bfloat16)
    plan = ScanPlan(raw, tr, ti, gamma, read_dtype=torch.bfloat16, norm_weight=w)
    plan.run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run()
    g = torch.Generator().manual_seed(3)
    for _ in range(4):
        raw.copy_((torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16).to(dev))
        graph.replay()
        torch.cuda.synchronize()
        eager, state = field_scan_norm(raw, tr, ti, gamma, w, return_state=True,
                                       out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        torch.testing.assert_close(plan.read, eager, rtol=0, atol=0)
        torch.testing.assert_close(plan.state_out, state, rtol=0, atol=0)
    assert nat.workspace_error(plan.workspace) == 0


@pytest.mark.parametrize("name", ["scan_b8_t2048_d1024", "scan_b1_t65536_d1024"])
def test_norm_full_size_workloads(dev, name):
    """Configs 2 and 4: fused bf16 and fp32 outputs against the float64 oracle's normalised read,
    norm-wise and token row by token row (each row's four planes on their own scale)."""
    from fields_lm_amd import ScanPlan
    from fields_lm_amd import _native as nat
    from fields_lm_amd.workloads import make_scan_workload

    print(f"[case] scan_norm full size {name}", flush=True)
    wl = make_scan_workload(name, dev)
    C = wl.channels
    w = _weight(C, 4).to(dev)
    exp_read, exp_state = oracle.scan_f64(wl.raw.float().cpu(), wl.tr.cpu(), wl.ti.cpu(), wl.gamma.cpu())
    exp = oracle.rms_norm_f64(exp_read, w.cpu(), 1e-6)
    del exp_read
    for out_dtype, tol in ((torch.bfloat16, 4e-3), (torch.float32, TOL)):  # bf16 rounds to within 2^-8 relative
        plan = ScanPlan(wl.raw, wl.tr, wl.ti, wl.gamma, read_dtype=out_dtype, norm_weight=w)
        out = plan.run()
        torch.cuda.synchronize()
        assert nat.workspace_error(plan.workspace) == 0
        got = out.float().cpu()
        e_rows = oracle.rel_err_rows(got, exp, planes=4)
        print(f"[case] scan_norm full size {name} {out_dtype}: norm-wise {oracle.rel_err(got, exp):.2e}, "
              f"row-wise {e_rows:.2e}", flush=True)
        assert oracle.rel_err(got, exp) <= tol, out_dtype
        assert e_rows <= tol, out_dtype
        assert oracle.rel_err(plan.state_out.cpu(), exp_state) <= TOL
        assert oracle.rel_err_rows(plan.state_out.cpu(), exp_state, planes=2) <= TOL
        del plan, out, got


def test_norm_errors(dev):
    from fields_lm_amd import field_scan_norm

    print("[case] scan_norm errors", flush=True)
    C = 4160  # 65 channel tiles: above the resident-group cap
    raw = torch.zeros(1, 4, 3 * C, device=dev)
    p = torch.ones(C, device=dev)
    with pytest.raises(ValueError):
        field_scan_norm(raw, p, p, p, torch.ones(4 * C, device=dev))
    raw = torch.zeros(1, 4, 96, device=dev)
    p = torch.ones(32, device=dev)
    with pytest.raises(ValueError):
        field_scan_norm(raw, p, p, p, torch.ones(64, device=dev))  # weight not 4C
    with pytest.raises(TypeError):
        field_scan_norm(raw, p, p, p, torch.ones(128, device=dev), out_dtype=torch.float16)
    with pytest.raises(ValueError):
        field_scan_norm(raw, p, p, p, torch.ones(128, device=dev), eps=-1.0)


# ---------------------------------------------------------------------------------------------
# decode step with the epilogue
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("C", [32, 5, 512, 1000, 1500, 2100])  # register variants 1,1,2,4,8; 2100: recompute
def test_decode_norm_steps_reproduce_scan_norm(dev, C, dtype):
    from fields_lm_amd import field_decode_norm_step, field_scan_norm

    B, T = 3, 40
    print(f"[case] decode_norm C={C} dtype={dtype}", flush=True)
    g = torch.Generator().manual_seed(C + 5)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dtype)
    tr, ti, gamma = _params(C, C)
    w = _weight(C, C)
    draw, dtr, dti, dgm, dw = _to(dev, raw, tr, ti, gamma, w)
    full = field_scan_norm(draw, dtr, dti, dgm, dw)
    state = torch.zeros(B, 2 * C, device=dev)
    state16 = torch.zeros(B, 2 * C, device=dev)
    rows, rows16 = [], []
    for t in range(T):
        rows.append(field_decode_norm_step(draw[:, t], dtr, dti, dgm, state, dw))
        rows16.append(field_decode_norm_step(draw[:, t], dtr, dti, dgm, state16, dw,
                                             out_dtype=torch.bfloat16))
    steps = torch.stack(rows, 1)
    exp_read, exp_state = oracle.scan_f64(raw.float(), tr, ti, gamma)
    assert oracle.rel_err(steps.cpu(), oracle.rms_norm_f64(exp_read, w, 1e-6)) <= TOL
    assert oracle.rel_err(state.cpu(), exp_state) <= TOL
    assert oracle.rel_err(steps.cpu(), full.cpu()) <= TOL
    torch.testing.assert_close(torch.stack(rows16, 1), steps.to(torch.bfloat16), rtol=0, atol=0)
    torch.testing.assert_close(state16, state, rtol=0, atol=0)


def test_decode_norm_b64_against_oracle(dev):
    from fields_lm_amd import field_decode_norm_step

    B, C = 64, 512
    print("[case] decode_norm B64", flush=True)
    g = torch.Generator().manual_seed(64)
    raw_t = torch.randn(B, 3 * C, generator=g).to(torch.bfloat16)
    state = torch.randn(B, 2 * C, generator=g) * 0.5
    tr, ti, gamma = _params(C, 64)
    w = _weight(C, 64)
    dstate = state.to(dev)
    out = field_decode_norm_step(*_to(dev, raw_t, tr, ti, gamma), dstate, w.to(dev), 1e-6)
    exp_out, exp_state = oracle.decode_step_f64(raw_t.float(), tr, ti, gamma, state)
    assert oracle.rel_err(out.cpu(), oracle.rms_norm_f64(exp_out, w, 1e-6)) <= TOL
    assert oracle.rel_err(dstate.cpu(), exp_state) <= TOL


# ---------------------------------------------------------------------------------------------
# module paths
# ---------------------------------------------------------------------------------------------

def test_module_fused_equals_unfused(dev):
    from fields_lm_amd import FieldBlock

    print("[case] module fused vs unfused", flush=True)
    torch.manual_seed(21)
    block = FieldBlock(512, "triton", 32, 32, 64, 1024).to(dev)
    with torch.no_grad():
        block.mixer.read_norm.weight.copy_(_weight(256, 21))
    x = torch.randn(2, 300, 512, device=dev)
    with torch.no_grad():
        block.mixer.fuse_read_norm = False
        ref_out = block(x)
        y_ref, s_ref = block.prefill(x[:, :200])
        _, s_end_ref = block.prefill(x)
        block.mixer.fuse_read_norm = True
        out = block(x)
        y, s = block.prefill(x[:, :200])
        s_200 = s.clone()
        params = block.mixer.transition()
        steps = [block.step(x[:, t], s, params) for t in range(200, 300)]  # advances s in place
    assert oracle.rel_err(out.cpu(), ref_out.cpu()) <= 1e-5
    assert oracle.rel_err(y.cpu(), y_ref.cpu()) <= 1e-5
    torch.testing.assert_close(s_200, s_ref, rtol=0, atol=0)  # same recurrence, same rounding
    assert oracle.rel_err(s.cpu(), s_end_ref.cpu()) <= 1e-4
    assert oracle.rel_err(torch.stack(steps, 1).cpu(), ref_out[:, 200:].cpu()) <= 1e-4
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        block.mixer.fuse_read_norm = False
        ref16 = block(x)
        block.mixer.fuse_read_norm = True
        out16 = block(x)
    assert oracle.rel_err(out16.float().cpu(), ref16.float().cpu()) <= 2e-2


def test_module_path_follows_gradient_need(dev):
    """Inference (no gradient) runs read_norm inside the scan; with gradients the mixer runs the
    scan + the RMSNorm module (read_norm's hook fires) and backward works through fl_scan_backward."""
    from fields_lm_amd import IndependentVacancyField

    print("[case] module path vs gradient need", flush=True)
    mixer = IndependentVacancyField(64, "triton", 32, 32, 64).to(dev)
    calls = []
    mixer.read_norm.register_forward_hook(lambda m, i, o: calls.append(1))
    x = torch.randn(1, 10, 64, device=dev)
    with torch.no_grad():
        y0 = mixer(x)
    assert not calls  # fused
    y = mixer(x.requires_grad_())
    assert calls  # unfused, differentiable
    y.sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()
    assert mixer.radius_logit.grad is not None and mixer.theta.grad is not None
    assert oracle.rel_err(y.detach().cpu(), y0.cpu()) <= 1e-5


# ---------------------------------------------------------------------------------------------
# fused elementwise tail of the Field block (fl_gate_residual_norm, fl_swiglu)
# ---------------------------------------------------------------------------------------------

def _close_to_stock(got, exp, scale):
    """Every element within one bf16 step of the stock result (an fp32 sigmoid / exp may differ
    from the stock one in its last bit and flip a bf16 rounding; ``scale`` bounds the magnitude of
    the rounded intermediate), and >= 99 % of them within 1e-5 relative (sums in another order)."""
    got, exp, scale = got.float(), exp.float(), scale.float().abs()
    diff = (got - exp).abs()
    assert bool((diff <= 2.0 ** -7 * (exp.abs() + scale) + 1e-6).all()), float(diff.max())
    assert float((diff <= 1e-5 * exp.abs() + 1e-7).float().mean()) >= 0.99


@pytest.mark.parametrize("xd,gd", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                                   (torch.float32, torch.float32)], ids=["bf16", "f32_bf16", "f32"])
@pytest.mark.parametrize("rows,dim", [(64, 1024), (3, 2048), (5, 100), (2, 3000), (1, 1)])
def test_gate_residual_norm_matches_stock_ops(dev, xd, gd, rows, dim):
    from fields_lm_amd import RMSNorm, gate_residual_norm

    print(f"[case] gate_residual_norm {xd} {gd} {rows}x{dim}", flush=True)
    g = torch.Generator().manual_seed(rows * 7 + dim)
    x = torch.randn(rows, dim, generator=g).to(xd).to(dev)
    out = torch.randn(rows, dim, generator=g).to(gd).to(dev)
    gp = (torch.randn(rows, dim, generator=g) * 2).to(gd).to(dev)
    norm = RMSNorm(dim).to(dev)
    with torch.no_grad():
        norm.weight.copy_(1.0 + 0.3 * torch.randn(dim, generator=g))
        exp_x = x + (out * torch.sigmoid(gp)).to(x.dtype)   # canon:1193-1195
        exp_h = norm(exp_x)                                   # canon:300-309
    x1, h = gate_residual_norm(x, out, gp, norm.weight, norm.eps)
    assert x1.dtype == xd and h.dtype == xd
    _close_to_stock(x1, exp_x, out)
    _close_to_stock(h, exp_h, out * h.float() / exp_x.float().abs().clamp_min(1e-6))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_swiglu_matches_stock_ops(dev, dtype):
    from fields_lm_amd import swiglu

    print(f"[case] swiglu {dtype}", flush=True)
    g = torch.Generator().manual_seed(3)
    for shape in [(64, 2 * 2528), (2, 7, 2 * 96), (1, 2)]:
        gu = (torch.randn(*shape, generator=g) * 3).to(dtype).to(dev)
        gate, up = gu.chunk(2, dim=-1)
        exp = torch.nn.functional.silu(gate) * up             # canon:323-325
        _close_to_stock(swiglu(gu), exp, up)


def test_field_block_fused_tail_equals_stock_ops(dev):
    from fields_lm_amd import FieldBlock
    from fields_lm_amd.model import GateUpSwiGLU

    print("[case] FieldBlock fused tail", flush=True)
    torch.manual_seed(31)
    block = FieldBlock(256, "triton", 32, 32, 64, 512).to(dev)
    x = torch.randn(2, 70, 256, device=dev)
    with torch.no_grad():
        block.fuse_tail = False
        ref32 = block(x)
        y_ref, s_ref = block.prefill(x[:, :50])
        block.fuse_tail = True
        got32 = block(x)
        y, s = block.prefill(x[:, :50])
        params = block.mixer.decode_params()
        steps = [block.step(x[:, t], s, params) for t in range(50, 70)]
        block.ff = GateUpSwiGLU(256, 384).to(dev)  # the R1-resized FFN layout
        block.fuse_tail = False
        ref_gu = block(x)
        block.fuse_tail = True
        got_gu = block(x)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            block.fuse_tail = False
            ref16 = block(x)
            block.fuse_tail = True
            got16 = block(x)
    assert oracle.rel_err(got32.cpu(), ref32.cpu()) <= 1e-5
    assert oracle.rel_err(y.cpu(), y_ref.cpu()) <= 1e-5
    assert oracle.rel_err(torch.stack(steps, 1).cpu(), ref32[:, 50:].cpu()) <= 1e-4
    assert oracle.rel_err(got_gu.cpu(), ref_gu.cpu()) <= 1e-5
    assert oracle.rel_err(got16.float().cpu(), ref16.float().cpu()) <= 2e-2


def test_gate_residual_norm_strided_gate(dev):
    """gate_pre as a column slice of a wider GEMM output (rows a fixed stride apart) gives the
    same bits as the contiguous copy; a slice whose rows are not evenly spaced is copied first."""
    from fields_lm_amd import gate_residual_norm

    print("[case] gate_residual_norm strided gate", flush=True)
    g = torch.Generator(device=dev).manual_seed(41)
    for dt in (torch.bfloat16, torch.float32):
        x = torch.randn(3, 17, 1024, device=dev, generator=g).to(dt)
        out = torch.randn(3, 17, 1024, device=dev, generator=g).to(dt)
        wide = torch.randn(3, 17, 2560, device=dev, generator=g).to(dt)
        w = torch.rand(1024, device=dev, generator=g) + 0.5
        for gp in (wide[..., 1536:], wide[:, 2:9, 1536:]):
            a = gate_residual_norm(x[:, :gp.shape[1]], out[:, :gp.shape[1]], gp, w)
            b = gate_residual_norm(x[:, :gp.shape[1]], out[:, :gp.shape[1]], gp.contiguous(), w)
            for u, v in zip(a, b):
                torch.testing.assert_close(u, v, rtol=0, atol=0)


def test_field_block_packed_in_proj(dev):
    """Without gradients write_proj and gate_proj run as one GEMM over the stacked weights: the
    block's forward, prefill and decode steps agree with the separate GEMMs, and the packed copy
    follows an in-place weight update."""
    from fields_lm_amd import FieldBlock

    print("[case] FieldBlock packed in_proj", flush=True)
    torch.manual_seed(43)
    block = FieldBlock(256, "triton", 32, 32, 64, 512).to(dev)
    x = torch.randn(2, 70, 256, device=dev)
    with torch.no_grad():
        block.mixer.fuse_in_proj = False
        ref = block(x)
        _, s_ref = block.prefill(x[:, :50])
        steps_ref = [block.step(x[:, t], s_ref) for t in range(50, 70)]
        block.mixer.fuse_in_proj = True
        got = block(x)
        _, s = block.prefill(x[:, :50])
        steps = [block.step(x[:, t], s) for t in range(50, 70)]
        assert oracle.rel_err(got.cpu(), ref.cpu()) <= 1e-5
        assert oracle.rel_err(torch.stack(steps, 1).cpu(), torch.stack(steps_ref, 1).cpu()) <= 1e-5
        assert oracle.rel_err(s.cpu(), s_ref.cpu()) <= 1e-5
        block.mixer.gate_proj.weight.mul_(1.5)
        block.mixer.write_proj.bias.add_(0.1)
        got2 = block(x)
        block.mixer.fuse_in_proj = False
        ref2 = block(x)
        assert oracle.rel_err(got2.cpu(), ref2.cpu()) <= 1e-5
        assert oracle.rel_err(got2.cpu(), got.cpu()) > 1e-3
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            ref16 = block(x)
            block.mixer.fuse_in_proj = True
            got16 = block(x)
        assert oracle.rel_err(got16.float().cpu(), ref16.float().cpu()) <= 2e-2
