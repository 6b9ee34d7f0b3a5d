"""GPU parity of the backward scan (fl_scan_backward; canon:1020-1105) against the gradients of
the float64 oracle (torch autograd through ``oracle.scan_f64_autograd``, itself pinned by finite
differences), and the autograd path of the Field modules.

Tolerance: norm-wise relative error <= 1e-4 for grad_raw, the transition-parameter gradients and
grad_state_in (fp32 adjoint against float64); the reference's own Triton-vs-reference bar is 2e-2
(canon:1479-1488). bf16 grad_raw equals the fp32 one rounded to nearest even, bit for bit.
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


def _oracle_grads(raw, tr, ti, gamma, grad_read, state_in=None, grad_state_out=None):
    """float64 gradients of <grad_read, read> + <grad_state_out, state_out>."""
    r = raw.double().clone().requires_grad_()
    p = [t.double().clone().requires_grad_() for t in (tr, ti, gamma)]
    s0 = None if state_in is None else state_in.double().clone().requires_grad_()
    read, state = oracle.scan_f64_autograd(r, *p, s0)
    loss = (read * grad_read.double()).sum()
    if grad_state_out is not None:
        loss = loss + (state * grad_state_out.double()).sum()
    loss.backward()
    return r.grad, p[0].grad, p[1].grad, p[2].grad, (None if s0 is None else s0.grad)


# (16, 1000, 512), (24, 700, 200): more tiles than one round of resident blocks; (1, 4099, 64):
# more than 64 chunks per chain (tickets from the counter)
SHAPES = [(2, 37, 32), (1, 1, 32), (3, 64, 48), (2, 100, 6), (2, 65, 5), (1, 130, 512),
          (4, 257, 512), (2, 1000, 1024), (1, 4099, 64), (16, 1000, 512), (24, 700, 200)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_backward_matches_oracle_gradients(dev, shape, dtype):
    from fields_lm_amd import field_scan, field_scan_backward

    B, T, C = shape
    print(f"[case] backward shape={shape} dtype={dtype}", flush=True)
    g = torch.Generator().manual_seed(B * 1000 + T + C + 7)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dtype)
    tr, ti, gamma = _params(C, seed=C + 1)
    sin = torch.randn(B, 2 * C, generator=g) * 0.3
    gread = torch.randn(B, T, 4 * C, generator=g)
    gso = torch.randn(B, 2 * C, generator=g)
    d = [t.to(dev) for t in (raw, tr, ti, gamma, sin, gread, gso)]
    read, _ = field_scan(d[0], d[1], d[2], d[3], state_in=d[4], return_state=True)
    g_raw, g_tr, g_ti, g_gm, g_sin = field_scan_backward(d[0], d[1], d[2], d[3], read, d[5], state_in=d[4],
                                                         grad_state_out=d[6], return_state_grad=True)
    torch.cuda.synchronize()
    e_raw, e_tr, e_ti, e_gm, e_sin = _oracle_grads(raw.float(), tr, ti, gamma, gread, sin, gso)
    assert g_raw.dtype == dtype
    tol_raw = TOL if dtype == torch.float32 else 4e-3  # bf16 rounding of grad_raw: at most 2^-8 relative
    assert oracle.rel_err(g_raw.float().cpu(), e_raw) <= tol_raw
    assert oracle.rel_err(g_tr.cpu(), e_tr) <= TOL
    assert oracle.rel_err(g_ti.cpu(), e_ti) <= TOL
    assert oracle.rel_err(g_gm.cpu(), e_gm) <= TOL
    assert oracle.rel_err(g_sin.cpu(), e_sin) <= TOL


def test_backward_bf16_grad_is_rounded_fp32_grad(dev):
    from fields_lm_amd import _native as nat
    from fields_lm_amd import field_scan

    print("[case] backward bf16 grad_raw", flush=True)
    B, T, C = 3, 700, 512
    g = torch.Generator().manual_seed(5)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16).to(dev)
    tr, ti, gamma = (t.to(dev) for t in _params(C, 5))
    read = field_scan(raw, tr, ti, gamma)
    gread = torch.randn(B, T, 4 * C, generator=g).to(dev)
    lib = nat.load()
    outs = {}
    for gd in (torch.float32, torch.bfloat16):
        gr = torch.empty(B, T, 3 * C, device=dev, dtype=gd)
        gp = [torch.empty(C, device=dev) for _ in range(3)]
        n = int(lib.fl_scan_backward_workspace_bytes(B, T, C))
        ws = torch.zeros(n, device=dev, dtype=torch.uint8)
        code = lib.fl_scan_backward(nat.ptr(raw), nat.FL_DTYPE_BF16, B, T, C, raw.stride(0), raw.stride(1),
                                    nat.ptr(tr), nat.ptr(ti), nat.ptr(gamma), None, nat.ptr(read),
                                    nat.ptr(gread), None, nat.ptr(gr), nat.dtype_code(gd), *[nat.ptr(x) for x in gp],
                                    None, nat.ptr(ws), n, nat.stream_handle(dev))
        nat.check(code, "fl_scan_backward")
        torch.cuda.synchronize()
        assert nat.workspace_error(ws) == 0
        outs[gd] = (gr, gp)
    torch.testing.assert_close(outs[torch.bfloat16][0], outs[torch.float32][0].to(torch.bfloat16), rtol=0, atol=0)
    for a, b in zip(outs[torch.bfloat16][1], outs[torch.float32][1]):
        torch.testing.assert_close(a, b, rtol=0, atol=0)


def test_backward_is_linear_and_deterministic(dev):
    """backward(g1 + 2 g2) = backward(g1) + 2 backward(g2) (the adjoint is linear), and repeated
    calls give identical bits (fixed reduction order)."""
    from fields_lm_amd import field_scan, field_scan_backward

    print("[case] backward linearity", flush=True)
    B, T, C = 2, 900, 256
    g = torch.Generator().manual_seed(6)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dev)
    tr, ti, gamma = (t.to(dev) for t in _params(C, 6))
    read = field_scan(raw, tr, ti, gamma)
    g1 = torch.randn(B, T, 4 * C, generator=g).to(dev)
    g2 = torch.randn(B, T, 4 * C, generator=g).to(dev)
    a = field_scan_backward(raw, tr, ti, gamma, read, g1)
    b = field_scan_backward(raw, tr, ti, gamma, read, g2)
    c = field_scan_backward(raw, tr, ti, gamma, read, g1 + 2 * g2)
    c2 = field_scan_backward(raw, tr, ti, gamma, read, g1 + 2 * g2)
    for x, y, z, z2 in zip(a, b, c, c2):
        assert oracle.rel_err(z.cpu(), (x + 2 * y).cpu()) <= 1e-5
        torch.testing.assert_close(z, z2, rtol=0, atol=0)


def test_backward_full_size_config2_row(dev):
    """Config 2 (B=8, T=2048, d=1024) at full size: batch row 3's grad_raw against the float64
    oracle, and the parameter gradients against the sum of per-row oracle gradients of two rows
    run alone (rows are independent)."""
    from fields_lm_amd import field_scan, field_scan_backward
    from fields_lm_amd.workloads import make_scan_workload

    print("[case] backward config 2", flush=True)
    wl = make_scan_workload("scan_b8_t2048_d1024", dev)
    read = field_scan(wl.raw, wl.tr, wl.ti, wl.gamma)
    g = torch.Generator().manual_seed(8)
    gread = torch.randn(read.shape, generator=g).to(dev)
    g_raw, g_tr, _, _ = field_scan_backward(wl.raw, wl.tr, wl.ti, wl.gamma, read, gread)
    row = 3
    e_raw, _, _, _, _ = _oracle_grads(wl.raw[row:row + 1].float().cpu(), wl.tr.cpu(), wl.ti.cpu(), wl.gamma.cpu(),
                                      gread[row:row + 1].cpu())
    assert oracle.rel_err(g_raw[row:row + 1].float().cpu(), e_raw) <= 4e-3
    # row by row, each of grad_raw's three gate planes on its own scale: the bf16 output (2^-8
    # relative rounding) and the fp32 output of the same values (raw upcast exactly)
    assert oracle.rel_err_rows(g_raw[row:row + 1].float().cpu(), e_raw, planes=3) <= 4e-3
    g32 = field_scan_backward(wl.raw[row:row + 1].float(), wl.tr, wl.ti, wl.gamma,
                              read[row:row + 1].contiguous(), gread[row:row + 1].contiguous())[0]
    e_rows = oracle.rel_err_rows(g32.cpu(), e_raw, planes=3)
    print(f"[case] backward config 2 fp32 grad_raw: norm-wise {oracle.rel_err(g32.cpu(), e_raw):.2e}, "
          f"row-wise {e_rows:.2e}", flush=True)
    assert oracle.rel_err(g32.cpu(), e_raw) <= TOL
    assert e_rows <= TOL
    rows = [field_scan_backward(wl.raw[r:r + 1], wl.tr, wl.ti, wl.gamma, read[r:r + 1].contiguous(),
                                gread[r:r + 1].contiguous())[1] for r in range(8)]
    assert oracle.rel_err(g_tr.cpu(), sum(x.double() for x in rows).cpu()) <= 1e-5


def test_backward_many_reduction_rows(dev):
    """B=48, T=1500 (24 chunks, the last partial): 1,152 partial rows per channel tile, added up
    by the reduction launch. Batch rows are independent, so the parameter gradients equal the
    sum of those of four calls on 12 rows each, and grad_raw equals theirs bit for bit (a tile's
    arithmetic does not depend on B); repeated calls give the same bits."""
    from fields_lm_amd import field_scan, field_scan_backward

    print("[case] backward many reduction rows", flush=True)
    B, T, C = 48, 1500, 128
    g = torch.Generator().manual_seed(48)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dev)
    tr, ti, gamma = (t.to(dev) for t in _params(C, 48))
    read = field_scan(raw, tr, ti, gamma)
    gread = torch.randn(B, T, 4 * C, generator=g).to(dev)
    full = field_scan_backward(raw, tr, ti, gamma, read, gread)
    again = field_scan_backward(raw, tr, ti, gamma, read, gread)
    parts = [field_scan_backward(raw[i:i + 12], tr, ti, gamma, read[i:i + 12].contiguous(),
                                 gread[i:i + 12].contiguous()) for i in range(0, B, 12)]
    torch.cuda.synchronize()
    assert torch.equal(full[0], torch.cat([p[0] for p in parts]))
    for j in (1, 2, 3):
        assert oracle.rel_err(full[j].cpu(), sum(p[j].double() for p in parts).cpu()) <= 1e-5, j
    for x, y in zip(full, again):
        assert torch.equal(x, y)


def test_fused_field_read_autograd(dev):
    """fused_field_read's backward (autograd) equals the oracle's gradients, through the
    transition parameters' torch graph as well."""
    from fields_lm_amd import fused_field_read

    print("[case] fused_field_read autograd", flush=True)
    B, T, C = 2, 150, 64
    g = torch.Generator().manual_seed(9)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dev).requires_grad_()
    tr, ti, gamma = (t.to(dev).requires_grad_() for t in _params(C, 9))
    gread = torch.randn(B, T, 4 * C, generator=g).to(dev)
    read = fused_field_read(raw, tr, ti, gamma, 32, 64)
    (read * gread).sum().backward()
    e_raw, e_tr, e_ti, e_gm, _ = _oracle_grads(raw.detach().cpu(), tr.detach().cpu(), ti.detach().cpu(),
                                               gamma.detach().cpu(), gread.cpu())
    assert oracle.rel_err(raw.grad.cpu(), e_raw) <= TOL
    assert oracle.rel_err(tr.grad.cpu(), e_tr) <= TOL
    assert oracle.rel_err(ti.grad.cpu(), e_ti) <= TOL
    assert oracle.rel_err(gamma.grad.cpu(), e_gm) <= TOL


def test_field_block_training_gradients(dev):
    """A FieldBlock with gradients enabled takes the unfused path (fp32 read saved); its parameter
    gradients equal those of a float64 CPU copy of the block whose scan is the oracle."""
    from fields_lm_amd import FieldBlock

    print("[case] FieldBlock gradients", flush=True)
    torch.manual_seed(10)
    block = FieldBlock(64, "triton", 32, 32, 64, 128)
    x = torch.randn(2, 40, 64)
    w = torch.randn(2, 40, 64)
    gblock = block.to(dev)
    y = gblock(x.to(dev))
    (y * w.to(dev)).sum().backward()
    got = {k: p.grad.detach().cpu() for k, p in gblock.named_parameters()}

    cpu = FieldBlock(64, "triton", 32, 32, 64, 128).double()
    cpu.load_state_dict({k: v.detach().cpu().double() for k, v in gblock.state_dict().items()})
    m = cpu.mixer
    xd = x.double()
    raw = m.write_proj(xd)
    tr, ti, gamma = m.transition()
    read, _ = oracle.scan_f64_autograd(raw, tr.double(), ti.double(), gamma.double())
    out = m.out_proj(m.read_norm(read))
    h = xd + out * torch.sigmoid(m.gate_proj(xd))
    yd = h + cpu.ff(cpu.ff_norm(h))
    (yd * w.double()).sum().backward()
    for k, p in cpu.named_parameters():
        assert oracle.rel_err(got[k], p.grad) <= 2e-4, k


def test_autocast_training_keeps_read_fp32(dev):
    """Training under bf16 autocast: the mixer's read reaches read_norm in fp32 and its gradient
    reaches the scan's backward in fp32 (canon:1168 ``.float()``, RMSNorm on the fp32 read, the
    cast to bf16 only at out_proj); the gradients equal those of the same computation written out
    with an explicit fp32 read."""
    from fields_lm_amd import IndependentVacancyField, fused_field_read

    print("[case] autocast training read dtype", flush=True)
    torch.manual_seed(31)
    mixer = IndependentVacancyField(128, "triton", 32, 32, 64).to(dev)
    x = torch.randn(2, 50, 128, device=dev)
    w = torch.randn(2, 50, 128, device=dev)
    seen = []
    h1 = mixer.read_norm.register_forward_pre_hook(lambda m, i: seen.append(("in", i[0].dtype)))
    h2 = mixer.read_norm.register_full_backward_hook(lambda m, gi, go: seen.append(("grad", gi[0].dtype)))
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        y = mixer(x)
    (y.float() * w).sum().backward()
    h1.remove()
    h2.remove()
    assert ("in", torch.float32) in seen and ("grad", torch.float32) in seen, seen
    got = {k: p.grad.clone() for k, p in mixer.named_parameters()}
    mixer.zero_grad()
    with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        raw = mixer.write_proj(x).float()
        tr, ti, gamma = mixer.transition()
        read = fused_field_read(raw, tr, ti, gamma)
        assert read.dtype == torch.float32
        out = mixer.out_proj(mixer.read_norm(read))
        y2 = x + (out * torch.sigmoid(mixer.gate_proj(x))).to(x.dtype)
    (y2.float() * w).sum().backward()
    for k, p in mixer.named_parameters():
        assert oracle.rel_err(got[k].float().cpu(), p.grad.float().cpu()) <= 1e-5, k


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_backward_lds_staged_equals_register_loads(dev, dtype):
    """The second pass's inputs staged in LDS (every channel tile full, 16-byte aligned raw rows)
    and loaded into registers (the same values in raw rows with an odd stride) give identical
    gradients: the same arithmetic in the same order. Ragged T (partial last tile), the first tile
    (its row before the sequence start comes from state_in), B > 1, and more than 64 chunks."""
    from fields_lm_amd import field_scan, field_scan_backward

    for (B, T, C) in [(3, 1000, 512), (2, 77, 128), (1, 4099, 64), (2, 8, 64), (4, 130, 192)]:
        print(f"[case] backward lds staged B={B} T={T} C={C} {dtype}", flush=True)
        g = torch.Generator().manual_seed(B * 100 + T + C)
        raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dtype)
        tr, ti, gamma = _params(C, seed=C + 3)
        sin = torch.randn(B, 2 * C, generator=g) * 0.3
        gread = torch.randn(B, T, 4 * C, generator=g)
        gso = torch.randn(B, 2 * C, generator=g)
        d = [t.to(dev) for t in (raw, tr, ti, gamma, sin, gread, gso)]
        odd = torch.zeros(B, T, 3 * C + 1, device=dev, dtype=dtype)[..., :3 * C]
        odd.copy_(d[0])
        read = field_scan(d[0], d[1], d[2], d[3], state_in=d[4])
        a = field_scan_backward(d[0], d[1], d[2], d[3], read, d[5], state_in=d[4], grad_state_out=d[6],
                                return_state_grad=True)
        b = field_scan_backward(odd, d[1], d[2], d[3], read, d[5], state_in=d[4], grad_state_out=d[6],
                                return_state_grad=True)
        torch.cuda.synchronize()
        for x, y in zip(a, b):
            assert torch.equal(x, y), (B, T, C)
        e_raw = _oracle_grads(raw.float(), tr, ti, gamma, gread, sin, gso)[0]
        tol_raw = TOL if dtype == torch.float32 else 4e-3
        assert oracle.rel_err(a[0].float().cpu(), e_raw) <= tol_raw


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_backward_repeated_calls_with_empty_waves(dev, dtype):
    """Regression: T = 1000 leaves the last 64-step tile 40 rows, so three of its eight waves hold
    no rows. Such a wave once issued its LDS-staged loads without waiting for them, and writes
    still in flight when the block retired landed in the LDS of the next block on the CU (a few
    calls in a hundred came out different). 40 calls must give identical gradients."""
    from fields_lm_amd import _native as nat
    from fields_lm_amd import field_scan, field_scan_backward

    B, T, C = 16, 1000, 512
    print(f"[case] backward repeated calls B={B} T={T} C={C} {dtype}", flush=True)
    g = torch.Generator().manual_seed(63)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dtype).to(dev)
    tr, ti, gamma = (t.to(dev) for t in _params(C, 63))
    read = field_scan(raw, tr, ti, gamma)
    gread = torch.randn(B, T, 4 * C, generator=g).to(dev)
    first = None
    for call in range(40):
        got = [x.clone() for x in field_scan_backward(raw, tr, ti, gamma, read, gread)]
        if first is None:
            first = got
            continue
        for a, b in zip(got, first):
            assert torch.equal(a, b), call
    torch.cuda.synchronize()
    assert nat.workspace_error(nat.scan_workspace(dev, 0, "backward")) == 0


def test_backward_in_hip_graph(dev):
    """fl_scan_backward (the reverse scan and its reduction launch) captured in a HIP graph on a
    stream whose workspace already exists: every replay, with eager work between replays and the
    outputs overwritten with NaN before each, equals the eager call bit for bit (grad_raw, the
    parameter gradients, grad_state_in), so a replay writes every element of every output."""
    from fields_lm_amd import field_scan, field_scan_backward

    print("[case] backward hipGraph", flush=True)
    B, T, C = 3, 700, 128
    g = torch.Generator().manual_seed(91)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16).to(dev)
    tr, ti, gamma = (t.to(dev) for t in _params(C, 91))
    sin = torch.randn(B, 2 * C, generator=g).to(dev)
    read = field_scan(raw, tr, ti, gamma, state_in=sin)
    gread = torch.randn(B, T, 4 * C, generator=g).to(dev)
    gso = torch.randn(B, 2 * C, generator=g).to(dev)
    kw = dict(state_in=sin, grad_state_out=gso, return_state_grad=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # the eager call also creates the stream's backward workspace
        eager = [t.clone() for t in field_scan_backward(raw, tr, ti, gamma, read, gread, **kw)]
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = field_scan_backward(raw, tr, ti, gamma, read, gread, **kw)
    for rep in range(3):
        for t in out:
            t.fill_(float("nan"))
        field_scan(raw, tr, ti, gamma)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for x, y in zip(out, eager):
            assert torch.equal(x, y), rep


def test_backward_workspace_reuse_across_shapes(dev):
    """One backward workspace (the per-stream cache), calls alternating shape: the parameter
    gradients of every call equal those of the shape's first call bit for bit (every tile writes
    its row of partials before the reduction launch reads it, so nothing an earlier call or shape
    left in the workspace is summed)."""
    from fields_lm_amd import field_scan, field_scan_backward

    print("[case] backward workspace reuse", flush=True)
    cases = []
    for i, (B, T, C) in enumerate([(2, 900, 256), (3, 300, 512), (1, 4099, 64), (16, 1000, 512)]):
        g = torch.Generator().manual_seed(60 + i)
        raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dev)
        tr, ti, gamma = (t.to(dev) for t in _params(C, 60 + i))
        read = field_scan(raw, tr, ti, gamma)
        gread = torch.randn(B, T, 4 * C, generator=g).to(dev)
        cases.append((raw, tr, ti, gamma, read, gread))
    from fields_lm_amd import _native as nat

    first = [None] * len(cases)
    for rep in range(3):
        for i in ([0, 1, 2, 3] if rep % 2 == 0 else [3, 1, 0, 2]):
            raw, tr, ti, gamma, read, gread = cases[i]
            got = [x.clone() for x in field_scan_backward(raw, tr, ti, gamma, read, gread)[1:]]
            torch.cuda.synchronize()
            ws = nat.scan_workspace(dev, 0, "backward")
            assert nat.workspace_error(ws) == 0, (rep, i)
            if first[i] is None:
                first[i] = got
                _, e_tr, e_ti, e_gm, _ = _oracle_grads(raw.cpu(), tr.cpu(), ti.cpu(), gamma.cpu(), gread.cpu())
                for a, e in zip(got, (e_tr, e_ti, e_gm)):
                    assert oracle.rel_err(a.cpu(), e) <= TOL, i
            else:
                for a, b in zip(got, first[i]):
                    torch.testing.assert_close(a, b, rtol=0, atol=0, msg=lambda m, rep=rep, i=i: f"rep {rep} case {i}: {m}")
