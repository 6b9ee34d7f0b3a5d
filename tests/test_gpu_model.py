"""GPU: the softpatch boundary scan kernel, the softpatch block against the reference, and the
whole model's incremental decode (every block type) against its full forward, eager and in HIP
graphs, at a small geometry and at the promoted 300M geometry.

Tolerances: the boundary scan against a float64 recurrence at 1e-5 (fp32, a short sum); whole
small model fp32 decode vs forward at 1e-4 norm-wise; promoted model in bf16 at 2e-2.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from fields_lm_amd import model as M

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from fields_lm_amd import _native

    _native.load()
    return torch.device("cuda:0")


def _boundary_f64(a, drive, s0=None):
    a, d = a.double().numpy(), drive.double().numpy()
    b, t, r = d.shape
    s = np.zeros((b, r)) if s0 is None else s0.double().numpy().copy()
    out = np.empty_like(d)
    for i in range(t):
        s = a[:, i, None] * s + d[:, i]
        out[:, i] = s
    return out, s


@pytest.mark.parametrize("shape", [(2, 41, 8), (3, 5, 64), (1, 2048, 64), (2, 1000, 100), (1, 1, 3),
                                   (2, 17, 130)], ids=lambda s: "x".join(map(str, s)))
def test_boundary_scan_matches_recurrence(dev, shape):
    from fields_lm_amd import boundary_scan

    B, T, R = shape
    print(f"[case] boundary_scan {shape}", flush=True)
    g = torch.Generator().manual_seed(B * 100 + T + R)
    a = torch.rand(B, T, generator=g) * 0.98 + 0.01
    drive = torch.randn(B, T, R, generator=g)
    s0 = torch.randn(B, R, generator=g)
    out, last = boundary_scan(a.to(dev), drive.to(dev), state_in=s0.to(dev), return_state=True)
    exp, exp_last = _boundary_f64(a, drive, s0)
    assert oracle.rel_err(out.cpu(), exp) <= 1e-5
    assert oracle.rel_err(last.cpu(), exp_last) <= 1e-5
    out0 = boundary_scan(a.to(dev), drive.to(dev))
    exp0, _ = _boundary_f64(a, drive)
    assert oracle.rel_err(out0.cpu(), exp0) <= 1e-5


def test_boundary_scan_errors(dev):
    from fields_lm_amd import boundary_scan

    print("[case] boundary_scan errors", flush=True)
    with pytest.raises(ValueError):
        boundary_scan(torch.ones(2, 5, device=dev), torch.ones(2, 4, 3, device=dev))
    with pytest.raises(TypeError):
        boundary_scan(torch.ones(2, 5, device=dev, dtype=torch.float64), torch.ones(2, 5, 3, device=dev))
    with pytest.raises(RuntimeError):
        boundary_scan(torch.ones(2, 5), torch.ones(2, 5, 3))


def test_softpatch_matches_reference_golden(dev, golden_dir):
    d = np.load(golden_dir / "model_blocks.npz")
    print("[case] softpatch golden", flush=True)
    sd = {k[len("softpatch::param::"):]: torch.from_numpy(d[k]) for k in d.files
          if k.startswith("softpatch::param::")}
    sp = M.BoundaryStateMixer(64, 8, learned=True, vocab=16384)
    sp.load_state_dict(sd, strict=True)
    sp = sp.to(dev)
    with torch.no_grad():
        y = sp(torch.from_numpy(d["softpatch::x"]).to(dev), torch.from_numpy(d["softpatch::tokens"]).to(dev))
    assert oracle.rel_err(y.cpu(), d["softpatch::y"]) <= 1e-5


def test_softpatch_steps_equal_forward(dev):
    print("[case] softpatch steps", flush=True)
    torch.manual_seed(4)
    sp = M.BoundaryStateMixer(64, 8, learned=True, vocab=100).to(dev)
    with torch.no_grad():
        sp.up.weight.normal_(0, 0.1)
        sp.score.weight.normal_(0, 0.2)
    x = torch.randn(2, 30, 64, device=dev)
    tok = torch.randint(0, 100, (2, 30), device=dev)
    with torch.no_grad():
        full = sp(x, tok)
        y, s = sp(x[:, :12], tok[:, :12], return_state=True)
        steps = [sp.step(x[:, t], tok[:, t], s) for t in range(12, 30)]
    assert oracle.rel_err(y.cpu(), full[:, :12].cpu()) <= 1e-5
    assert oracle.rel_err(torch.stack(steps, 1).cpu(), full[:, 12:].cpu()) <= 1e-5


def _small_model(dev, dtype=torch.float32):
    torch.manual_seed(12)
    core = M.FieldTokenSystem(vocab=300, dim=128, ff_hidden=256, refresh_windows=(8, 16, 16, 16),
                              q_heads=4, kv_heads=2, latent_dim=32, landmark_chunk=8, softpatch_rank=16,
                              mamba=dict(d_state=16, d_conv=4, expand=2, headdim=32, ngroups=1, chunk_size=16),
                              late_ff_delta=64)
    with torch.no_grad():  # make the zero-initialised softpatch and gates reach the output
        core.softpatch.up.weight.normal_(0, 0.05)
        core.softpatch.score.weight.normal_(0, 0.1)
        for b in core.blocks:
            if isinstance(b, M.RefreshBlock):
                b.residual_gate.weight.normal_(0, 0.02)
    core = core.to(dev)
    if dtype != torch.float32:
        M.cast_for_inference(core, dtype)
    return core.eval()


@pytest.mark.parametrize("prompt", [19, 32])
def test_small_model_decode_equals_forward(dev, prompt):
    """Prefill + greedy-free decode of given tokens reproduces the full forward's logits at every
    position, through all four block kinds and the softpatch."""
    print(f"[case] small model decode prompt={prompt}", flush=True)
    core = _small_model(dev)
    tokens = torch.randint(0, 300, (3, 57), device=dev, generator=torch.Generator(device=dev).manual_seed(1))
    with torch.no_grad():
        _, logits = core.states_logits(tokens)
        last, cache = core.prefill(tokens[:, :prompt], max_len=64)
        steps = [core.step(tokens[:, t], cache) for t in range(prompt, 57)]
    assert int(cache["pos"]) == 57
    assert oracle.rel_err(last.cpu(), logits[:, prompt - 1].cpu()) <= 1e-4
    got = torch.stack(steps, 1)  # logits after token t predict t+1: compare with forward at t
    assert oracle.rel_err(got.cpu(), logits[:, prompt:].cpu()) <= 1e-4


def test_small_model_decode_step_in_hip_graph(dev):
    """One decode step captured in a HIP graph, replayed token after token (the token buffer
    refilled in between, eager work and synchronisations between replays), equals eager steps."""
    print("[case] small model decode graph", flush=True)
    core = _small_model(dev)
    g = torch.Generator(device=dev).manual_seed(2)
    tokens = torch.randint(0, 300, (2, 40), device=dev, generator=g)
    with torch.no_grad():
        _, eager_cache = core.prefill(tokens[:, :20], max_len=48)
        eager = [core.step(tokens[:, t], eager_cache) for t in range(20, 40)]
        _, cache = core.prefill(tokens[:, :20], max_len=48)
        tok = tokens[:, 20].clone()
        core.step(tok, cache)  # warm-up outside capture (advances the cache by one token)
        _, cache = core.prefill(tokens[:, :20], max_len=48)
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            core.step(tok, cache)  # second warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(s)
        _, fresh = core.prefill(tokens[:, :20], max_len=48)
        _copy_cache(cache, fresh)
        with torch.cuda.graph(graph):
            out = core.step(tok, cache)
        _copy_cache(cache, fresh)
        for i, t in enumerate(range(20, 40)):
            tok.copy_(tokens[:, t])
            graph.replay()
            torch.cuda.synchronize()
            assert oracle.rel_err(out.cpu(), eager[i].cpu()) <= 1e-5, t
    assert int(cache["pos"]) == 40


def _copy_cache(dst, src):
    for i, st in enumerate(src["blocks"]):
        if isinstance(st, dict):
            for k, v in st.items():
                dst["blocks"][i][k].copy_(v)
        else:
            dst["blocks"][i].copy_(st)
    dst["softpatch"].copy_(src["softpatch"])
    dst["pos"].copy_(src["pos"])


def test_promoted_model_bf16_decode_equals_forward(dev):
    """The promoted 300M model (18F/2M/4R), bf16 weights: topology, finite logits, and prefill +
    decode against the full forward at the bf16 tolerance."""
    print("[case] promoted model bf16", flush=True)
    lm = M.build_official_fields(device=dev)
    assert lm.topology_audit["field"] == 18
    core = M.cast_for_inference(lm.core_model).eval()
    tokens = torch.randint(0, 16384, (2, 300), device=dev, generator=torch.Generator(device=dev).manual_seed(3))
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
        out = lm(tokens)
        logits = out.logits
        last, cache = core.prefill(tokens[:, :280], max_len=512)
        steps = [core.step(tokens[:, t], cache) for t in range(280, 300)]
    assert logits.shape == (2, 300, 16384) and torch.isfinite(logits).all()
    assert oracle.rel_err(last.float().cpu(), logits[:, 279].float().cpu()) <= 2e-2
    assert oracle.rel_err(torch.stack(steps, 1).float().cpu(), logits[:, 280:].float().cpu()) <= 2e-2
