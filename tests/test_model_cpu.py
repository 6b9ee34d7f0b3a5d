"""Whole-model pieces that run as stock PyTorch (refresh attention, Mamba-2, topology) on the
CPU: each is checked against a library routine or a brute-force restatement, and every block's
incremental decode against its own full-sequence forward.

Parity with the reference for Mamba-2 is unpinned (mamba_ssm is absent); the checks here pin the
SSD scan to its defining recurrence and decode to prefill.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from fields_lm_amd import model as M


def test_topology_parameter_count_and_names():
    """api:72-91 topology, r1:263-321 parameter matching (within 0.75 % of 300M, width step 32),
    r1:174-203 FFN reallocation, v21/v25/v6 parameter names."""
    ff = M.solve_ff_hidden()
    assert ff % 32 == 0
    with torch.device("meta"):
        core = M.FieldTokenSystem(vocab=16384, dim=1024, ff_hidden=ff)
    audit = M.topology_audit(core)
    assert audit["mamba_positions"] == [10, 22] and audit["refresh_positions"] == [5, 11, 17, 23]
    total = sum(p.numel() for p in core.parameters())
    assert abs(total - 300_000_000) / 300_000_000 <= 0.0075, total
    keys = set(core.state_dict())
    for k in ["emb.weight", "lm_head.weight", "final_norm.weight", "softpatch.score.bias",
              "softpatch.up.weight", "cache.router.5.weight", "cache.shared_weight",
              "blocks.0.ff.gate_up.weight", "blocks.4.ff.w12.weight", "blocks.21.ff.down.weight",
              "blocks.5.attn.q_latent_proj.weight", "blocks.5.attn.kv_up.weight",
              "blocks.5.residual_gate.bias", "blocks.11.attn.global_mix_logit",
              "blocks.10.mixer.in_proj.weight", "blocks.10.mixer.conv1d.weight", "blocks.22.mixer.A_log",
              "blocks.22.mixer.dt_bias", "blocks.22.mixer.D", "blocks.22.mixer.norm.weight",
              "blocks.12.mixer.radius_logit"]:
        assert k in keys, k
    assert core.blocks[0].ff.gate_up.out_features == 2 * (ff - 256)
    assert core.blocks[21].ff.gate_up.out_features == 2 * (ff + 256)
    assert core.blocks[12].ff.w12.out_features == 2 * ff
    assert core.lm_head.weight is core.emb.weight
    assert [core.blocks[i].window for i in (5, 11, 17, 23)] == [256, 512, 1024, 1024]
    mix = core.blocks[10].mixer
    assert (mix.d_inner, mix.nheads, mix.conv_dim, mix.in_proj.out_features) == (2048, 32, 2304, 4384)


@pytest.mark.parametrize("causal", [True, False])
def test_gqa_attention_matches_torch_sdpa(causal):
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 8, 13, 16, generator=g)
    k = torch.randn(2, 2, 13, 16, generator=g)
    v = torch.randn(2, 2, 13, 16, generator=g)
    mask = None if causal else (torch.rand(13, 13, generator=g) > 0.4) | torch.eye(13, dtype=torch.bool)
    got = M.gqa_attention(q, k, v, mask, causal)
    exp = F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1),
                                         attn_mask=mask, is_causal=causal)
    torch.testing.assert_close(got, exp, rtol=1e-5, atol=1e-5)


def _attn(window=8, chunk=4):
    torch.manual_seed(5)
    a = M.LandmarkAttention(64, 4, 2, 16, window, chunk)
    with torch.no_grad():
        a.global_mix_logit.fill_(0.3)
    return a


def test_landmark_attention_local_branch_is_windowed_and_causal():
    """Output at t depends only on tokens of t's window (local) and on complete earlier chunks."""
    a = _attn()
    x = torch.randn(1, 30, 64)
    with torch.no_grad():
        y = a(x)
        x2 = x.clone()
        x2[:, 20:] += 1.0  # future tokens
        torch.testing.assert_close(a(x2)[:, :20], y[:, :20], rtol=0, atol=0)


@pytest.mark.parametrize("prompt", [1, 7, 8, 13, 16])
def test_landmark_attention_decode_equals_forward(prompt):
    a = _attn()
    x = torch.randn(2, 37, 64)
    with torch.no_grad():
        full = a(x)
        y, st = a.prefill(x[:, :prompt], max_len=64)
        steps = [a.step(x[:, t], torch.tensor(t), st) for t in range(prompt, 37)]
    torch.testing.assert_close(y, full[:, :prompt], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(torch.stack(steps, 1), full[:, prompt:], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("max_len", [20, 21, 22, 23, 24, 25])
def test_landmark_attention_decode_to_max_len(max_len):
    """Decoding to the last position the state is sized for (max_len - 1), for max_len on and a
    few tokens past a chunk boundary. Each step writes its own chunk's running landmark to the
    slot after the completed chunks', so the state needs that slot too: with one slot too few the
    write landed on the previous chunk's landmark, which every later token of the chunk reads."""
    a = _attn()
    x = torch.randn(2, max_len, 64)
    with torch.no_grad():
        full = a(x)
        y, st = a.prefill(x[:, :5], max_len=max_len)
        steps = [a.step(x[:, t], torch.tensor(t), st) for t in range(5, max_len)]
    torch.testing.assert_close(y, full[:, :5], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(torch.stack(steps, 1), full[:, 5:], rtol=1e-4, atol=1e-5)


def test_refresh_block_decode_equals_forward():
    torch.manual_seed(6)
    blk = M.RefreshBlock(64, 4, 2, 16, 8, 4, 96)
    with torch.no_grad():
        blk.residual_gate.weight.normal_(0, 0.05)
    x = torch.randn(2, 29, 64)
    with torch.no_grad():
        full = blk(x)
        y, st = blk.prefill(x[:, :10], 40)
        steps = [blk.step(x[:, t], torch.tensor(t), st) for t in range(10, 29)]
    torch.testing.assert_close(y, full[:, :10], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(torch.stack(steps, 1), full[:, 10:], rtol=1e-4, atol=1e-5)


def _ssd_naive(x, dt, A, B, C, h0=None):
    """Defining recurrence in float64: h_t = exp(dt A) h + dt x B^T, y = h C."""
    x, dt, A, B, C = (t.double() for t in (x, dt, A, B, C))
    b, l, h, p = x.shape
    n = B.shape[-1]
    s = torch.zeros(b, h, p, n, dtype=torch.float64) if h0 is None else h0.double()
    ys = []
    for t in range(l):
        s = s * torch.exp(dt[:, t] * A)[:, :, None, None] + (x[:, t] * dt[:, t, :, None])[..., None] * B[:, t, None, None, :]
        ys.append(torch.einsum("bhpn,bn->bhp", s, C[:, t]))
    return torch.stack(ys, 1), s


@pytest.mark.parametrize("l,chunk", [(1, 4), (7, 4), (16, 4), (37, 8), (37, 64), (20, 1)])
def test_ssd_chunked_matches_recurrence(l, chunk):
    g = torch.Generator().manual_seed(l * 10 + chunk)
    b, h, p, n = 2, 3, 4, 5
    x = torch.randn(b, l, h, p, generator=g)
    dt = F.softplus(torch.randn(b, l, h, generator=g))
    A = -torch.rand(h, generator=g) * 3 - 0.5
    B = torch.randn(b, l, n, generator=g)
    C = torch.randn(b, l, n, generator=g)
    h0 = torch.randn(b, h, p, n, generator=g)
    y, s = M.ssd_chunked(x, dt, A, B, C, chunk, initial_state=h0)
    ey, es = _ssd_naive(x, dt, A, B, C, h0)
    torch.testing.assert_close(y.double(), ey, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(s.double(), es, rtol=1e-4, atol=1e-5)


def test_ssd_planted_error_is_caught():
    """A scan that drops the decay of the carried state differs from the recurrence."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 12, 2, 3, generator=g)
    dt = F.softplus(torch.randn(1, 12, 2, generator=g))
    A = -torch.ones(2)
    B, C = torch.randn(1, 12, 4, generator=g), torch.randn(1, 12, 4, generator=g)
    ey, _ = _ssd_naive(x, dt, A, B, C)
    y_wrong, _ = _ssd_naive(x, dt, torch.zeros(2), B, C)
    assert float((y_wrong - ey).abs().max()) > 1e-2
    y, _ = M.ssd_chunked(x, dt, A, B, C, 4)
    torch.testing.assert_close(y.double(), ey, rtol=1e-4, atol=1e-5)


def test_mamba2_decode_equals_forward():
    torch.manual_seed(8)
    mix = M.Mamba2Mixer(32, d_state=8, d_conv=4, expand=2, headdim=16, chunk_size=8)
    blk = M.Mamba2ResidualBlock(32, d_state=8, d_conv=4, expand=2, headdim=16, ngroups=1, chunk_size=8)
    for module in (mix, blk):
        x = torch.randn(2, 27, 32)
        with torch.no_grad():
            if module is mix:
                full = mix(x)
                y, st = mix(x[:, :11], return_state=True)
                steps = [mix.step(x[:, t], st) for t in range(11, 27)]
            else:
                full = blk(x)
                y, st = blk.prefill(x[:, :11], 40)
                steps = [blk.step(x[:, t], torch.tensor(t), st) for t in range(11, 27)]
        torch.testing.assert_close(y, full[:, :11], rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(torch.stack(steps, 1), full[:, 11:], rtol=1e-4, atol=1e-5)


def test_mamba2_short_prompt_conv_state():
    """Prompts shorter than the convolution width leave zero history in the conv state."""
    torch.manual_seed(9)
    mix = M.Mamba2Mixer(32, d_state=8, d_conv=4, expand=2, headdim=16, chunk_size=8)
    x = torch.randn(1, 9, 32)
    with torch.no_grad():
        full = mix(x)
        _, st = mix(x[:, :2], return_state=True)
        steps = [mix.step(x[:, t], st) for t in range(2, 9)]
    torch.testing.assert_close(torch.stack(steps, 1), full[:, 2:], rtol=1e-4, atol=1e-5)


def test_mamba2_forward_matches_conv1d_and_recurrence():
    """The mixer's forward equals torch's causal depthwise conv1d followed by the brute-force
    SSD recurrence, D skip, gated norm and out_proj."""
    torch.manual_seed(12)
    mix = M.Mamba2Mixer(32, d_state=8, d_conv=4, expand=2, headdim=16, chunk_size=8)
    u = torch.randn(2, 19, 32)
    with torch.no_grad():
        z, xbc_raw, dt = mix._split(mix.in_proj(u))
        xbc = F.conv1d(xbc_raw.transpose(1, 2), mix.conv1d.weight, mix.conv1d.bias, padding=3,
                       groups=mix.conv_dim)[..., :19].transpose(1, 2)
        x, bm, cm, dtp = mix._ssm_in(F.silu(xbc), dt)
        xh = x.reshape(2, 19, mix.nheads, mix.headdim)
        y, _ = _ssd_naive(xh, dtp, -torch.exp(mix.A_log), bm, cm)
        y = y.float() + mix.D[:, None] * xh
        exp = mix.out_proj(mix.norm(y.reshape(2, 19, mix.d_inner), z))
        got = mix(u)
    torch.testing.assert_close(got, exp, rtol=1e-4, atol=1e-5)


def test_mamba2_init_ranges():
    torch.manual_seed(10)
    mix = M.Mamba2Mixer(1024)
    dt = F.softplus(mix.dt_bias.detach())
    assert float(dt.min()) >= 1e-4 - 1e-9 and float(dt.max()) <= 0.1 + 1e-6
    A = torch.exp(mix.A_log.detach())
    assert float(A.min()) >= 1.0 and float(A.max()) <= 16.0
    assert torch.equal(mix.D.detach(), torch.ones(32))


def test_cast_for_inference_keeps_fp32_state_parameters():
    torch.manual_seed(11)
    core = M.FieldTokenSystem(vocab=64, dim=32, ff_hidden=64, refresh_windows=(4, 4, 4, 4),
                              q_heads=4, kv_heads=2, latent_dim=8, landmark_chunk=4, softpatch_rank=4,
                              mamba=dict(d_state=4, d_conv=4, expand=2, headdim=8, ngroups=1, chunk_size=4),
                              late_ff_delta=32)
    M.cast_for_inference(core)
    for name, p in core.named_parameters():
        fp32 = name.endswith(("radius_logit", "theta", "A_log", "dt_bias", ".D"))
        assert p.dtype == (torch.float32 if fp32 else torch.bfloat16), name
    assert core.lm_head.weight is core.emb.weight


def test_public_api_errors():
    cfg = M.FieldsConfig()
    assert cfg.model_seed == 1234 and cfg.embedding_seed == 314159 and cfg.pcaf_enabled
    with torch.device("meta"):
        core = M.FieldTokenSystem(vocab=16384, dim=1024, ff_hidden=M.solve_ff_hidden())
    lm = M.FieldsForCausalLM(core, backend_name="x", source_audit={}, topology_audit={})
    with pytest.raises(TypeError):
        lm(torch.zeros(2, 3, dtype=torch.int32))
    assert lm.pcaf_enabled
    lm.set_pcaf_enabled(False)
    assert not lm.pcaf_enabled
    assert lm.config_dict["refresh_windows"] == (256, 512, 1024, 1024)


def test_refresh_block_matches_reference_golden(golden_dir):
    """The reference's FusionRefreshBlockV21 (v21:131-293) on two lengths: several windows with
    padding and landmarks, and a single window without landmarks."""
    d = np.load(golden_dir / "model_blocks.npz")
    sd = {k[len("refresh::param::"):]: torch.from_numpy(d[k]) for k in d.files if k.startswith("refresh::param::")}
    blk = M.RefreshBlock(64, 4, 2, 16, 8, 4, 96)
    assert list(blk.state_dict()) == list(sd)  # same names, same registration order
    blk.load_state_dict(sd, strict=True)
    for name in ("long", "short"):
        with torch.no_grad():
            y = blk(torch.from_numpy(d[f"refresh::{name}::x"]))
        np.testing.assert_allclose(y.numpy(), d[f"refresh::{name}::y"], rtol=1e-5, atol=2e-6, err_msg=name)
