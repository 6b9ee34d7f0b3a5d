"""Drop-in module surface on the CPU: constructor signatures, parameter names, seeded
initialisation and error behaviour of the reference's Field block API (canon:1131-1221)."""
from __future__ import annotations

import inspect

import numpy as np
import pytest
import torch

import fields_lm_amd as fl
from fields_lm_amd import FieldBlock, IndependentVacancyField, fused_field_read


def test_constructor_signatures_match_reference():
    # canon:1134-1141 and canon:1199-1207
    assert list(inspect.signature(IndependentVacancyField.__init__).parameters)[1:] == [
        "dim", "backend", "field_chunk", "triton_block_c", "triton_chunk_t"]
    assert list(inspect.signature(FieldBlock.__init__).parameters)[1:] == [
        "dim", "backend", "field_chunk", "triton_block_c", "triton_chunk_t", "ff_hidden"]
    params = inspect.signature(fused_field_read).parameters
    positional = [n for n, p in params.items() if p.kind != inspect.Parameter.KEYWORD_ONLY]
    assert positional == ["raw", "transition_r", "transition_i", "gamma", "block_c", "chunk_t"]
    # extensions are keyword-only, so every reference call site binds identically
    assert all(p.kind == inspect.Parameter.KEYWORD_ONLY for n, p in params.items() if n not in positional)


def test_seeded_construction_equals_reference_fixture(golden_dir):
    d = np.load(golden_dir / "selftest_block.npz")
    ref_sd = {k[len("param::"):]: d[k] for k in d.files if k.startswith("param::")}
    torch.manual_seed(7721)
    block = FieldBlock(64, "triton", 8, 8, 16, 192)
    sd = block.state_dict()
    assert list(sd) == list(ref_sd)  # same keys in the same registration order
    for k, v in sd.items():
        np.testing.assert_array_equal(v.numpy(), ref_sd[k], err_msg=k)
    block.load_state_dict({k: torch.from_numpy(v) for k, v in ref_sd.items()}, strict=True)


def test_parameter_count_promoted_geometry():
    mixer = IndependentVacancyField(1024, "triton", 32, 32, 64)
    assert sum(p.numel() for p in mixer.parameters()) == 4_725_248


def test_constructor_errors():
    with pytest.raises(ValueError):
        IndependentVacancyField(63, "triton", 32, 32, 64)
    with pytest.raises(ValueError):
        IndependentVacancyField(64, "cuda", 32, 32, 64)
    for backend in fl.BACKENDS:
        IndependentVacancyField(64, backend, 32, 32, 64)


def test_no_cpu_fallback():
    """The HIP path is the only path: CPU tensors raise like the reference's Triton path."""
    raw = torch.randn(1, 4, 24)
    p = torch.ones(8)
    with pytest.raises(RuntimeError):
        fused_field_read(raw, p, p, p, 32, 64)
    block = FieldBlock(16, "reference", 8, 8, 16, 64)
    with pytest.raises(RuntimeError):
        block(torch.randn(1, 4, 16))


def test_transition_params_match_oracle():
    from oracle import reference_path as ref

    mixer = IndependentVacancyField(256, "triton", 32, 32, 64)
    tr, ti, gamma = mixer.transition()
    etr, eti, egm = ref.transition_params(mixer.radius_logit.detach(), mixer.theta.detach())
    torch.testing.assert_close(tr, etr, rtol=0, atol=0)
    torch.testing.assert_close(ti, eti, rtol=0, atol=0)
    torch.testing.assert_close(gamma, egm, rtol=0, atol=0)
    assert float(gamma.min()) >= 0.01 - 1e-9 and float(tr.abs().max()) <= 0.99995
