"""GPU: batch rows longer than 2 GiB. The kernels address raw, read, grad_read and grad_raw
through 32-bit buffer descriptors that cover one tile's rows only, so T * 4C * 4 bytes may exceed
2^31 (here B=1, T=300,000, C=512: one fp32 read row is 2.46 GB).

* Forward (bf16 raw, fp32 read, the default LDS-staged path): a subset of 64 channels (raw and
  read planes gathered on the device) against the float64 oracle at 1e-4, the final state included.
* Forward and backward equal the same computation split at T0 = 150,016 (each part within 2 GiB)
  and chained through the state: the prefix's state_out is the suffix's state_in, and the suffix
  backward's grad_state_in is the prefix backward's grad_state_out (the reference's chunked carry,
  canon:519-550, 1020-1105, at one boundary). The split changes only where chunk boundaries and
  carries round: read at 1e-5, grad_raw (bf16) at 1e-2 (one bf16 rounding step of the largest
  values), the parameter gradients (sums over all 300,000 rows) and grad_state_in at 1e-4.
"""
from __future__ import annotations

import pytest
import torch

import oracle
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

B, T, C, T0 = 1, 300_000, 512, 150_016


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from fields_lm_amd import _native

    _native.load()
    return torch.device("cuda:0")


def _rel_err_dev(got, exp):
    """Norm-wise relative error max|got - exp| / max|exp|, computed on the device."""
    return float((got.float() - exp.float()).abs().max() / exp.float().abs().max())


@pytest.fixture(scope="module")
def inputs(dev):
    print(f"[case] long rows B={B} T={T} C={C}", flush=True)
    assert T * 4 * C * 4 > (1 << 31)  # one read row beyond 2 GiB
    g = torch.Generator(device=dev).manual_seed(17)
    raw = (torch.randn(B, T, 3 * C, device=dev, generator=g) * 2).to(torch.bfloat16)
    rl, th = ref.init_radius_theta(C)
    gc = torch.Generator().manual_seed(18)
    tr, ti, gamma = ref.transition_params(rl + 0.5 * torch.randn(C, generator=gc),
                                          th + 0.3 * torch.randn(C, generator=gc))
    return raw, tr.to(dev), ti.to(dev), gamma.to(dev)


def test_long_row_forward_matches_oracle_and_split(dev, inputs):
    from fields_lm_amd import field_scan

    raw, tr, ti, gamma = inputs
    read, state = field_scan(raw, tr, ti, gamma, return_state=True)
    torch.cuda.synchronize()
    # 64 channels spread over all channel tiles, against the float64 oracle
    ch = torch.arange(0, C, C // 64, device=dev)
    raw_sub = torch.cat([raw[..., p * C + ch] for p in range(3)], dim=-1).float().cpu()
    read_sub = torch.cat([read[..., p * C + ch] for p in range(4)], dim=-1).cpu()
    exp_read, exp_state = oracle.scan_f64(raw_sub, tr[ch].cpu(), ti[ch].cpu(), gamma[ch].cpu())
    assert oracle.rel_err(read_sub, exp_read) <= 1e-4
    # the rows past 2 GiB on their own, so that a wrong base there cannot hide behind the rest
    far = T * 4 * C * 4 - (1 << 31)
    t_far = T - far // (4 * C * 4) - 1
    assert oracle.rel_err(read_sub[:, t_far:], exp_read[:, t_far:]) <= 1e-4
    state_sub = torch.cat([state[:, ch], state[:, C + ch]], dim=-1).cpu()
    assert oracle.rel_err(state_sub, exp_state) <= 1e-4
    # split at T0 and chained through the state
    read_a, state_a = field_scan(raw[:, :T0], tr, ti, gamma, return_state=True)
    read_b, state_b = field_scan(raw[:, T0:], tr, ti, gamma, state_in=state_a, return_state=True)
    assert _rel_err_dev(read[:, :T0], read_a) <= 1e-5
    assert _rel_err_dev(read[:, T0:], read_b) <= 1e-5
    assert _rel_err_dev(state, state_b) <= 1e-5


def test_long_row_backward_matches_split(dev, inputs):
    from fields_lm_amd import field_scan, field_scan_backward

    raw, tr, ti, gamma = inputs
    read = field_scan(raw, tr, ti, gamma)
    g = torch.Generator(device=dev).manual_seed(19)
    grad_read = torch.randn(B, T, 4 * C, device=dev, generator=g)
    g_raw, g_tr, g_ti, g_gm, g_sin = field_scan_backward(raw, tr, ti, gamma, read, grad_read,
                                                         return_state_grad=True)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(g_raw).all())
    # suffix from the forward state entering T0 (read's Re s | Im s planes at row T0 - 1), then
    # the prefix with the suffix's carry as dL/dstate_out
    s_t0 = read[:, T0 - 1, :2 * C].contiguous()
    b_raw, b_tr, b_ti, b_gm, b_sin = field_scan_backward(
        raw[:, T0:], tr, ti, gamma, read[:, T0:], grad_read[:, T0:], state_in=s_t0,
        return_state_grad=True)
    a_raw, a_tr, a_ti, a_gm, a_sin = field_scan_backward(
        raw[:, :T0], tr, ti, gamma, read[:, :T0], grad_read[:, :T0], grad_state_out=b_sin,
        return_state_grad=True)
    assert _rel_err_dev(g_raw[:, :T0], a_raw) <= 1e-2
    assert _rel_err_dev(g_raw[:, T0:], b_raw) <= 1e-2
    assert _rel_err_dev(g_tr, a_tr + b_tr) <= 1e-4
    assert _rel_err_dev(g_ti, a_ti + b_ti) <= 1e-4
    assert _rel_err_dev(g_gm, a_gm + b_gm) <= 1e-4
    assert _rel_err_dev(g_sin, a_sin) <= 1e-4
