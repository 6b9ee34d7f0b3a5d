"""Pins the CPU oracle (oracle/) — closed forms, invariants, golden vectors from the reference.

The oracle is what every GPU parity test compares against, so each of its functions is checked
here against something other than a retyping of its own formula:
  * golden fixtures written by the reference's own FieldBlock (tests/golden/make_golden.py);
  * scipy.signal.lfilter (a library linear filter) for constant-vacancy sequences;
  * the closed-form geometric series for constant inputs, and T = 1;
  * the two independent restatements (sequential float64 C vs blocked complex64 torch);
  * invariants: chunk-size independence, state continuation, decode == scan, causality,
    s_t + disp_t = lam*s_{t-1} + b_t, boundedness.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
from scipy.signal import lfilter

import oracle
from oracle import reference_path as ref


def _params(C, seed=None):
    rl, th = ref.init_radius_theta(C)
    if seed is not None:
        g = torch.Generator().manual_seed(seed)
        rl = rl + 0.5 * torch.randn(C, generator=g)
        th = th + 0.3 * torch.randn(C, generator=g)
    return ref.transition_params(rl, th)


def _np_gates(raw, gamma):
    """Elementwise gates with numpy's own tanh/exp (independent of the C oracle's code)."""
    C = raw.shape[-1] // 3
    inj = np.tanh(raw[..., :C]) + 1j * np.tanh(raw[..., C:2 * C])
    v = 0.9 / (1.0 + np.exp(-raw[..., 2 * C:]))
    return v, gamma * v * inj


def _split(read):
    C = read.shape[-1] // 4
    s = read[..., :C] + 1j * read[..., C:2 * C]
    d = read[..., 2 * C:3 * C] + 1j * read[..., 3 * C:]
    return s, d


# ---------------------------------------------------------------------------------------------
# golden vectors from the reference
# ---------------------------------------------------------------------------------------------

def test_golden_selftest_scan_and_block(golden_dir):
    d = np.load(golden_dir / "selftest_block.npz")
    sd = {k[len("param::"):]: torch.from_numpy(d[k]) for k in d.files if k.startswith("param::")}
    tr, ti, gamma = ref.transition_params(sd["mixer.radius_logit"], sd["mixer.theta"])
    read, state = oracle.scan_f64(d["raw"], tr, ti, gamma)
    assert oracle.rel_err(read, d["read"]) <= 1e-6
    assert oracle.rel_err(state, d["read"][:, -1, :64]) <= 1e-6
    y, r = ref.block_forward(sd, torch.from_numpy(d["x"]), field_chunk=8, return_read=True)
    assert oracle.rel_err(r, d["read"]) <= 1e-6
    assert oracle.rel_err(y, d["block_out"]) <= 1e-6
    m = ref.mixer_forward(sd, torch.from_numpy(d["x"]), field_chunk=8)
    assert oracle.rel_err(m, d["mixer_out"]) <= 1e-6


def test_golden_config1_rows(golden_dir):
    """Config 1 (B=1, T=2048, d=1024, seed 0): rebuild the block, compare rows and final state."""
    from fields_lm_amd import FieldBlock

    d = np.load(golden_dir / "config1_block.npz")
    torch.manual_seed(0)
    block = FieldBlock(1024, "triton", 32, 32, 64, 2752)
    x = torch.randn(1, 2048, 1024)
    sd = block.state_dict()
    keys = [str(k) for k in d["param_keys"]]
    assert sorted(sd) == keys
    for i, k in enumerate(keys):
        assert float(sd[k].double().sum()) == pytest.approx(float(d["param_sum"][i]), rel=1e-12, abs=1e-9), k
        np.testing.assert_array_equal(sd[k].flatten()[:8].numpy(), d["param_head"][i])
    assert float(x.double().sum()) == pytest.approx(float(d["x_sum"]), rel=1e-12)
    rows = d["rows"]
    with torch.no_grad():
        y, read = ref.block_forward(sd, x, field_chunk=32, return_read=True)
    assert oracle.rel_err(read[0, rows], d["read_rows"]) <= 1e-6
    assert oracle.rel_err(y[0, rows], d["block_rows"]) <= 1e-6
    raw = torch.nn.functional.linear(x, sd["mixer.write_proj.weight"], sd["mixer.write_proj.bias"])
    tr, ti, gamma = ref.transition_params(sd["mixer.radius_logit"], sd["mixer.theta"])
    r64, s64 = oracle.scan_f64(raw, tr, ti, gamma)
    assert oracle.rel_err(r64[0, rows], d["read_rows"]) <= 1e-5
    assert oracle.rel_err(s64[0], d["final_state"].reshape(-1)) <= 1e-5


def _mixer_out_from_read(sd, x, normed):
    """x + out_proj(normed) * sigmoid(gate_proj(x)) in float64 from the golden parameters."""
    x = x.astype(np.float64)
    w = lambda k: sd["mixer." + k].double().numpy()  # noqa: E731
    out = normed @ w("out_proj.weight").T + w("out_proj.bias")
    gate = 1.0 / (1.0 + np.exp(-(x @ w("gate_proj.weight").T + w("gate_proj.bias"))))
    return x + out * gate


def test_golden_rms_norm_of_read(golden_dir):
    """rms_norm_f64 applied to the reference's read reproduces the reference's mixer output
    (its read_norm sits between them, eps 1e-6, canon:1193); mean over 2C instead of 4C, or eps
    outside the root, miss it."""
    d = np.load(golden_dir / "selftest_block.npz")
    sd = {k[len("param::"):]: torch.from_numpy(d[k]) for k in d.files if k.startswith("param::")}
    w = sd["mixer.read_norm.weight"]
    normed = oracle.rms_norm_f64(d["read"], w, 1e-6)
    assert oracle.rel_err(_mixer_out_from_read(sd, d["x"], normed), d["mixer_out"]) <= 1e-5
    r = d["read"].astype(np.float64)
    half = r / np.sqrt(np.mean(r[..., : r.shape[-1] // 2] ** 2, axis=-1, keepdims=True) + 1e-6)
    assert oracle.rel_err(_mixer_out_from_read(sd, d["x"], half), d["mixer_out"]) > 1e-3
    r = d["read"][:, :3].astype(np.float64) * 1e-3  # tiny rows: eps inside vs outside the root
    inside = oracle.rms_norm_f64(r, np.ones(r.shape[-1]), 1e-6)
    outside = r / (np.sqrt(np.mean(r * r, axis=-1, keepdims=True)) + 1e-6)
    assert oracle.rel_err(outside, inside) > 1e-4


def test_rms_norm_invariants():
    """Unit RMS with unit weight and eps 0; scale invariance; weight acts per column; eps -> big
    gives x / sqrt(eps)."""
    g = np.random.default_rng(5)
    x = g.standard_normal((3, 7, 64)) * g.uniform(0.1, 10, (3, 7, 1))
    y = oracle.rms_norm_f64(x, np.ones(64), 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, rtol=1e-12)
    np.testing.assert_allclose(oracle.rms_norm_f64(x * 37.0, np.ones(64), 0.0), y, rtol=1e-12)
    w = g.standard_normal(64)
    np.testing.assert_allclose(oracle.rms_norm_f64(x, w, 0.0), y * w, rtol=1e-12)
    np.testing.assert_allclose(oracle.rms_norm_f64(x, np.ones(64), 1e12), x / 1e6, rtol=1e-9)


def test_autograd_oracle_forward_equals_c_oracle():
    g = torch.Generator().manual_seed(21)
    B, T, C = 2, 45, 6
    raw = torch.randn(B, T, 3 * C, generator=g, dtype=torch.float64) * 2
    tr, ti, gamma = (t.double() for t in _params(C, seed=21))
    s0 = torch.randn(B, 2 * C, generator=g, dtype=torch.float64) * 0.3
    read, state = oracle.scan_f64_autograd(raw, tr, ti, gamma, s0)
    exp_read, exp_state = oracle.scan_f64(raw, tr, ti, gamma, state_in=s0)
    assert oracle.rel_err(read.detach(), exp_read) <= 1e-12
    assert oracle.rel_err(state.detach(), exp_state) <= 1e-12


def test_autograd_oracle_gradients_match_finite_differences():
    """torch.autograd.gradcheck (central differences) pins the oracle's gradients with respect
    to raw, the transition parameters and the initial state."""
    g = torch.Generator().manual_seed(22)
    B, T, C = 1, 7, 2
    raw = (torch.randn(B, T, 3 * C, generator=g, dtype=torch.float64) * 1.5).requires_grad_()
    tr, ti, gamma = (t.double().clone().requires_grad_() for t in _params(C, seed=22))
    s0 = (torch.randn(B, 2 * C, generator=g, dtype=torch.float64) * 0.3).requires_grad_()

    def f(raw, tr, ti, gamma, s0):
        read, state = oracle.scan_f64_autograd(raw, tr, ti, gamma, s0)
        return read, state

    assert torch.autograd.gradcheck(f, (raw, tr, ti, gamma, s0), eps=1e-6, atol=1e-7, rtol=1e-6)


# ---------------------------------------------------------------------------------------------
# closed forms
# ---------------------------------------------------------------------------------------------

def test_t1_closed_form():
    rng = np.random.default_rng(1)
    B, C = 3, 16
    raw = rng.normal(size=(B, 1, 3 * C)) * 2
    tr, ti, gamma = (t.double().numpy() for t in _params(C, seed=1))
    read, state = oracle.scan_f64(raw, tr, ti, gamma)
    v, b = _np_gates(raw[:, 0], gamma)
    s, d = _split(read[:, 0])
    np.testing.assert_allclose(s, b, rtol=1e-13, atol=1e-15)
    np.testing.assert_array_equal(d, 0.0)
    np.testing.assert_allclose(state[:, :C] + 1j * state[:, C:], b, rtol=1e-13, atol=1e-15)


def test_constant_vacancy_matches_lfilter():
    """z_v constant in time => a = (1-v)*lam constant => s = lfilter([1], [1, -a], b)."""
    rng = np.random.default_rng(2)
    B, T, C = 2, 300, 12
    raw = rng.normal(size=(B, T, 3 * C)) * 1.5
    raw[:, :, 2 * C:] = rng.normal(size=(B, 1, C))  # broadcast over t
    tr, ti, gamma = (t.double().numpy() for t in _params(C, seed=2))
    read, _ = oracle.scan_f64(raw, tr, ti, gamma)
    s, d = _split(read)
    v, b = _np_gates(raw, gamma)
    lam = tr + 1j * ti
    for bi in range(B):
        for c in range(C):
            a = (1.0 - v[bi, 0, c]) * lam[c]
            expect = lfilter([1.0], [1.0, -a], b[bi, :, c])
            np.testing.assert_allclose(s[bi, :, c], expect, rtol=1e-11, atol=1e-13)
            prev = np.concatenate([[0.0], expect[:-1]])
            np.testing.assert_allclose(d[bi, :, c], v[bi, 0, c] * lam[c] * prev, rtol=1e-11, atol=1e-13)


def test_geometric_series():
    """Constant inputs: s_t = b (1 - a^{t+1}) / (1 - a)."""
    B, T, C = 1, 200, 8
    rng = np.random.default_rng(3)
    row = rng.normal(size=(3 * C,))
    raw = np.broadcast_to(row, (B, T, 3 * C)).copy()
    tr, ti, gamma = (t.double().numpy() for t in _params(C, seed=3))
    read, _ = oracle.scan_f64(raw, tr, ti, gamma)
    s, _ = _split(read)
    v, b = _np_gates(row[None, None], gamma)
    a = (1.0 - v[0, 0]) * (tr + 1j * ti)
    t = np.arange(T)[:, None]
    expect = b[0, 0] * (1.0 - a[None, :] ** (t + 1)) / (1.0 - a[None, :])
    np.testing.assert_allclose(s[0], expect, rtol=1e-11, atol=1e-13)


def test_zero_vacancy_gives_zero_state():
    B, T, C = 2, 40, 8
    rng = np.random.default_rng(4)
    raw = rng.normal(size=(B, T, 3 * C))
    raw[..., 2 * C:] = -1e4  # sigmoid -> 0
    tr, ti, gamma = (t.double().numpy() for t in _params(C))
    read, state = oracle.scan_f64(raw, tr, ti, gamma)
    np.testing.assert_array_equal(read, 0.0)
    np.testing.assert_array_equal(state, 0.0)


def test_real_rotation_free_channel():
    """theta = 0 and z_i = 0: the imaginary parts vanish identically."""
    B, T, C = 2, 64, 8
    rng = np.random.default_rng(5)
    raw = rng.normal(size=(B, T, 3 * C))
    raw[..., C:2 * C] = 0.0
    rl, _ = ref.init_radius_theta(C)
    tr, ti, gamma = ref.transition_params(rl, torch.zeros(C))
    read, _ = oracle.scan_f64(raw, tr, ti, gamma)
    np.testing.assert_array_equal(read[..., C:2 * C], 0.0)
    np.testing.assert_array_equal(read[..., 3 * C:], 0.0)
    assert np.abs(read[..., :C]).max() > 1e-3


# ---------------------------------------------------------------------------------------------
# invariants and restatement agreement
# ---------------------------------------------------------------------------------------------

def test_step_identity_and_bound():
    """s_t + disp_t = lam*s_{t-1} + b_t, and |s| <= max|b| / (1 - max|a|)."""
    B, T, C = 2, 257, 16
    rng = np.random.default_rng(6)
    raw = rng.normal(size=(B, T, 3 * C)) * 3
    tr, ti, gamma = (t.double().numpy() for t in _params(C, seed=6))
    read, _ = oracle.scan_f64(raw, tr, ti, gamma)
    s, d = _split(read)
    v, b = _np_gates(raw, gamma)
    lam = tr + 1j * ti
    prev = np.concatenate([np.zeros((B, 1, C)), s[:, :-1]], axis=1)
    np.testing.assert_allclose(s + d, lam * prev + b, rtol=1e-12, atol=1e-14)
    amax = np.abs((1 - v) * lam).max()
    assert amax <= 0.99995 + 1e-12
    assert np.abs(s).max() <= np.abs(b).max() / (1 - amax) + 1e-12


@pytest.mark.parametrize("block", [1, 8, 16, 32, 64])
def test_blocked_restatement_matches_sequential(block):
    B, T, C = 2, 133, 24
    g = torch.Generator().manual_seed(block)
    raw = torch.randn(B, T, 3 * C, generator=g) * 2
    tr, ti, gamma = _params(C, seed=block)
    r64, _ = oracle.scan_f64(raw, tr, ti, gamma)
    r32 = ref.field_read(raw, tr, ti, gamma, block)
    assert oracle.rel_err(r32, r64) <= 2e-6


def test_state_continuation_and_decode():
    B, T, C, cut = 2, 90, 16, 41
    rng = np.random.default_rng(7)
    raw = rng.normal(size=(B, T, 3 * C))
    tr, ti, gamma = (t.double().numpy() for t in _params(C, seed=7))
    full, s_full = oracle.scan_f64(raw, tr, ti, gamma)
    head, s_head = oracle.scan_f64(raw[:, :cut], tr, ti, gamma)
    tail, s_tail = oracle.scan_f64(raw[:, cut:], tr, ti, gamma, state_in=s_head)
    np.testing.assert_allclose(np.concatenate([head, tail], 1), full, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(s_tail, s_full, rtol=1e-13, atol=1e-15)
    state = np.zeros((B, 2 * C))
    for t in range(T):
        row, state = oracle.decode_step_f64(raw[:, t], tr, ti, gamma, state)
        np.testing.assert_allclose(row, full[:, t], rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(state, s_full, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(s_full, full[:, -1, :2 * C], rtol=0, atol=0)


def test_causality_prefix():
    """The reference's own causality check (prefix 23 of 37, canon:1456-1461)."""
    B, T, C = 2, 37, 32
    rng = np.random.default_rng(8)
    raw = rng.normal(size=(B, T, 3 * C))
    tr, ti, gamma = (t.double().numpy() for t in _params(C))
    full, _ = oracle.scan_f64(raw, tr, ti, gamma)
    pre, _ = oracle.scan_f64(raw[:, :23], tr, ti, gamma)
    np.testing.assert_array_equal(full[:, :23], pre)


def test_planted_sign_error_is_caught():
    """A plausible transcription slip (disp = -v*lam*s) fails the step identity check."""
    B, T, C = 1, 50, 8
    rng = np.random.default_rng(9)
    raw = rng.normal(size=(B, T, 3 * C))
    tr, ti, gamma = (t.double().numpy() for t in _params(C))
    read, _ = oracle.scan_f64(raw, tr, ti, gamma)
    s, d = _split(read)
    v, b = _np_gates(raw, gamma)
    lam = tr + 1j * ti
    prev = np.concatenate([np.zeros((B, 1, C)), s[:, :-1]], axis=1)
    planted = -d  # the mistake, planted on the CPU
    assert not np.allclose(s + planted, lam * prev + b, rtol=1e-6, atol=1e-9)
    # and a transposed (re, im) readout fails the lfilter-backed constant-vacancy identity
    swapped = read.copy()
    swapped[..., :C], swapped[..., C:2 * C] = read[..., C:2 * C], read[..., :C]
    s2, _ = _split(swapped)
    assert not np.allclose(s2 + d, lam * prev + b, rtol=1e-6, atol=1e-9)


def test_row_wise_metric_sees_what_the_norm_wise_one_divides_away():
    """oracle.rel_err_rows normalises every (row, plane) by its own scale: a 1e-3 relative error
    in a row 1e-3 the size of the largest (an early displaced-readout row, say) is 1e-6 of the
    tensor's maximum, under the 1e-4 bar of rel_err, but 1e-3 row by row. A planted error in one
    plane of one row is attributed to that plane; an all-zero row is compared absolutely."""
    rng = np.random.default_rng(12)
    exp = rng.normal(size=(3, 5, 4 * 8))
    exp[1, 2] *= 1e-3
    got = exp.copy()
    got[1, 2] *= 1.0 + 1e-3
    assert oracle.rel_err(got, exp) < 1e-5
    assert oracle.rel_err_rows(got, exp, planes=4) == pytest.approx(1e-3, rel=1e-6)
    assert oracle.rel_err_rows(exp, exp, planes=4) == 0.0
    # one plane of one row off by 2e-3 of that plane's own maximum
    got = exp.copy()
    k = int(np.argmax(np.abs(exp[0, 0, 16:24])))
    got[0, 0, 16 + k] += 2e-3 * np.abs(exp[0, 0, 16:24]).max()
    assert oracle.rel_err_rows(got, exp, planes=4) == pytest.approx(2e-3, rel=1e-6)
    assert oracle.rel_err_rows(got, exp, planes=1) < 2e-3
    # an expected row of zeros: absolute difference
    exp0 = np.zeros((2, 8))
    got0 = exp0.copy()
    got0[1, 3] = 5e-5
    assert oracle.rel_err_rows(got0, exp0) == pytest.approx(5e-5)
    with pytest.raises(ValueError):
        oracle.rel_err_rows(np.zeros((2, 6)), np.zeros((2, 6)), planes=4)
