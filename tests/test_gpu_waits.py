"""GPU: a look-back wait that gives up is visible: its outputs are NaN, every kernel returns, and
the next call on the workspace raises RuntimeError (the kernels set a host-visible word named in
the workspace header, so no device read is needed).

The failure is forced from the host, with every kernel still exiting normally: the workspace's
ticket counter is pre-seeded so that a launch hands out only its last few tickets (the blocks
with the others refuse and exit), so the tiles that do run wait on predecessors that never
publish, and the header's spin limit is 16 polls. The launch after it finds the counter re-armed
(blocks that refused count toward the launch's end) and is correct again.
"""
from __future__ import annotations

import pytest
import torch

import oracle
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu

TICKET_OFFSET = 256


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
    return ref.transition_params(rl + 0.5 * torch.randn(C, generator=g), th + 0.3 * torch.randn(C, generator=g))


def _seed_counter(ws, epoch, first_ticket):
    """Ticket counter word: epoch in the high half, the next ticket to hand out in the low half."""
    word = torch.tensor([(epoch << 32) | first_ticket], dtype=torch.int64).view(torch.uint8)
    ws[TICKET_OFFSET:TICKET_OFFSET + 8].copy_(word)


# T = 66 chunks of 128 steps: more than 64 chunks per chain, so tickets come from the counter
CASES = [(1, 66 * 128, 64, "plain"), (1, 66 * 128 - 5, 128, "norm")]


@pytest.mark.parametrize("B,T,C,kind", CASES, ids=[c[3] for c in CASES])
def test_given_up_wait_poisons_outputs_and_raises(dev, B, T, C, kind, monkeypatch):
    from fields_lm_amd import ScanPlan
    from fields_lm_amd import _native as nat

    monkeypatch.setattr(nat, "CHECK_WAITS", False)  # the default reporting path, not the check mode
    print(f"[case] forced give-up {kind} B={B} T={T} C={C}", flush=True)
    g = torch.Generator().manual_seed(T + C)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16)
    tr, ti, gamma = _params(C, seed=C)
    weight = torch.rand(4 * C, generator=g) + 0.5
    kw = {} if kind == "plain" else {"norm_weight": weight.to(dev)}
    plan = ScanPlan(raw.to(dev), tr.to(dev), ti.to(dev), gamma.to(dev), **kw)
    n_ctiles = (C + 63) // 64
    n_chunks = (T + 127) // 128
    n_tiles = B * n_ctiles * n_chunks
    ws = plan.workspace
    sentinel = 7.0
    plan.read.fill_(sentinel)
    # only the last chunk's tiles run (one channel tile waits for its chain's predecessors, and
    # in the norm case also for the partner channel tile of its rows, which never runs)
    keep = 1 if kind == "norm" else n_ctiles
    _seed_counter(ws, epoch=5, first_ticket=n_tiles - keep)
    nat.set_spin_limit(ws, 16)
    plan.run()
    torch.cuda.synchronize()  # every kernel returned
    err = nat.workspace_error(ws)
    assert err & 1 and err & 2, hex(err)  # a wait gave up; tickets past the launch were refused
    read = plan.read.cpu()
    t_last = (n_chunks - 1) * 128
    ran = read[:, t_last:]
    if kind == "plain":
        assert bool(torch.isnan(ran).all())  # the carry was missing: every value is poisoned
    else:
        c_tile = slice(64, 128)  # the tile that ran: the second channel tile
        planes = [ran[..., p * C:(p + 1) * C][..., c_tile] for p in range(4)]
        assert all(bool(torch.isnan(x).all()) for x in planes)
    assert bool((read[:, :t_last] == sentinel).all())  # tiles that never ran wrote nothing
    # reported at the next call on the workspace, without a device read
    with pytest.raises(RuntimeError, match="wait give up"):
        plan.run()
    # the counter was re-armed by the failed launch: the next call is correct again
    nat.set_spin_limit(ws, 0)
    out = plan.run()
    torch.cuda.synchronize()
    assert nat.workspace_error(ws) == 0
    exp, _ = oracle.scan_f64(raw.float(), tr, ti, gamma)
    if kind == "norm":
        exp = oracle.rms_norm_f64(exp, weight)
    assert oracle.rel_err(out.cpu(), exp) <= 1e-4


def test_given_up_backward_wait_poisons_gradients(dev, monkeypatch):
    from fields_lm_amd import _native as nat
    from fields_lm_amd import field_scan, field_scan_backward

    monkeypatch.setattr(nat, "CHECK_WAITS", False)  # the default reporting path, not the check mode
    B, T, C = 1, 66 * 64, 64  # 66 chunks of 64 steps (the backward's tiles): counter tickets
    print(f"[case] forced give-up backward B={B} T={T} C={C}", flush=True)
    g = torch.Generator().manual_seed(11)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(dev)
    tr, ti, gamma = (t.to(dev) for t in _params(C, seed=3))
    read = field_scan(raw, tr, ti, gamma)
    gread = torch.randn(B, T, 4 * C, generator=g).to(dev)
    field_scan_backward(raw, tr, ti, gamma, read, gread)  # creates the stream's backward workspace
    torch.cuda.synchronize()
    ws = nat.scan_workspace(dev, 0, "backward")
    n_tiles = 66
    _seed_counter(ws, epoch=9, first_ticket=n_tiles - 3)
    nat.set_spin_limit(ws, 16)
    g_raw, g_tr, g_ti, g_gm = field_scan_backward(raw, tr, ti, gamma, read, gread)
    torch.cuda.synchronize()
    err = nat.workspace_error(ws)
    assert err & 1 and err & 2, hex(err)
    # tickets are taken in reverse time order: the tiles that ran hold the first rows in time
    # order 63..65 from the end, i.e. rows 0 .. 3*64; their carries were missing
    assert bool(torch.isnan(g_raw[:, :3 * 64]).all())
    # the parameter gradients sum the partials of every tile, and the refused tiles wrote none:
    # the reduction launch poisons them when the scan refused tickets
    for grad in (g_tr, g_ti, g_gm):
        assert bool(torch.isnan(grad).all())
    with pytest.raises(RuntimeError, match="wait give up"):
        field_scan_backward(raw, tr, ti, gamma, read, gread)
    nat.set_spin_limit(ws, 0)
    g_raw2, g_tr2, _, _ = field_scan_backward(raw, tr, ti, gamma, read, gread)
    torch.cuda.synchronize()
    assert nat.workspace_error(ws) == 0
    r = raw.double().cpu().requires_grad_()
    p = [t.double().cpu().requires_grad_() for t in (tr, ti, gamma)]
    out, _ = oracle.scan_f64_autograd(r, *p)
    (out * gread.double().cpu()).sum().backward()
    assert oracle.rel_err(g_raw2.cpu(), r.grad) <= 1e-4
    assert oracle.rel_err(g_tr2.cpu(), p[0].grad) <= 1e-4


def test_workspace_at_a_reused_address_has_its_own_guard(dev, monkeypatch):
    """A plan whose workspace is allocated where a freed plan's workspace was (the caching
    allocator hands the block back) gets a guard of its own: its header names its own host word,
    and a forced give-up on it is reported at its next call."""
    import gc

    from fields_lm_amd import ScanPlan
    from fields_lm_amd import _native as nat

    monkeypatch.setattr(nat, "CHECK_WAITS", False)
    B, T, C = 1, 66 * 128, 64
    print(f"[case] reused workspace address B={B} T={T} C={C}", flush=True)
    g = torch.Generator().manual_seed(23)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16).to(dev)
    tr, ti, gamma = (t.to(dev) for t in _params(C, seed=5))
    plan = ScanPlan(raw, tr, ti, gamma)
    plan.run()
    torch.cuda.synchronize()
    first = plan.workspace.data_ptr()
    del plan
    gc.collect()
    plan = ScanPlan(raw, tr, ti, gamma)
    ws = plan.workspace
    guard = nat._guards[(dev.index, ws.data_ptr())]
    named = int(ws[392:400].cpu().view(torch.int64).item())
    assert named == guard.host_error.data_ptr()
    print(f"[case] same address as the freed plan: {ws.data_ptr() == first}", flush=True)
    _seed_counter(ws, epoch=3, first_ticket=66 - 1)
    nat.set_spin_limit(ws, 16)
    plan.run()
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="wait give up"):
        plan.run()
    nat.set_spin_limit(ws, 0)
    out = plan.run()
    torch.cuda.synchronize()
    exp, _ = oracle.scan_f64(raw.float().cpu(), tr.cpu(), ti.cpu(), gamma.cpu())
    assert oracle.rel_err(out.cpu(), exp) <= 1e-4


def _plant_stale_words(ws):
    """Every 32-bit word after the header set to 2: a status word saying "inclusive state
    published" and data words carrying that tag, for the first epoch after the 30-bit wrap. They
    stand for words left 2^30 launches earlier, with a carry of ~0 that no correct scan has."""
    ws[2048:].view(torch.int32).fill_(2)


def _inputs(B, T, C, seed):
    g = torch.Generator().manual_seed(seed)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16)
    tr, ti, gamma = _params(C, seed=seed + 1)
    return raw, tr, ti, gamma, torch.rand(4 * C, generator=g) + 0.5, torch.randn(B, T, 4 * C, generator=g)


# the wrap launch runs a small shape; the launch after it a larger one, whose look-back reads
# status and data words the small launch never wrote (planted with the new cycle's tags)
SMALL, LARGE = (1, 256, 64), (2, 1000, 128)


@pytest.mark.parametrize("kind", ["plain", "norm", "backward"])
def test_epoch_wrap_clears_published_words(dev, kind):
    """The launch that advances the epoch to 2^30 (whose 30 tag bits are 0) zero-fills the
    workspace after its header, so that no word left from 2^30 launches earlier can pass for one
    of the new cycle. Stale words carrying the new cycle's tags are planted in the whole buffer,
    the epoch is set to 2^30 - 1, and a small shape runs (the wrap launch); a larger shape then
    reads planted words the small one never rewrote. Both are bit-identical to ordinary calls. For
    the forward workspace everything after the header is zero between the two calls. The backward
    keeps the wrap launch's parameter-gradient partials, which its reduction launch reads."""
    from fields_lm_amd import _native as nat
    from fields_lm_amd import field_scan, field_scan_backward, field_scan_norm

    print(f"[case] epoch wrap {kind}", flush=True)
    data = {shape: [t.to(dev) for t in _inputs(*shape, seed=81 + shape[2])] for shape in (SMALL, LARGE)}

    def call(shape):
        raw, tr, ti, gamma, weight, gread = data[shape]
        if kind == "norm":
            return [field_scan_norm(raw, tr, ti, gamma, weight, 1e-6, out_dtype=torch.bfloat16)]
        if kind == "plain":
            return [field_scan(raw, tr, ti, gamma)]
        read = field_scan(raw, tr, ti, gamma)
        return list(field_scan_backward(raw, tr, ti, gamma, read, gread))

    ref_large = [t.clone() for t in call(LARGE)]  # also sizes the stream's workspace for LARGE
    ref_small = [t.clone() for t in call(SMALL)]
    torch.cuda.synchronize()
    ws = nat.scan_workspace(dev, 0, "backward" if kind == "backward" else "forward")
    _plant_stale_words(ws)
    _seed_counter(ws, epoch=(1 << 30) - 1, first_ticket=0)
    wrap_small = call(SMALL)
    torch.cuda.synchronize()
    for x, y in zip(wrap_small, ref_small):
        assert torch.equal(x, y)
    epoch = int(ws[TICKET_OFFSET:TICKET_OFFSET + 8].view(torch.int64).item()) >> 32
    assert epoch == 1 << 30
    if kind != "backward":
        assert int(ws[2048:].count_nonzero()) == 0
    after_large = call(LARGE)
    torch.cuda.synchronize()
    for x, y in zip(after_large, ref_large):
        assert torch.equal(x, y)
    assert nat.workspace_error(ws) == 0


def test_refused_launch_at_the_epoch_wrap_still_clears(dev, monkeypatch):
    """A wrap launch whose every block refuses its ticket (the counter seeded past the launch's
    tiles): the last block to count is one that refused, and it still zero-fills the workspace
    after its header and re-arms the counter for the new cycle. Outputs are left untouched, the
    next call raises, and the call after that is correct."""
    from fields_lm_amd import ScanPlan
    from fields_lm_amd import _native as nat

    monkeypatch.setattr(nat, "CHECK_WAITS", False)  # the default reporting path, not the check mode
    B, T, C = 1, 66 * 128, 64  # 66 chunks: tickets from the counter
    print(f"[case] refused wrap launch B={B} T={T} C={C}", flush=True)
    g = torch.Generator().manual_seed(31)
    raw = (torch.randn(B, T, 3 * C, generator=g) * 2).to(torch.bfloat16).to(dev)
    tr, ti, gamma = (t.to(dev) for t in _params(C, seed=7))
    plan = ScanPlan(raw, tr, ti, gamma)
    ws = plan.workspace
    _plant_stale_words(ws)
    _seed_counter(ws, epoch=(1 << 30) - 1, first_ticket=66)  # every ticket out of range
    plan.read.fill_(7.0)
    plan.run()
    torch.cuda.synchronize()
    assert nat.workspace_error(ws) & 2
    assert bool((plan.read == 7.0).all())
    assert int(ws[2048:].count_nonzero()) == 0
    word = int(ws[TICKET_OFFSET:TICKET_OFFSET + 8].view(torch.int64).item())
    assert word == (1 << 30) << 32  # re-armed: the new cycle's first epoch, ticket 0
    with pytest.raises(RuntimeError, match="ticket"):
        plan.run()
    out = plan.run()
    torch.cuda.synchronize()
    assert nat.workspace_error(ws) == 0
    exp, _ = oracle.scan_f64(raw.float().cpu(), tr.cpu(), ti.cpu(), gamma.cpu())
    assert oracle.rel_err(out.cpu(), exp) <= 1e-4


def test_epoch_wrap_clear_time_at_a_large_workspace(dev):
    """The wrap launch's clear (one wave of the last block, 16 bytes per lane and store) on the
    workspace of B=1, T=65,536, C=512 (config 4, ~67 MB): timed against an ordinary launch of the
    same plan, and the workspace is zero after its header."""
    from fields_lm_amd import ScanPlan
    from fields_lm_amd.workloads import make_scan_workload

    print("[case] epoch wrap clear time, config 4 workspace", flush=True)
    wl = make_scan_workload("scan_b1_t65536_d1024", dev)
    plan = ScanPlan(wl.raw, wl.tr, wl.ti, wl.gamma)
    ws = plan.workspace
    plan.run()
    ref = plan.read.clone()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    plan.run()
    b.record()
    torch.cuda.synchronize()
    ordinary_ms = a.elapsed_time(b)
    _plant_stale_words(ws)
    _seed_counter(ws, epoch=(1 << 30) - 1, first_ticket=0)
    a.record()
    plan.run()
    b.record()
    torch.cuda.synchronize()
    wrap_ms = a.elapsed_time(b)
    print(f"[case] workspace {ws.numel() / 1e6:.1f} MB: ordinary launch {ordinary_ms:.3f} ms, "
          f"wrap launch {wrap_ms:.3f} ms", flush=True)
    assert torch.equal(plan.read, ref)
    assert int(ws[2048:].count_nonzero()) == 0
    assert wrap_ms < 100.0
