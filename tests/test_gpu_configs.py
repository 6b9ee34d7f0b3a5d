"""GPU: the whole-model configurations at full size, and the refresh block against the
reference's fixture on the device.

* Config 3: the promoted 18F/2M/4R model, random init, bf16, prefill of
  B=4 x T=2048 tokens uniform over [0, 16384) (seed 2). Logits are finite; the incremental
  prefill's last-position logits equal the full forward's at the bf16 tolerance (2e-2); one Field
  block's scan + read_norm output, hooked inside the model run, equals the float64 oracle
  (``rms_norm_f64(scan_f64(raw))``) at rows t in {0, 1, 2047} at 1e-4.
* Config 5: B=64 streams, a 2,048-token prompt (seed 5), then decode steps: eager steps and HIP
  graph replays of one step agree bit for bit, every step's logits equal the full forward at the
  same positions at 2e-2, and one Field block's fused step equals the oracle step at 1e-4.
* The refresh block (v21:131-293) against ``model_blocks.npz`` (written from the reference's
  module), forward and prefill-then-step, fp32 on the device at 1e-5 / 1e-4.

The reference path these follow: ``FieldsForCausalLM.forward`` (fields_official.py:276-299) ->
``states_logits`` (official_source/field_fusion_system_smoke_v21.py:619-627).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from fields_lm_amd import model as M

pytestmark = pytest.mark.gpu

TOL = 1e-4
TOL_BF16 = 2e-2


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from fields_lm_amd import _native

    _native.load()
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def promoted(dev):
    lm = M.build_official_fields(device=dev)
    core = M.cast_for_inference(lm.core_model).eval()
    return lm, core


def _field_indices(core):
    return [i for i, k in enumerate(core.kinds()) if k == "field"]


class _Hook:
    """Wraps one mixer method (an instance attribute shadows the class method) and records its
    arguments and result while ``on``."""

    def __init__(self, mixer, name, keep):
        self.mixer, self.name, self.keep = mixer, name, keep
        self.orig = getattr(mixer, name)
        self.records = []
        self.on = True
        setattr(mixer, name, self)

    def __call__(self, *args, **kw):
        before = self.keep(*args, **kw) if self.on else None
        out = self.orig(*args, **kw)
        if self.on:
            self.records.append((before, out))
        return out

    def remove(self):
        delattr(self.mixer, self.name)


def test_config3_prefill_full_size(dev, promoted):
    """Config 3 at its full size: B=4, T=2048, bf16 weights under bf16 autocast."""
    lm, core = promoted
    print("[case] config 3 prefill B=4 T=2048", flush=True)
    torch.manual_seed(2)
    tokens = torch.randint(0, 16384, (4, 2048)).to(dev)
    fidx = _field_indices(core)
    block = core.blocks[fidx[6]]  # a Field block after the first refresh block
    mixer = block.mixer
    mixer.read_dtype = torch.float32  # the fused scan + read_norm then hands out fp32 values
    hook = _Hook(mixer, "normed_read", lambda x, raw=None: raw.detach().float().cpu())
    try:
        with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            _, logits = core.states_logits(tokens)
            hook.on = False
            last, _ = core.prefill(tokens, max_len=2049)
    finally:
        hook.remove()
        mixer.read_dtype = "auto"
    assert logits.shape == (4, 2048, 16384)
    assert bool(torch.isfinite(logits).all())
    assert oracle.rel_err(last.float().cpu(), logits[:, -1].float().cpu()) <= TOL_BF16
    assert len(hook.records) == 1
    raw, normed = hook.records[0]
    assert raw.shape == (4, 2048, 1536) and normed.dtype == torch.float32
    tr, ti, gamma = (t.detach().cpu() for t in mixer.transition())
    read, _ = oracle.scan_f64(raw, tr, ti, gamma)
    rows = [0, 1, 2047]
    exp = oracle.rms_norm_f64(read[:, rows], mixer.read_norm.weight.detach().float().cpu(),
                              mixer.read_norm.eps)
    got = normed[:, rows].float().cpu()
    assert oracle.rel_err(got, exp) <= TOL


def _clone_cache(cache):
    out = {"blocks": [], "softpatch": cache["softpatch"].clone(), "pos": cache["pos"].clone(),
           "params": cache["params"]}
    for st in cache["blocks"]:
        out["blocks"].append({k: v.clone() for k, v in st.items()} if isinstance(st, dict) else st.clone())
    return out


def _copy_cache(dst, src):
    for i, st in enumerate(src["blocks"]):
        if isinstance(st, dict):
            for k, v in st.items():
                dst["blocks"][i][k].copy_(v)
        else:
            dst["blocks"][i].copy_(st)
    dst["softpatch"].copy_(src["softpatch"])
    dst["pos"].copy_(src["pos"])


def test_config5_decode_full_size(dev, promoted):
    """Config 5 at its full size: B=64, a 2,048-token prompt, 8 decode steps eager and as HIP graph
    replays of one captured step."""
    lm, core = promoted
    B, P, N = 64, 2048, 8
    print(f"[case] config 5 decode B={B} prompt={P} steps={N}", flush=True)
    torch.manual_seed(5)
    tokens = torch.randint(0, 16384, (B, P + N)).to(dev)
    fidx = _field_indices(core)
    bi = fidx[9]
    mixer = core.blocks[bi].mixer
    mixer.read_dtype = torch.float32  # fp32 output of the fused step, checked against the oracle
    try:
        with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            _, cache = core.prefill(tokens[:, :P], max_len=P + N + 2)
            fresh = _clone_cache(cache)
            hook = _Hook(mixer, "normed_step",
                         lambda x_t, state, params=None, raw_t=None: (raw_t.detach().float().cpu(),
                                                                      state.detach().clone().cpu()))
            try:
                eager = [core.step(tokens[:, P + i], cache).clone() for i in range(N)]
                hook.on = False
                # capture: warm-up on a side stream, then one step into the graph, from the state
                # after the prompt
                _copy_cache(cache, fresh)
                tok = tokens[:, P].clone()
                s = torch.cuda.Stream()
                s.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(s):
                    core.step(tok, cache)
                torch.cuda.current_stream().wait_stream(s)
                _copy_cache(cache, fresh)
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    out = core.step(tok, cache)
                _copy_cache(cache, fresh)
                for i in range(N):
                    tok.copy_(tokens[:, P + i])
                    graph.replay()
                    torch.cuda.synchronize()
                    assert torch.equal(out, eager[i]), i  # same kernels, same inputs: same bits
                assert int(cache["pos"]) == P + N
            finally:
                hook.remove()
            _, logits = core.states_logits(tokens[:, :P + N])
    finally:
        mixer.read_dtype = "auto"
    got = torch.stack(eager, 1).float().cpu()
    assert bool(torch.isfinite(got).all())
    # the step consuming token P + i predicts token P + i + 1: the forward's logits at P + i
    assert oracle.rel_err(got, logits[:, P:P + N].float().cpu()) <= TOL_BF16
    # the hooked Field block's fused step against the float64 oracle step + RMSNorm
    params = fresh["params"][bi]
    tr, ti, gamma, w = (t.detach().float().cpu() for t in params)
    assert len(hook.records) == N
    for i, ((raw_t, state), normed) in enumerate(hook.records):
        read_t, _ = oracle.decode_step_f64(raw_t, tr, ti, gamma, state)
        exp = oracle.rms_norm_f64(read_t, w, mixer.read_norm.eps)
        assert oracle.rel_err(normed.float().cpu(), exp) <= TOL, i


def _refresh_block(dev, golden_dir):
    d = np.load(golden_dir / "model_blocks.npz")
    sd = {k[len("refresh::param::"):]: torch.from_numpy(d[k]) for k in d.files
          if k.startswith("refresh::param::")}
    blk = M.RefreshBlock(64, 4, 2, 16, 8, 4, 96)
    blk.load_state_dict(sd, strict=True)
    return blk.to(dev).eval(), d


@pytest.mark.parametrize("name", ["long", "short"])
def test_refresh_block_matches_reference_golden_on_gpu(dev, golden_dir, name):
    """FusionRefreshBlockV21 (v21:131-293) fixture, fp32 on the device: the forward, and a prefill
    of part of the sequence followed by single-token steps, both against the reference's output."""
    blk, d = _refresh_block(dev, golden_dir)
    print(f"[case] refresh golden {name}", flush=True)
    x = torch.from_numpy(d[f"refresh::{name}::x"]).to(dev)
    exp = d[f"refresh::{name}::y"]
    T = x.shape[1]
    with torch.no_grad():
        y = blk(x)
        k = max(1, T // 3)
        yp, st = blk.prefill(x[:, :k], max_len=T + 4)
        steps = [blk.step(x[:, t], torch.tensor(t, device=dev), st) for t in range(k, T)]
    assert oracle.rel_err(y.cpu(), exp) <= 1e-5
    assert oracle.rel_err(yp.cpu(), exp[:, :k]) <= 1e-5
    if steps:
        assert oracle.rel_err(torch.stack(steps, 1).cpu(), exp[:, k:]) <= TOL
