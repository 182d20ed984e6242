"""Grouped dispatch (pairs sorted by expert, one read of an expert's tile per
work item of up to 16 tokens): identical outputs to the per-pair kernels and
parity with the oracle, including BASELINE config 3 (T=128, Zipf(1.1))."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import FFN_BAR, MFMA_TOL, Q4K_TOL, rel_max, to_np
from moe_cases import _expert_set, _layer, _oracle_layer, _small
from oracle import moe as OM

pytestmark = pytest.mark.gpu


def _pair_and_grouped(cfg, t):
    return _layer(cfg, t, "t64", dispatch="pairs"), _layer(cfg, t, "t64", dispatch="grouped")


@pytest.mark.parametrize("T", [1, 3, 8, 17, 64, 200])
def test_grouped_equals_pairs_bitwise(dev, T):
    """Same K-chunks and summation order per token: the dispatch does not change a bit."""
    from nurostream_amd import synth
    cfg = _small("gptoss-small")
    t = synth.make_layer(cfg, seed=11, device=dev)
    lp, lg = _pair_and_grouped(cfg, t)
    h = synth.activations(T, cfg.n_embd, seed=100 + T, device=dev)
    op, ip, wp = lp(h)
    og, ig, wg = lg(h)
    assert torch.equal(ip, ig) and torch.equal(wp, wg)
    assert torch.equal(op, og)


@pytest.mark.parametrize("T", [8, 15, 40])
def test_grouped_one_hot_expert(dev, T):
    """Every token routed to the same experts (a bias that dominates the logits):
    one expert holds all pairs, several items per expert from 17 tokens (below
    16 tokens the gate/up kernel sorts the pairs itself)."""
    from nurostream_amd import synth
    cfg = _small("gptoss-small")
    t = synth.make_layer(cfg, seed=12, device=dev)
    b = torch.full((cfg.n_expert,), -50.0, device=dev)
    b[[3, 7, 8, 12]] = 50.0
    t["router_b"] = b
    lp, lg = _pair_and_grouped(cfg, t)
    h = synth.activations(T, cfg.n_embd, seed=7, device=dev)
    op, ip, _ = lp(h)
    og, ig, _ = lg(h)
    assert torch.equal(ip, ig) and torch.equal(op, og)
    assert set(np.unique(to_np(ig)).tolist()) == {3, 7, 8, 12}
    ref, rid, _, _ = _oracle_layer(cfg, t, h.cpu().numpy())
    assert rel_max(to_np(og), ref) < MFMA_TOL


def test_grouped_splits_large_batches(dev):
    """More than 4096 pairs: forward runs grouped passes in token order."""
    from nurostream_amd import synth
    cfg = _small("gptoss-small")
    t = synth.make_layer(cfg, seed=13, device=dev)
    lp, lg = _pair_and_grouped(cfg, t)
    T = 4096 // cfg.top_k + 77
    h = synth.activations(T, cfg.n_embd, seed=3, device=dev)
    op, ip, _ = lp(h)
    og, ig, _ = lg(h)
    assert torch.equal(ip, ig) and torch.equal(op, og)
    ref, rid, _, _ = _oracle_layer(cfg, t, h[-40:].cpu().numpy())
    assert rel_max(to_np(og[-40:]), ref) < MFMA_TOL


def test_grouped_phases_match_forward(dev):
    from nurostream_amd import _native as N
    from nurostream_amd import synth
    cfg = _small("gptoss-small")
    t = synth.make_layer(cfg, seed=14, device=dev)
    lg = _layer(cfg, t, "t64", dispatch="grouped")
    T = 33
    h = synth.activations(T, cfg.n_embd, seed=4, device=dev)
    out, ids, w = lg(h)
    o2 = torch.empty_like(out)
    i2 = torch.empty_like(ids)
    w2 = torch.empty_like(w)
    ws = lg.new_workspace(T)
    for ph in (N.PHASE_ROUTER, N.PHASE_GATE_UP, N.PHASE_DOWN, N.PHASE_COMBINE):
        lg.phase(ph, h, o2, i2, w2, ws)
    assert torch.equal(out, o2) and torch.equal(ids, i2) and torch.equal(w, w2)


def _near_tie_tokens(logits, k, h, W, b):
    """Tokens whose k-th/(k+1)-th logit gap is within the fp32 error bound of the router's dot."""
    bound = 4 * np.finfo(np.float32).eps * (np.abs(h) @ np.abs(W).T).max(axis=1) * np.sqrt(h.shape[1])
    return OM.topk_margin(logits, k) <= bound


def _check_all_tokens(cfg, t, h, ids, wts, out, tol, ex=None, oracle=None):
    """Every token against the oracle: ids and weights exact (weights to 1e-5) outside fp32 near-ties
    of the router, outputs of those tokens within tol of max|y_ref|. oracle: a cached
    _oracle_layer result for the same inputs."""
    hn = h.cpu().numpy()
    ref, rid, rw, rlog = oracle if oracle is not None else _oracle_layer(cfg, t, hn, ex=ex)
    Wn = t["router_w"].float().cpu().numpy()
    # (Qwen3 selects on the softmax of the logits, which keeps their order: the same margin rule)
    bn = t["router_b"].float().cpu().numpy() if cfg.router_mode == "gptoss" else None
    ok = ~_near_tie_tokens(rlog, cfg.top_k, hn, Wn, bn)
    assert ok.sum() >= len(hn) - 2, int(ok.sum())
    got_ids = to_np(ids)
    if cfg.router_mode == "gptoss":
        np.testing.assert_array_equal(got_ids[ok], rid[ok])
        np.testing.assert_allclose(to_np(wts)[ok], rw[ok], rtol=1e-5)
    else:  # Qwen3: the same set (slot order of equal probabilities aside)
        np.testing.assert_array_equal(np.sort(got_ids[ok], 1), np.sort(rid[ok], 1))
    y = to_np(out)
    err = float(np.abs(y[ok] - ref[ok]).max() / np.abs(ref).max())
    assert err < tol, err
    return err


def test_config3_gptoss_t128_zipf(dev):
    """the GPT-OSS-120B-shaped MXFP4 layer at T=128 with
    router logits skewed to Zipf(1.1) expert popularity. Grouped == per-pair
    bit for bit on all 128 tokens, and all 128 against the oracle (ids exact
    outside fp32 near-ties of the router, outputs within the MFMA bound)."""
    from nurostream_amd import synth
    cfg = synth.GPTOSS_120B
    t, c = synth.make_zipf_layer(cfg, seed=0, device=dev)
    lp, lg = _pair_and_grouped(cfg, t)
    h = synth.activations(128, cfg.n_embd, seed=5, device=dev)
    og, ig, wg = lg(h)
    op, ip, wp = lp(h)
    assert torch.equal(ig, ip) and torch.equal(og, op)
    ids = to_np(ig)
    counts = np.bincount(ids.reshape(-1), minlength=cfg.n_expert)
    distinct = int((counts > 0).sum())
    assert 40 < distinct < 128, distinct  # skewed, not uniform (uniform: ~126 of 128)
    del lp, op, ip, wp
    torch.cuda.empty_cache()
    err = _check_all_tokens(cfg, t, h, ig, wg, og, min(FFN_BAR, MFMA_TOL), ex=_expert_set(cfg, t))
    print(f"config 3: {distinct} distinct experts, max rel err {err:.2e} over 128 tokens", flush=True)


def test_config3_graph_replays_bit_stable(dev):
    """The config 3 layer captured as a graph: the gate/up workgroups past the
    first two rounds take units from per-XCD counters that the sort kernel zeroes
    on every launch, so each replay -- back to back, and after eager forwards of
    other tokens on the same workspace -- gives the eager output bit for bit."""
    from nurostream_amd import synth
    cfg = synth.GPTOSS_120B
    t, _ = synth.make_zipf_layer(cfg, seed=0, device=dev)
    lg = _layer(cfg, t, "t64", dispatch="grouped")
    h = synth.activations(128, cfg.n_embd, seed=5, device=dev)
    h2 = synth.activations(128, cfg.n_embd, seed=6, device=dev)
    ref = [x.clone() for x in lg(h)]
    out, ids, wts = torch.empty_like(ref[0]), torch.empty_like(ref[1]), torch.empty_like(ref[2])
    lg(h, out=out, ids=ids, weights=wts)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s), torch.cuda.graph(g, stream=s):
        lg(h, out=out, ids=ids, weights=wts)
    for i in range(4):
        out.zero_()
        ids.fill_(-1)
        if i % 2:
            lg(h2)  # eager work on the same workspace between replays
        torch.cuda.synchronize()
        g.replay()
        if i == 3:
            g.replay()  # and two replays back to back
        torch.cuda.synchronize()
        assert torch.equal(out, ref[0]) and torch.equal(ids, ref[1]) and torch.equal(wts, ref[2]), i
    # phase by phase on one workspace, the down phase three times over: its persistent kernel takes units from
    # counters that no sort zeroes in between, so each launch must leave them as it found them
    from nurostream_amd import _native as N
    ws = lg.new_workspace(128)
    out2, ids2, wts2 = torch.full_like(out, float("nan")), torch.full_like(ids, -1), torch.empty_like(wts)
    for ph in (N.PHASE_ROUTER, N.PHASE_GATE_UP, N.PHASE_DOWN, N.PHASE_DOWN, N.PHASE_DOWN, N.PHASE_COMBINE):
        lg.phase(ph, h, out2, ids2, wts2, ws)
        if ph == N.PHASE_DOWN:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    assert torch.equal(out2, ref[0]) and torch.equal(ids2, ref[1])


def _q4k_pair_and_grouped(cfg, t):
    return _layer(cfg, t, "gguf", dispatch="pairs"), _layer(cfg, t, "gguf", dispatch="grouped")


@pytest.mark.parametrize("T", [1, 5, 8, 40])
def test_grouped_q4k_equals_pairs_bitwise(dev, T):
    """Grouped Q4_K (rows in registers, the item's tokens one at a time) keeps
    each (pair, row)'s arithmetic: identical to the per-pair Q4_K kernels."""
    from nurostream_amd import synth
    cfg = _small("qwen3-small")
    t = synth.make_layer(cfg, seed=21, device=dev)
    lp, lg = _q4k_pair_and_grouped(cfg, t)
    h = synth.activations(T, cfg.n_embd, seed=200 + T, device=dev)
    op, ip, wp = lp(h)
    og, ig, wg = lg(h)
    assert torch.equal(ip, ig) and torch.equal(wp, wg)
    assert torch.equal(op, og)
    ref, _, _, _ = _oracle_layer(cfg, t, h.cpu().numpy())
    assert rel_max(to_np(og), ref) < Q4K_TOL


@pytest.fixture(scope="module")
def config4_t32(dev):
    """The config 4 layer at T=32, the per-pair (int8 dot) outputs and the oracle's, built once for the
    tests below and freed after them (later tests look at fresh device allocations)."""
    from nurostream_amd import synth
    cfg = synth.QWEN3_235B
    t = synth.make_layer(cfg, seed=0, device=dev)
    h = synth.activations(32, cfg.n_embd, seed=9, device=dev)
    op, ip, wp = _layer(cfg, t, "gguf", dispatch="pairs")(h)
    c = dict(cfg=cfg, t=t, h=h, op=op, ip=ip, wp=wp, oracle=_oracle_layer(cfg, t, h.cpu().numpy()))
    yield c
    c.clear()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def test_config4_qwen3_t32_grouped(config4_t32):
    """BASELINE config 4 at T=32: the Qwen3-235B-shaped Q4_K layer, grouped
    == per-pair on all 32 tokens, and all 32 against the oracle."""
    c = config4_t32
    cfg, t, h = c["cfg"], c["t"], c["h"]
    oa, ia, wa = _layer(cfg, t, "gguf", dispatch="grouped")(h)
    assert torch.equal(ia, c["ip"]) and torch.equal(oa, c["op"])
    _check_all_tokens(cfg, t, h, ia, wa, oa, Q4K_TOL, oracle=c["oracle"])


@pytest.mark.parametrize("T,scale", [(1, 1.0), (5, 1.0), (8, 1.0), (40, 1.0), (5, 1e3), (5, 1e-3)])
def test_mfma_q4k_matches_oracle_and_pairs(dev, T, scale):
    """NSX_DISPATCH_MFMA (grouped Q4_K on the matrix cores: f16 products of the exact sc * q
    codes with a two-term split of power-of-two-scaled activations): the same routing as the
    per-pair kernels (int8 dot), outputs within 1e-5 of the float64 oracle and within the
    per-pair kernels' bound of theirs, also for activations scaled far from 1 (T=40 splits
    busy experts over several work items)."""
    from nurostream_amd import synth
    cfg = _small("qwen3-small")
    t = synth.make_layer(cfg, seed=21, device=dev)
    lp = _layer(cfg, t, "gguf", dispatch="pairs")
    lm = _layer(cfg, t, "gguf", dispatch="mfma")
    h = synth.activations(T, cfg.n_embd, seed=300 + T, device=dev) * scale
    op, ip, wp = lp(h)
    om, im, wm = lm(h)
    assert torch.equal(ip, im) and torch.equal(wp, wm)
    assert bool(torch.isfinite(om).all())
    assert rel_max(to_np(om), to_np(op)) < Q4K_TOL
    ref, _, _, _ = _oracle_layer(cfg, t, h.cpu().numpy())
    assert rel_max(to_np(om), ref) < 1e-5


def test_config4_qwen3_t32_mfma(config4_t32):
    """BASELINE config 4 at T=32 on the matrix cores: within the per-pair kernels' bound of
    theirs on all 32 tokens, and all 32 against the oracle."""
    c = config4_t32
    cfg, t, h = c["cfg"], c["t"], c["h"]
    om, im, wm = _layer(cfg, t, "gguf", dispatch="mfma")(h)
    assert torch.equal(im, c["ip"])
    assert rel_max(to_np(om), to_np(c["op"])) < Q4K_TOL
    _check_all_tokens(cfg, t, h, im, wm, om, 1e-5, oracle=c["oracle"])
