"""Parity of the fused router and MoE layer with the CPU oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import FFN_BAR, MFMA_TOL, Q4K_TOL, rel_max, to_np
from moe_cases import _layer, _oracle_layer, _small
from oracle import moe as OM
from oracle import quant as OQ

pytestmark = pytest.mark.gpu

FFN_TOL = FFN_BAR  # north-star parity bar for FFN outputs (max rel, fp32 accumulate)


def _tol(layout, cfg=None):
    """Regression bound: block-scaled MFMA (t64), Q4_K rows on the int8 dot with two-term
    activations, fp32 VALU products (other GGUF rows)."""
    from nurostream_amd.format.gguf import GGMLType
    if layout == "t64":
        return MFMA_TOL
    return Q4K_TOL if cfg is not None and cfg.ggml_type == GGMLType.Q4_K else 1e-5


def _near_tie_tokens(logits, k, h, W, b):
    """Tokens whose k-th/(k+1)-th logit gap is within the fp32 error bound."""
    bound = 4 * np.finfo(np.float32).eps * (np.abs(h) @ np.abs(W).T).max(axis=1) * np.sqrt(h.shape[1])
    return OM.topk_margin(logits, k) <= bound


@pytest.mark.parametrize("mode", ["gptoss", "qwen3"])
@pytest.mark.parametrize("T,E,K,k", [(1, 128, 2880, 4), (8, 128, 2880, 4), (33, 128, 4096, 8), (5, 7, 64, 3)])
@pytest.mark.parametrize("wdt", [torch.bfloat16, torch.float32])
def test_router_topk(dev, mode, T, E, K, k, wdt):
    from nurostream_amd.moe.fused import router_topk
    g = torch.Generator().manual_seed(T * 131 + E + K + k)
    h = torch.randn(T, K, generator=g)
    W = (torch.randn(E, K, generator=g) * 0.02).to(wdt)
    b = torch.randn(E, generator=g) * 0.02 if mode == "gptoss" else None
    ids, wts, logits = router_topk(h.to(dev), W.to(dev), None if b is None else b.to(dev), k, mode)
    hn, Wn = h.numpy(), W.float().numpy()
    bn = None if b is None else b.numpy()
    if mode == "gptoss":
        rid, rw, rlog = OM.route_gptoss(hn, Wn, bn, k)
    else:
        rid, rw, rlog = OM.route_qwen3(hn, Wn, k)
    assert rel_max(to_np(logits), rlog) < 1e-5
    tie = _near_tie_tokens(rlog, k, hn, Wn, bn)
    ok = ~tie
    np.testing.assert_array_equal(to_np(ids)[ok], rid[ok])
    np.testing.assert_allclose(to_np(wts)[ok], rw[ok], rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize("name,layout,T", [("gptoss-120b", "t64", 16), ("gptoss-120b", "t64", 40),
                                           ("qwen3-235b", "gguf", 33), ("gptoss-small", "t64", 70),
                                           ("qwen3-small", "gguf", 17)])
def test_router_mfma_tiles(dev, name, layout, T):
    """T >= 16: the layer's router runs as fp32 MFMA tiles over K-chunks and a
    fixed-order chunk sum fused with the top-k. Logits (read from the
    workspace, where the later phases read them), ids and weights of every
    token against the oracle router; E not a multiple of 64 and T not a
    multiple of 16 exercise the tile masks."""
    from nurostream_amd import _native as N
    from nurostream_amd import synth
    cfg = {"gptoss-120b": synth.GPTOSS_120B, "qwen3-235b": synth.QWEN3_235B}.get(name) or _small(name)
    t = synth.make_layer(cfg, seed=41, device=dev)
    layer = _layer(cfg, t, layout)
    h = synth.activations(T, cfg.n_embd, seed=T, device=dev)
    E, k = cfg.n_expert, cfg.top_k
    out = torch.empty(T, cfg.n_embd, device=dev)
    ids = torch.empty(T, k, dtype=torch.int32, device=dev)
    w = torch.empty(T, k, device=dev)
    ws = layer.new_workspace(T)
    layer.phase(N.PHASE_ROUTER, h, out, ids, w, ws)
    logits = ws[: T * E * 4].view(torch.float32).reshape(T, E)  # the workspace starts with the logits
    hn, Wn = h.cpu().numpy(), t["router_w"].float().cpu().numpy()
    if cfg.router_mode == "gptoss":
        bn = t["router_b"].float().cpu().numpy()
        rid, rw, rlog = OM.route_gptoss(hn, Wn, bn, k)
    else:
        bn = None
        rid, rw, rlog = OM.route_qwen3(hn, Wn, k)
    assert rel_max(to_np(logits), rlog) < 1e-5
    ok = ~_near_tie_tokens(rlog, k, hn, Wn, bn)
    assert ok.sum() >= T - 2
    np.testing.assert_array_equal(to_np(ids)[ok], rid[ok])
    np.testing.assert_allclose(to_np(w)[ok], rw[ok], rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize("name,layout,slabs", [("gptoss-small", "t64", False), ("gptoss-small", "t64", True),
                                               ("gptoss-small", "gguf", False), ("gptoss-small", "gguf", True),
                                               ("qwen3-small", "gguf", False), ("qwen3-small", "gguf", True),
                                               ("qwen3b-small", "gguf", False),
                                               ("q4_0-small", "gguf", False), ("q8_0-small", "gguf", False),
                                               ("q8_0-small", "gguf", True)])
@pytest.mark.parametrize("T", [1, 2, 9])
def test_moe_small_layers(dev, name, layout, slabs, T):
    from nurostream_amd import synth
    cfg = _small(name)
    t = synth.make_layer(cfg, seed=5, device=dev)
    layer = _layer(cfg, t, layout, slabs)
    h = synth.activations(T, cfg.n_embd, seed=T, device="cpu")
    out, ids, w = layer(h.to(dev))
    ref, rid, rw, rlog = _oracle_layer(cfg, t, h.numpy())
    np.testing.assert_array_equal(np.sort(to_np(ids), 1), np.sort(rid, 1))
    assert rel_max(to_np(out), ref) < _tol(layout, cfg)
    # a second call reuses the workspace
    out2, _, _ = layer(h.to(dev))
    assert torch.equal(out, out2)


@pytest.mark.parametrize("dispatch,T", [("pairs", 1), ("pairs", 20), ("grouped", 20), ("mfma", 20)])
def test_q4k_biases_every_dispatch(dev, dispatch, T):
    """Q4_K experts with gate, up and down biases through each Q4_K path (the
    per-pair int8-dot kernels, their grouped form, the matrix-core kernels)
    against the oracle."""
    from nurostream_amd import synth
    cfg = _small("qwen3b-small")
    t = synth.make_layer(cfg, seed=8, device=dev)
    assert t["down_b"] is not None
    layer = _layer(cfg, t, "gguf", dispatch=dispatch)
    h = synth.activations(T, cfg.n_embd, seed=80 + T, device="cpu")
    out, ids, w = layer(h.to(dev))
    ref, rid, rw, rlog = _oracle_layer(cfg, t, h.numpy())
    np.testing.assert_array_equal(np.sort(to_np(ids), 1), np.sort(rid, 1))
    assert rel_max(to_np(out), ref) < _tol("gguf", cfg)


N_DECODE = 8  # single-token calls per full-shape decode test


def _decode_calls(layer, h):
    """Each row of h through the layer as its own T=1 call (decode batch 1)."""
    outs, ids, ws = zip(*(layer(h[i:i + 1]) for i in range(h.shape[0])))
    return torch.cat(outs), torch.cat(ids), torch.cat(ws)


@pytest.mark.parametrize("layout", ["t64", "gguf"])
def test_gptoss_layer_decode(dev, layout):
    """GPT-OSS-120B-shaped MXFP4 layer at decode batch 1,
    eight tokens each in its own call, every one against the oracle."""
    from nurostream_amd import synth
    cfg = synth.GPTOSS_120B
    t = synth.make_layer(cfg, seed=0, device=dev)
    layer = _layer(cfg, t, layout)
    h = synth.activations(N_DECODE, cfg.n_embd, seed=1, device="cpu")
    out, ids, w = _decode_calls(layer, h.to(dev))
    ref, rid, rw, rlog = _oracle_layer(cfg, t, h.numpy())
    ok = ~_near_tie_tokens(rlog, cfg.top_k, h.numpy(), t["router_w"].float().cpu().numpy(),
                           t["router_b"].float().cpu().numpy())
    assert ok.sum() >= N_DECODE - 1
    np.testing.assert_array_equal(to_np(ids)[ok], rid[ok])
    np.testing.assert_allclose(to_np(w)[ok], rw[ok], rtol=1e-5)
    err = float(np.abs(to_np(out)[ok] - ref[ok]).max() / np.abs(ref).max())
    assert err < FFN_TOL
    assert err < _tol(layout), err


def test_qwen3_layer_decode(dev):
    """BASELINE config 4 at T=1: Qwen3-235B-shaped Q4_K layer, eight tokens
    each in its own call, every one against the oracle."""
    from nurostream_amd import synth
    cfg = synth.QWEN3_235B
    t = synth.make_layer(cfg, seed=0, device=dev)
    layer = _layer(cfg, t, "gguf")
    h = synth.activations(N_DECODE, cfg.n_embd, seed=2, device="cpu")
    out, ids, w = _decode_calls(layer, h.to(dev))
    ref, rid, rw, rlog = _oracle_layer(cfg, t, h.numpy())
    ok = ~_near_tie_tokens(rlog, cfg.top_k, h.numpy(), t["router_w"].float().cpu().numpy(), None)
    assert ok.sum() >= N_DECODE - 1
    np.testing.assert_array_equal(to_np(ids)[ok], rid[ok])
    np.testing.assert_allclose(to_np(w)[ok], rw[ok], rtol=2e-5, atol=1e-6)
    err = float(np.abs(to_np(out)[ok] - ref[ok]).max() / np.abs(ref).max())
    assert err < Q4K_TOL, err


@pytest.mark.parametrize("name,layout,T,dispatch", [("gptoss-small", "t64", 3, "auto"),
                                                    ("gptoss-small", "t64", 20, "auto"),
                                                    ("gptoss-small", "t64", 5, "grouped"),
                                                    ("qwen3-small", "gguf", 1, "auto"),
                                                    ("qwen3-small", "gguf", 2, "auto"),
                                                    ("qwen3-small", "gguf", 17, "auto"),
                                                    ("qwen3-small", "gguf", 3, "mfma"),
                                                    ("qwen3-small", "gguf", 20, "mfma"),
                                                    ("q4_0-small", "gguf", 3, "auto")])
def test_router_phase_alone_writes_ids(dev, name, layout, T, dispatch):
    """NSX_PHASE_ROUTER run on its own leaves the ids and weights written for
    every layout and dispatch (a caller reads them to queue expert block reads
    before the gate/up phase), equal to what the whole forward writes; the
    later phases then give the forward's output. (Matrix-core Q4_K at T=20:
    the forward's router builds h's term rows, the gate/up phase called alone
    builds them itself -- the same bits.)"""
    from nurostream_amd import _native as N
    from nurostream_amd import synth
    cfg = _small(name)
    t = synth.make_layer(cfg, seed=41, device=dev)
    layer = _layer(cfg, t, layout, dispatch=dispatch)
    h = synth.activations(T, cfg.n_embd, seed=42, device=dev)
    ref_out, ref_ids, ref_w = layer.forward(h)
    ws = layer.new_workspace(T)
    out = torch.full_like(ref_out, float("nan"))
    ids = torch.full_like(ref_ids, -1)
    wts = torch.full_like(ref_w, float("nan"))
    layer.phase(N.PHASE_ROUTER, h, out, ids, wts, ws)
    torch.cuda.synchronize()
    assert torch.equal(ids, ref_ids)
    assert torch.equal(wts, ref_w)
    for ph in (N.PHASE_GATE_UP, N.PHASE_DOWN, N.PHASE_COMBINE):
        layer.phase(ph, h, out, ids, wts, ws)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out)


def test_qwen3_one_token_forward_equals_phases(dev):
    """BASELINE config 4 at T=1: the forward (its gate/up kernel selects the
    top-k) and the same layer phase by phase (a top-k launch, gate/up from the
    ids) give equal outputs, ids and weights, also on a repeated forward."""
    from nurostream_amd import _native as N
    from nurostream_amd import synth
    cfg = synth.QWEN3_235B
    t = synth.make_layer(cfg, seed=3, device=dev)
    layer = _layer(cfg, t, "gguf")
    for i in range(2):
        h = synth.activations(1, cfg.n_embd, seed=50 + i, device=dev)
        ref_out, ref_ids, ref_w = layer.forward(h)
        again, _, _ = layer.forward(h)
        ws = layer.new_workspace(1)
        out = torch.full_like(ref_out, float("nan"))
        ids = torch.full_like(ref_ids, -1)
        wts = torch.full_like(ref_w, float("nan"))
        for ph in (N.PHASE_ROUTER, N.PHASE_GATE_UP, N.PHASE_DOWN, N.PHASE_COMBINE):
            layer.phase(ph, h, out, ids, wts, ws)
        torch.cuda.synchronize()
        assert torch.equal(ids, ref_ids) and torch.equal(wts, ref_w)
        assert bool(torch.isfinite(ref_out).all())
        assert torch.equal(out, ref_out) and torch.equal(again, ref_out)
