"""BASELINE config 5 at its real shape: 36 GPT-OSS-120B-shaped MXFP4 layers
(128 experts, hidden 2880, top-4) with every expert slab resident in HBM as
t64 tiles (61 GB), chained x <- x + moe_l(rms_norm(x)) as the reference's
decoder wraps its FFN blocks (model/gpt_oss.py:123-177, compute/ops.py:14-20);
and config 5b, the same stack with a seeded 25% of the 512-row expert blocks
in pinned host RAM, read by the kernels over PCIe, staged per layer, or
staged through BlockPrefetcher (model/gpt_oss.py:GptOssHostStreamedStack).

The stack folds each block's residual add and norm into other launches (the
router kernel up to two tokens, the combine kernel from three). Spelled out
with the separate add_rms_norm and one forward() per layer, the chain must
give the stack's bits at hidden 2880, where each of the norm's 256 threads
holds 12 values, the last one partial; and each layer, fed the GPU's own
input, must match the oracle's MoE block."""
from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

from helpers import FFN_BAR, MFMA_TOL, rel_max, to_np
from moe_cases import _expert_set
from oracle import moe as OM

pytestmark = pytest.mark.gpu

N_LAYERS = 36
SEED = 5


@pytest.fixture(scope="module")
def stack(dev):
    from nurostream_amd import synth
    from nurostream_amd.model.gpt_oss import GptOssFFNStack
    print(f"[stack_full] building {N_LAYERS} GPT-OSS-120B-shaped layers", flush=True)
    s = GptOssFFNStack.synthetic(synth.GPTOSS_120B, N_LAYERS, seed=SEED, device=dev)
    torch.cuda.synchronize()
    yield s
    del s
    gc.collect()
    torch.cuda.empty_cache()


def _graph_of(stack, x):
    out = torch.empty_like(x)
    stack(x, out=out)  # buffers and workspaces exist before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s), torch.cuda.graph(g, stream=s):
        stack(x, out=out)
    return g, out


@pytest.mark.parametrize("T", [1, 8])
def test_full_stack_graph_equals_eager(dev, stack, T):
    from nurostream_amd import synth
    print(f"[stack_full] T={T} eager vs graph", flush=True)
    x = synth.activations(T, synth.GPTOSS_120B.n_embd, seed=40 + T, device=dev)
    y = stack(x)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y).all())
    ids, wts = stack.last_routing(T)
    assert ids.shape == (N_LAYERS, T, 4)
    assert int(ids.min()) >= 0 and int(ids.max()) < 128
    # every token's four experts are distinct, and its weights sum to one
    srt = torch.sort(ids, dim=-1).values
    assert bool((srt[..., 1:] != srt[..., :-1]).all())
    assert torch.allclose(wts.sum(-1), torch.ones_like(wts.sum(-1)), atol=1e-5)
    g, out = _graph_of(stack, x)
    for _ in range(2):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y)
    # the chain moved x: each layer added its FFN output
    assert float((y - x).abs().max()) > 0


def test_full_stack_layer0_matches_oracle(dev, stack):
    """Layer 0's FFN block for 2 tokens against oracle.moe_gptoss at the real
    shape (128 experts x [2880, 2880] MXFP4, bias, clamped SwiGLU)."""
    from nurostream_amd import synth
    cfg = synth.GPTOSS_120B
    x = synth.activations(2, cfg.n_embd, seed=77, device=dev)
    got = stack._ffn_block(x, 0)
    torch.cuda.synchronize()
    t = synth.make_layer(cfg, seed=SEED, device=dev, layer=0)
    layer0 = [(t["router_w"].float().cpu().numpy(), t["router_b"].cpu().numpy(), _expert_set(cfg, t))]
    del t
    torch.cuda.empty_cache()
    ref = OM.ffn_stack(x.cpu().numpy(), layer0, cfg.top_k)
    err = rel_max(to_np(got), ref)
    assert err < FFN_BAR and err < MFMA_TOL, err


KEEP = (0, 1, 17, 35)  # layers whose inputs and outputs the chain keeps for the oracle


def _norm_weights(n_embd, dev):
    """Non-unit post-attention norm weights, so the fused norms' weight multiply is exercised."""
    return [(1 + 0.1 * torch.randn(n_embd, generator=torch.Generator().manual_seed(1000 + li))).to(dev)
            for li in range(N_LAYERS)]


@pytest.fixture(scope="module", params=[1, 8], ids=["T1", "T8"])
def chain(request, dev, stack):
    """The stack's output over T tokens and the same chain spelled out with
    add_rms_norm + MoELayer.forward per layer, keeping the inputs (x_l before
    the norm, h_l after it), outputs and routing of the KEEP layers on the
    host. At T=1 the stack runs the decode chain (MoELayer.chain_t1), so also:
    the folded-norm path's output (decode_chain off) and the decode chain
    spelled out call by call, with its own KEEP layers' inputs and outputs."""
    from nurostream_amd import synth
    from nurostream_amd.compute.ops import add_rms_norm
    T = request.param
    cfg = synth.GPTOSS_120B
    print(f"[stack_full] chain T={T}: fused stack vs spelled out", flush=True)
    saved = stack.norm_weights
    stack.norm_weights = nw = _norm_weights(cfg.n_embd, dev)
    rec = {"T": T}
    try:  # the weights go back before the fixture returns: later tests of the module share `stack`
        x = synth.activations(T, cfg.n_embd, seed=70 + T, device=dev)
        rec["y"] = stack(x).clone()
        rec["ids_y"], rec["wts_y"] = (t.clone() for t in stack.last_routing(T))
        if T == 1:
            stack.decode_chain = False
            try:
                rec["fold"] = stack(x).clone()
                rec["ids_fold"] = stack.last_routing(T)[0].clone()
            finally:
                stack.decode_chain = True
        res = torch.empty_like(x)
        h = add_rms_norm(x, None, nw[0], 1e-5, sum_out=res)
        kept, ids_c, wts_c = {}, [], []
        for li, layer in enumerate(stack.layers):
            if li:
                h = add_rms_norm(res, o, nw[li], 1e-5, sum_out=res)
            o, ids, w = layer.forward(h)
            ids_c.append(ids.clone())
            wts_c.append(w.clone())
            if li in KEEP:
                x_l = x if li == 0 else res
                kept[li] = tuple(t.cpu().numpy() for t in (x_l, h, o, ids, w)) + (nw[li].cpu().numpy(),)
        res.add_(o)
        rec.update(spelled=res, ids_spelled=torch.stack(ids_c), wts_spelled=torch.stack(wts_c), kept=kept)
        if T == 1:  # the decode chain call by call (the calls stack.forward makes at T=1)
            xs = x.clone()
            o = torch.empty_like(x)
            ids = torch.empty(1, cfg.top_k, dtype=torch.int32, device=dev)
            w = torch.empty(1, cfg.top_k, device=dev)
            share, n, kc = stack._share, len(stack.layers), {}
            for li, layer in enumerate(stack.layers):
                nxt = stack.layers[li + 1] if li + 1 < n else None
                x_l = xs.cpu().numpy() if li in KEEP else None
                layer.chain_t1(xs, nw[li], 1e-5, share if li else None, nxt, None if nxt is None else nw[li + 1],
                               None if nxt is None else share, o, ids, w)
                if li in KEEP:
                    kc[li] = (x_l, None) + tuple(t.cpu().numpy() for t in (o, ids, w)) + (nw[li].cpu().numpy(),)
            rec.update(chain_spelled=xs, kept_chain=kc)
        torch.cuda.synchronize()
    finally:
        stack.norm_weights = saved
    return rec


def test_full_stack_fused_norms_equal_spelled_out_chain(chain):
    """T=8 runs each block's norm inside the combine kernel
    (moe_combine_norm_kernel), T=1 with the decode chain off inside the router
    kernel (nsx_moe_forward_norm): both give the separate add_rms_norm's bits
    at hidden 2880 through all 36 layers. The decode chain (T=1) is its own
    calls spelled out bit for bit, and the separate-norm chain to rounding
    (the rms is summed in another order), with the same routing."""
    if chain["T"] == 8:
        assert torch.equal(chain["ids_y"], chain["ids_spelled"])
        assert torch.equal(chain["wts_y"], chain["wts_spelled"])
        assert torch.equal(chain["y"], chain["spelled"])
        return
    assert torch.equal(chain["fold"], chain["spelled"])
    assert torch.equal(chain["ids_fold"], chain["ids_spelled"])
    assert torch.equal(chain["y"], chain["chain_spelled"])
    assert torch.equal(chain["ids_y"], chain["ids_spelled"])
    err = rel_max(to_np(chain["y"]), to_np(chain["spelled"]))
    print(f"[stack_full] T=1 decode chain vs the separate-norm chain: max rel err {err:.3g}", flush=True)
    assert err < MFMA_TOL, err


def _teacher_forced(dev, layer, x_l, h, o, ids, w, nw, T, what):
    from nurostream_amd import synth
    cfg = synth.GPTOSS_120B
    href = OM.rms_norm(x_l, nw, 1e-5)
    if h is not None:
        assert rel_max(h, href) < 2e-6
    h = href if h is None else h
    t = synth.make_layer(cfg, seed=SEED, device=dev, layer=layer)
    Wr, br = t["router_w"].float().cpu().numpy(), t["router_b"].cpu().numpy()
    per = {k: cfg.expert_bytes(k) for k in ("gate", "up", "down")}
    dev_raw = {k: t[k] for k in ("gate", "up", "down")}
    raw = {k: (lambda e, k=k: dev_raw[k][e * per[k]:(e + 1) * per[k]].cpu().numpy()) for k in per}
    bias = {k: t[k + "_b"].cpu().numpy() for k in ("gate", "up", "down")}
    ex = OM.ExpertSet(int(cfg.ggml_type), cfg.n_embd, cfg.n_ff, raw, bias)
    ref, rid, rw, logits = OM.moe_gptoss(h, Wr, br, cfg.top_k, ex)
    del t, dev_raw
    torch.cuda.empty_cache()
    bound = 4 * np.finfo(np.float32).eps * (np.abs(h) @ np.abs(Wr).T).max(axis=1) * np.sqrt(h.shape[1])
    ok = OM.topk_margin(logits, cfg.top_k) > bound
    assert ok.sum() >= len(ok) - 1, "more than one near-tie token"
    np.testing.assert_array_equal(ids[ok], rid[ok])
    np.testing.assert_allclose(w[ok], rw[ok], rtol=2e-5, atol=1e-6)
    err = rel_max(o[ok], ref[ok])
    print(f"[stack_full] T={T} layer {layer} ({what}): max rel err {err:.3g}", flush=True)
    assert err < FFN_BAR and err < MFMA_TOL, err


@pytest.mark.parametrize("layer", KEEP)
def test_full_stack_layer_matches_oracle_teacher_forced(dev, chain, layer):
    """Layer `layer` of the chain, given the GPU's own input: the norm against
    oracle.rms_norm, the routing and the MoE block against oracle.moe_gptoss
    (ids exact outside fp32 near-ties; output within the MFMA bound on every
    token whose routing is not a near-tie). At T=1 also the decode chain's
    layer (x_l -> oracle.rms_norm -> oracle.moe_gptoss against its output)."""
    _teacher_forced(dev, layer, *chain["kept"][layer], chain["T"], "add_rms_norm + forward")
    if chain["T"] == 1:
        _teacher_forced(dev, layer, *chain["kept_chain"][layer], 1, "decode chain")


@pytest.fixture(scope="module")
def staged_stack(dev):
    """Config 5b with the host blocks staged per layer (modes "stage" and "prefetch" share it)."""
    from nurostream_amd import synth
    from nurostream_amd.model.gpt_oss import GptOssHostStreamedStack
    print("[stack_full] building the 25%-host stack (stage mode)", flush=True)
    hs = GptOssHostStreamedStack.synthetic(synth.GPTOSS_120B, N_LAYERS, seed=SEED, device=dev, host_fraction=0.25,
                                           block_rows=512, mode="prefetch", depth=4)
    torch.cuda.synchronize()
    yield hs
    del hs
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("mode", ["stage", "prefetch"])
@pytest.mark.parametrize("T", [1, 8])
def test_full_stack_host25_staged_equals_resident(dev, stack, staged_stack, mode, T):
    """Config 5b staged per layer -- every host block of the chosen experts
    DMA-copied into a staging slot at once (stage), or read through
    BlockPrefetcher at depth 4 in 512-row blocks (prefetch) -- gives the
    resident stack's outputs bit for bit at the real shape."""
    from nurostream_amd import synth
    hs = staged_stack
    hs.set_mode(mode)
    print(f"[stack_full] host25 {mode} T={T}", flush=True)
    x = synth.activations(T, synth.GPTOSS_120B.n_embd, seed=95 + T, device=dev)
    stack.decode_chain = False  # the staged modes run add_rms_norm + forward per layer: the folded-norm path's bits
    try:
        ref = stack(x)
    finally:
        stack.decode_chain = True
    b0 = hs.bytes_from_host
    got = hs(x)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(hs.last_routing(T)[0], stack.last_routing(T)[0])
    moved = hs.bytes_from_host - b0
    assert moved == hs.host_bytes_of_routing(hs.last_routing(T)[0].cpu()) > 0
    if mode == "prefetch":
        assert hs.arena.used == 0
        assert hs.prefetch_stats()["arena_peak"] <= hs.arena.budget


def test_full_stack_host25_read_equals_resident(dev, stack):
    """Config 5b (25% of the 512-row blocks in pinned host RAM, read over PCIe
    through tile tables) gives the resident stack's outputs bit for bit, at
    T=1 and T=8, eagerly and as a graph."""
    from nurostream_amd import synth
    from nurostream_amd.model.gpt_oss import GptOssHostStreamedStack
    cfg = synth.GPTOSS_120B
    print("[stack_full] building the 25%-host stack (read mode)", flush=True)
    hs = GptOssHostStreamedStack.synthetic(cfg, N_LAYERS, seed=SEED, device=dev, host_fraction=0.25,
                                           block_rows=512, mode="read")
    torch.cuda.synchronize()
    try:
        host_gb = sum(st.host_bytes for st in hs.stores) / 1e9
        assert 0.2 * 60.9 < host_gb < 0.3 * 60.9, host_gb
        for T in (1, 8):
            print(f"[stack_full] host25 T={T}", flush=True)
            x = synth.activations(T, cfg.n_embd, seed=90 + T, device=dev)
            ref = stack(x)
            got = hs(x)
            torch.cuda.synchronize()
            assert torch.equal(got, ref)
            assert torch.equal(hs.last_routing(T)[0], stack.last_routing(T)[0])
            g, out = _graph_of(hs, x)
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
            # the routing touched host blocks: the step really read over PCIe
            assert hs.host_bytes_of_routing(hs.last_routing(T)[0].cpu()) > 0
    finally:
        del hs
        gc.collect()
        torch.cuda.empty_cache()
