"""The model-level seams on the device: the GPT-OSS FFN stack (BASELINE
config 5's chain, model/gpt_oss.py:123-177) and the Qwen3 sparse FFN
(moe/router.py:173-219) over a cache that mixes HBM slabs and streamed reads."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import FFN_BAR, MFMA_TOL, rel_max, to_np
from moe_cases import _expert_set, _small
from oracle import moe as OM

pytestmark = pytest.mark.gpu


def _oracle_layers(cfg, seed, n_layers, dev):
    from nurostream_amd import synth
    out = []
    for li in range(n_layers):
        t = synth.make_layer(cfg, seed=seed, device=dev, layer=li)
        out.append((t["router_w"].float().cpu().numpy(), t["router_b"].cpu().numpy(), _expert_set(cfg, t)))
    return out


@pytest.mark.parametrize("T", [1, 5, 15, 16, 20])
def test_stack_norm_in_router_equals_separate_norm(dev, T):
    """GptOssFFNStack.forward runs the block's input norm inside the router
    kernel (MoELayer.forward_norm) where norm_folds(T); spelled out with
    add_rms_norm and forward() per layer the stack gives the same bits, and so
    does forward_norm for one layer below 16 tokens (x_out = x + r, out, ids,
    weights)."""
    from nurostream_amd import synth
    from nurostream_amd.compute.ops import add_rms_norm
    from nurostream_amd.model.gpt_oss import GptOssFFNStack
    cfg = _small("gptoss-small")
    L = 3
    stack = GptOssFFNStack.synthetic(cfg, L, seed=23, device=dev)
    stack.decode_chain = False  # the folded-norm path (one token's decode chain matches it to rounding)
    stack.norm_weights = [None] + [1 + 0.1 * torch.randn(cfg.n_embd, generator=torch.Generator().manual_seed(li))
                                   .to(dev) for li in range(1, L)]
    x = synth.activations(T, cfg.n_embd, seed=11, device=dev)
    y = stack(x)
    res = torch.empty_like(x)
    h = add_rms_norm(x, None, stack.norm_weights[0], 1e-5, sum_out=res)
    for li, layer in enumerate(stack.layers):
        if li:
            h = add_rms_norm(res, o, stack.norm_weights[li], 1e-5, sum_out=res)
        o, ids, w = layer.forward(h)
        if li == 1 and T < 16:  # one layer through forward_norm (the kernel takes T < 16)
            xo = torch.empty_like(x)
            o2 = torch.empty_like(x)
            o2, ids2, w2 = layer.forward_norm(prev_res, prev_o, stack.norm_weights[li], 1e-5, x_out=xo, out=o2)
            assert torch.equal(xo, res)
            assert torch.equal(o2, o) and torch.equal(ids2, ids) and torch.equal(w2, w)
        prev_res, prev_o = res.clone(), o.clone()
    res.add_(o)
    torch.cuda.synchronize()
    assert torch.equal(y, res)


@pytest.mark.parametrize("T,weight", [(2, True), (3, True), (5, True), (9, True), (40, False), (300, True)])
def test_forward_addnorm_equals_forward_then_norm(dev, T, weight):
    """MoELayer.forward_addnorm (nsx_moe_forward_addnorm: the next block's residual add and
    norm in the layer's last launch -- the combine kernel on the grouped path, from 3 tokens;
    a separate add + norm launch per pair)
    against forward() followed by add_rms_norm: the same bits for x + out and the normed
    h, in place (x_out = x, h_out = h) and apart, and the same routing."""
    from nurostream_amd import synth
    from nurostream_amd.compute.ops import add_rms_norm
    from nurostream_amd.moe.fused import MoELayer  # noqa: F401
    cfg = _small("gptoss-small")
    t = synth.make_layer(cfg, seed=31, device=dev)
    from moe_cases import _layer
    layer = _layer(cfg, t, "t64")
    h = synth.activations(T, cfg.n_embd, seed=41, device=dev)
    x = synth.activations(T, cfg.n_embd, seed=42, device=dev)
    w = (1 + 0.1 * torch.randn(cfg.n_embd, generator=torch.Generator().manual_seed(5))).to(dev) if weight else None
    out, ids, wts = layer.forward(h)
    xr = torch.empty_like(x)
    hr = add_rms_norm(x, out, w, 1e-5, sum_out=xr)
    xo, ho = torch.empty_like(x), torch.empty_like(x)
    ids2, wts2 = layer.forward_addnorm(h, x, w, 1e-5, x_out=xo, h_out=ho)
    assert torch.equal(ids2, ids) and torch.equal(wts2, wts)
    assert torch.equal(xo, xr) and torch.equal(ho, hr)
    xi, hi = x.clone(), h.clone()  # in place: x_out = x, h_out = h
    layer.forward_addnorm(hi, xi, w, 1e-5, x_out=xi, h_out=hi)
    assert torch.equal(xi, xr) and torch.equal(hi, hr)
    with pytest.raises(Exception):  # h_out over x
        layer.forward_addnorm(h, xi, w, 1e-5, x_out=xo, h_out=xi)


@pytest.mark.parametrize("name,layout,T", [("gptoss-small", "t64", 1025), ("gptoss-small", "t64", 1026),
                                           ("gptoss-small", "t64", 1027), ("qwen3-small", "gguf", 513),
                                           ("qwen3-small", "gguf", 525)])
def test_forward_addnorm_short_last_pass(dev, name, layout, T):
    """A grouped call longer than one pass (4096 pairs: 1024 tokens at top-4, 512
    at top-8) whose last pass is too short to group under AUTO (t64: fewer than 3
    tokens; Q4_K on the matrix cores: fewer than 104 pairs) runs that pass on the
    per-pair kernels; its x + out and normed rows must still be written, with the
    same bits as forward() followed by add_rms_norm on every token."""
    from nurostream_amd import synth
    from nurostream_amd.compute.ops import add_rms_norm
    from moe_cases import _layer
    cfg = _small(name)
    t = synth.make_layer(cfg, seed=33, device=dev)
    layer = _layer(cfg, t, layout)
    h = synth.activations(T, cfg.n_embd, seed=43, device=dev)
    x = synth.activations(T, cfg.n_embd, seed=44, device=dev)
    w = (1 + 0.1 * torch.randn(cfg.n_embd, generator=torch.Generator().manual_seed(6))).to(dev)
    out, ids, wts = layer.forward(h)
    xr = torch.empty_like(x)
    hr = add_rms_norm(x, out, w, 1e-5, sum_out=xr)
    xo = torch.full_like(x, float("nan"))
    ho = torch.full_like(x, float("nan"))
    ids2, wts2 = layer.forward_addnorm(h, x, w, 1e-5, x_out=xo, h_out=ho)
    torch.cuda.synchronize()
    assert torch.equal(ids2, ids) and torch.equal(wts2, wts)
    tail = slice(T - 8, T)  # the short pass's rows first, so a failure names them
    assert torch.equal(xo[tail], xr[tail]) and torch.equal(ho[tail], hr[tail])
    assert torch.equal(xo, xr) and torch.equal(ho, hr)


@pytest.mark.parametrize("router_dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_decode_chain_matches_separate_norm_and_oracle(dev, router_dtype):
    """One token through a stack as a decode chain (nsx_moe_chain_t1: after the
    first layer no router launch; each down kernel leaves the next layer's
    router shares, each gate/up kernel sums them and quantizes h itself):
    the same routing as the separate-norm path and its outputs to rounding
    (non-unit norm weights), the oracle's chain within the MFMA bound (unit
    weights), and graph replays bit-stable with eager work between them.
    Each router weight dtype the down kernel converts (f32, bf16, f16)."""
    import dataclasses
    from nurostream_amd import synth
    from nurostream_amd.model.gpt_oss import GptOssFFNStack
    cfg = dataclasses.replace(_small("gptoss-small"), router_dtype=router_dtype)
    L = 4
    stack = GptOssFFNStack.synthetic(cfg, L, seed=27, device=dev)
    assert all(layer.chain_share_bytes() > 0 for layer in stack.layers)
    x = synth.activations(1, cfg.n_embd, seed=13, device=dev)
    y = stack(x)
    ids_c = stack.last_routing(1)[0].clone()
    ref = OM.ffn_stack(x.cpu().numpy(), _oracle_layers(cfg, 27, L, dev), cfg.top_k)
    err = rel_max(to_np(y), ref)
    assert err < L * MFMA_TOL, err
    stack.norm_weights = [(1 + 0.1 * torch.randn(cfg.n_embd, generator=torch.Generator().manual_seed(70 + li)))
                          .to(dev) for li in range(L)]
    y_c = stack(x)
    ids_c = stack.last_routing(1)[0].clone()
    stack.decode_chain = False
    y_s = stack(x)
    ids_s = stack.last_routing(1)[0].clone()
    stack.decode_chain = True
    torch.cuda.synchronize()
    assert torch.equal(ids_c, ids_s)
    assert rel_max(to_np(y_c), to_np(y_s)) < 1e-5
    out = torch.empty_like(x)
    stack(x, out=out)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s), torch.cuda.graph(g, stream=s):
        stack(x, out=out)
    for i in range(3):
        out.zero_()
        stack(synth.activations(1, cfg.n_embd, seed=90 + i, device=dev))  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y_c), i


def test_decode_chain_first_layer_is_norm_then_forward(dev):
    """chain_t1 without shares (the first layer) routes from x itself: out,
    ids and weights are forward(add_rms_norm(x) * w) bit for bit, x becomes
    x + out in place, and with a next layer the shares it leaves give that
    layer the routing forward() gives from add_rms_norm of the new x."""
    from nurostream_amd import synth
    from nurostream_amd.compute.ops import add_rms_norm
    from nurostream_amd.model.gpt_oss import GptOssFFNStack
    cfg = _small("gptoss-small")
    stack = GptOssFFNStack.synthetic(cfg, 2, seed=29, device=dev)
    l0, l1 = stack.layers
    w0 = (1 + 0.1 * torch.randn(cfg.n_embd, generator=torch.Generator().manual_seed(3))).to(dev)
    w1 = (1 + 0.1 * torch.randn(cfg.n_embd, generator=torch.Generator().manual_seed(4))).to(dev)
    x = synth.activations(1, cfg.n_embd, seed=17, device=dev)
    o_ref, ids_ref, w_ref = l0.forward(add_rms_norm(x, None, w0, 1e-5))
    xr = x.clone()
    share = torch.zeros(l1.chain_share_bytes(), dtype=torch.uint8, device=dev)
    out = torch.empty_like(x)
    ids = torch.empty(1, cfg.top_k, dtype=torch.int32, device=dev)
    wts = torch.empty(1, cfg.top_k, device=dev)
    l0.chain_t1(xr, w0, 1e-5, None, l1, w1, share, out, ids, wts)
    torch.cuda.synchronize()
    assert torch.equal(out, o_ref) and torch.equal(ids, ids_ref) and torch.equal(wts, w_ref)
    assert torch.equal(xr, x + o_ref)
    o1, ids1_ref, _ = l1.forward(add_rms_norm(xr, None, w1, 1e-5))
    x2 = xr.clone()
    l1.chain_t1(x2, w1, 1e-5, share, None, None, None, out, ids, wts)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids1_ref)
    assert rel_max(to_np(out), to_np(o1)) < 1e-5
    assert torch.equal(x2, xr + out)


def test_decode_chain_refuses_what_it_cannot_run(dev):
    """Layers outside the chain's shapes report no share size and raise
    instead of running: GGUF-layout Q4_K experts, and grouped dispatch."""
    from nurostream_amd import synth
    from moe_cases import _layer
    q = _small("qwen3-small")
    lq = _layer(q, synth.make_layer(q, seed=5, device=dev), "gguf")
    assert lq.chain_share_bytes() < 0
    g = _small("gptoss-small")
    lg = _layer(g, synth.make_layer(g, seed=5, device=dev), "t64", dispatch="grouped")
    assert lg.chain_share_bytes() < 0
    x = torch.zeros(1, g.n_embd, device=dev)
    with pytest.raises(NotImplementedError):
        lg.chain_t1(x, None, 1e-5, None, None, None, None, torch.empty_like(x),
                    torch.empty(1, g.top_k, dtype=torch.int32, device=dev), torch.empty(1, g.top_k, device=dev))


@pytest.mark.parametrize("T", [1, 2, 9])
def test_gptoss_ffn_stack_matches_oracle(dev, T):
    from nurostream_amd import synth
    from nurostream_amd.model.gpt_oss import GptOssFFNStack
    cfg = _small("gptoss-small")
    L = 3
    stack = GptOssFFNStack.synthetic(cfg, L, seed=21, device=dev)
    x = synth.activations(T, cfg.n_embd, seed=9, device=dev)
    y = stack(x)
    ref = OM.ffn_stack(x.cpu().numpy(), _oracle_layers(cfg, 21, L, dev), cfg.top_k)
    err = rel_max(to_np(y), ref)
    assert err < FFN_BAR and err < L * MFMA_TOL, err
    ids, _ = stack.last_routing(T)
    assert ids.shape == (L, T, cfg.top_k)
    # the per-layer seam gives the same first step, and a graph replay the same chain
    x1 = stack._ffn_block(x, 0)
    r1 = OM.ffn_stack(x.cpu().numpy(), _oracle_layers(cfg, 21, 1, dev), cfg.top_k)
    assert rel_max(to_np(x1), r1) < MFMA_TOL
    assert stack.router_stats.tokens_routed == T
    g = torch.cuda.CUDAGraph()
    out = torch.empty_like(x)
    stack(x, out=out)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s), torch.cuda.graph(g, stream=s):
        stack(x, out=out)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y)


def _qwen3_cache(cfg, t, dev, slab_experts):
    from nurostream_amd.format.gguf import GGMLType, tensor_info
    from nurostream_amd.io.arena import Arena
    from nurostream_amd.io.source import HostSource
    from nurostream_amd.residency.cache import TieredCache
    tensors = {}
    Wr = t["router_w"].float().cpu().contiguous()
    info = tensor_info("blk.0.ffn_gate_inp.weight", (cfg.n_expert, cfg.n_embd), GGMLType.F32)
    tensors[info.name] = (info, Wr.reshape(-1).view(torch.uint8).clone())
    for kind in ("gate", "up", "down"):
        rows, K = cfg.rows_K(kind)
        info = tensor_info(f"blk.0.ffn_{kind}_exps.weight", (cfg.n_expert, rows, K), cfg.ggml_type)
        tensors[info.name] = (info, t[kind].cpu())
    src = HostSource(tensors, Arena(64 << 20), device=dev)
    cache = TieredCache(src, device=dev, vram_budget=1 << 20)
    cache.slab_budget = 1 << 30
    for kind in ("gate", "up", "down"):
        rows, _ = cfg.rows_K(kind)
        for e in slab_experts:
            assert cache.admit_slab(f"blk.0.ffn_{kind}_exps.weight", e * rows, (e + 1) * rows)
    return src, cache


@pytest.mark.parametrize("T", [1, 3, 20])
def test_qwen3_moe_ffn_over_cache(dev, T):
    """moe_ffn with half the experts in HBM slabs and the rest streamed from
    pinned host RAM through submit_expert_reads (T=20: dequantize + matmul)."""
    from nurostream_amd import synth
    from nurostream_amd.model.qwen3 import Qwen3MoE, Qwen3MoEConfig
    cfg = _small("qwen3-small")
    t = synth.make_layer(cfg, seed=6, device="cpu")
    src, cache = _qwen3_cache(cfg, t, dev, slab_experts=range(0, cfg.n_expert, 2))
    model = Qwen3MoE(cache, Qwen3MoEConfig(cfg.n_embd, cfg.n_expert, cfg.top_k, cfg.n_ff), dev)
    h = synth.activations(T, cfg.n_embd, seed=T, device="cpu")
    out = model.ffn(h.to(dev), 0)
    torch.cuda.synchronize()
    ref, rid, _, _ = OM.moe_qwen3(h.numpy(), t["router_w"].float().numpy(), cfg.top_k, _expert_set(cfg, t))
    assert rel_max(to_np(out), ref) < 1e-5
    st = model.router_stats
    assert st.tokens_routed == T and st.expert_reads == len(np.unique(rid))
    assert sum(st.hits.values()) == T * cfg.top_k
    assert src.arena.used == 0
    assert cache.stats.slab_hits > 0


@pytest.mark.parametrize("mode", ["stage", "prefetch", "read"])
@pytest.mark.parametrize("T,frac", [(1, 0.5), (5, 0.25), (9, 1.0)])
def test_host_streamed_stack_equals_resident(dev, T, frac, mode):
    """BASELINE config 5b on a small stack: with a share of the row blocks in
    pinned host RAM -- staged per step (all at once, or through
    BlockPrefetcher at depth 4), or read over PCIe by the kernels through
    tile tables -- the outputs equal the resident stack's."""
    from nurostream_amd import synth
    from nurostream_amd.model.gpt_oss import GptOssFFNStack, GptOssHostStreamedStack
    cfg = _small("gptoss-small")
    L = 3
    res = GptOssFFNStack.synthetic(cfg, L, seed=31, device=dev)
    hs = GptOssHostStreamedStack.synthetic(cfg, L, seed=31, device=dev, host_fraction=frac, block_rows=64,
                                           mode=mode)
    # staged modes run add_rms_norm + forward per layer: the resident stack's folded-norm path has their bits
    # (one token's decode chain matches them to rounding); read mode runs the resident stack's own path
    res.decode_chain = mode == "read"
    assert sum(st.host_bytes for st in hs.stores) > 0
    x = synth.activations(T, cfg.n_embd, seed=40 + T, device=dev)
    for _ in range(2):  # a second step reuses the slots and tables
        y_res = res(x)
        y_hs = hs(x)
        torch.cuda.synchronize()
        assert torch.equal(y_res, y_hs)
    if mode == "prefetch":  # every lease returned, never more than depth + 1 blocks held
        ps = hs.prefetch_stats()
        assert ps["blocks"] > 0 and hs.arena.used == 0
        assert 0 < ps["arena_peak"] <= ps["arena_budget"] == 5 * max(
            st.block_bytes[k] for st in hs.stores for k in st.kinds)
        ids, _ = hs.last_routing(T)
        assert hs.bytes_from_host == 2 * hs.host_bytes_of_routing(ids.cpu())
    if mode in ("stage", "prefetch"):
        assert hs.bytes_from_host > 0
        return
    ids, _ = hs.last_routing(T)
    assert hs.host_bytes_of_routing(ids.cpu()) > 0
    # read mode has no host synchronisation: a step is one graph
    x_in = x.clone()
    y_g = torch.empty_like(y_res)
    hs(x_in, out=y_g)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            hs(x_in, out=y_g)
    torch.cuda.synchronize()
    for i in range(4):
        xi = synth.activations(T, cfg.n_embd, seed=60 + i, device=dev)
        x_in.copy_(xi)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_g, res(xi)), i


def test_host_device_address(dev):
    """Pinned host memory maps to a device address; pageable memory is refused."""
    import ctypes as C
    from nurostream_amd import _native as N
    lib = N.load()
    out = C.c_uint64(0)
    pinned = torch.zeros(4096, dtype=torch.uint8).pin_memory()
    assert lib.nsx_host_device_address(pinned.data_ptr(), C.byref(out)) == N.OK and out.value != 0
    pageable = torch.zeros(4096, dtype=torch.uint8)
    assert lib.nsx_host_device_address(pageable.data_ptr(), C.byref(out)) == N.EHIP


def test_gather_and_block_copies_check_ranges(dev):
    from nurostream_amd import _native as N
    import ctypes as C
    lib = N.load()
    a = torch.arange(4096, dtype=torch.uint8, device=dev)
    b = torch.zeros(4096, dtype=torch.uint8, device=dev)
    h = torch.arange(256, dtype=torch.uint8).pin_memory()
    u64 = lambda *v: (C.c_uint64 * len(v))(*v)  # noqa: E731
    i64 = lambda *v: (C.c_int64 * len(v))(*v)  # noqa: E731
    s = N.stream_ptr(dev)
    assert lib.nsx_gather_copy(2, u64(a.data_ptr(), a.data_ptr() + 1024), u64(b.data_ptr() + 16, b.data_ptr() + 2048),
                               i64(512, 1024), s) == N.OK
    assert lib.nsx_copy_blocks_async(1, u64(h.data_ptr()), u64(b.data_ptr() + 3840), i64(256), s, None) == N.OK
    torch.cuda.synchronize()
    assert torch.equal(b[16:528], a[:512]) and torch.equal(b[2048:3072], a[1024:2048])
    assert torch.equal(b[3840:].cpu(), h)
    # misaligned, or past the end of the device allocation (a segment of its
    # own: the check sees allocations, not tensors): rejected before any copy
    assert lib.nsx_gather_copy(1, u64(a.data_ptr() + 8), u64(b.data_ptr()), i64(16), s) == N.EINVAL
    torch.cuda.empty_cache()
    big = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)
    end = big.data_ptr() + big.numel()
    assert lib.nsx_gather_copy(1, u64(a.data_ptr()), u64(end - 512), i64(1024), s) == N.EINVAL
    assert lib.nsx_copy_blocks_async(1, u64(h.data_ptr()), u64(end - 128), i64(256), s, None) == N.EINVAL
    torch.cuda.synchronize()
    assert int(big.sum()) == 0
