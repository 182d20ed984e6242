"""BASELINE config 5 at its real shape: 36 GPT-OSS-120B-shaped MXFP4 layers
(128 experts, hidden 2880, top-4) with every expert slab resident in HBM as
t64 tiles (61 GB), chained x <- x + moe_l(rms_norm(x)) as the reference's
decoder wraps its FFN blocks (model/gpt_oss.py:123-177); and config 5b, the
same stack with a seeded 25% of the 512-row expert blocks in pinned host RAM,
read by the kernels over PCIe (model/gpt_oss.py:GptOssHostStreamedStack)."""
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
