"""GPU parity of the streaming seam: stream_linear, BlockPrefetcher, HostSource
(pinned host RAM, side-stream copies) and TieredCache slabs, against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import MFMA_TOL, rel_max, to_np
from oracle import moe as OM
from oracle import quant as OQ

pytestmark = pytest.mark.gpu

FFN_TOL = 1e-3  # max|y - y_ref| / max|y_ref|


def _source(tensors, dev, budget=64 << 20):
    from nurostream_amd.io.arena import Arena
    from nurostream_amd.io.source import HostSource
    return HostSource(tensors, Arena(budget), device=dev)


def test_config1_q4_0_stream_linear(dev):
    """Q4_0 4096x4096 (d = fp16 |N(0, 0.02)|, uniform codes), x ~ N(0,1),
    block_rows 512, streamed from pinned host RAM through the fused GEMV."""
    from nurostream_amd import synth
    from nurostream_amd.compute.blockffn import stream_linear
    from nurostream_amd.format.gguf import GGMLType, tensor_info
    g = synth.generator(0, "cpu")
    raw = synth.matrix_bytes(GGMLType.Q4_0, 4096, 4096, g, "cpu")
    x = synth.activations(1, 4096, seed=0, device="cpu")
    info = tensor_info("w", (4096, 4096), GGMLType.Q4_0)
    src = _source({"w": (info, raw)}, dev, budget=4 * 512 * 2304)
    y = stream_linear(src, "w", x.to(dev), block_rows=512, device=dev, lookahead=2)
    torch.cuda.synchronize()
    ref = OQ.gemv(raw.numpy(), OQ.Q4_0, x.numpy(), 4096, 4096, f64=True)
    assert rel_max(to_np(y), ref) < 2e-5
    assert rel_max(to_np(y), ref) < FFN_TOL
    assert src.arena.used == 0 and src.arena.stats.peak_bytes <= src.arena.budget


def test_slab_known_answer_528_on_gpu(dev):
    """The reference's slab KAT (tests/test_tuning.py:104-153) with the slab in HBM."""
    from nurostream_amd.compute.blockffn import stream_linear
    from nurostream_amd.format.gguf import GGMLType, tensor_info
    from nurostream_amd.residency.cache import TieredCache
    row = torch.cat((torch.tensor([1.0], dtype=torch.float16).view(torch.uint8), torch.arange(1, 33, dtype=torch.uint8)))
    info = tensor_info("expert", (1, 4, 32), GGMLType.Q8_0)
    src = _source({"expert": (info, row.repeat(4))}, dev, budget=64)
    cache = TieredCache(src, device=dev)
    cache.slab_budget = info.nbytes
    assert cache.admit_slab("expert", 0, 4)
    reads = src.reads
    for lo, hi in ((0, 1), (1, 3), (2, 4), (0, 4)):
        torch.testing.assert_close(cache.fetch_rows("expert", lo, hi).cpu(),
                                   torch.arange(1, 33).float().repeat(hi - lo, 1))
    out = stream_linear(cache, "expert", torch.ones(2, 32, device=dev), block_rows=1, row_start=0, row_end=4,
                        device=dev)
    torch.testing.assert_close(out.cpu(), torch.full((2, 4), 528.0))
    assert src.reads == reads and src.arena.stats.total_acquired == 0


def _gptoss_small_tensors(dev_gen="cpu"):
    from nurostream_amd import synth
    from nurostream_amd.format.gguf import GGMLType, tensor_info
    cfg = synth.MoEConfig("s", GGMLType.MXFP4, 8, 4, 256, 192, "gptoss", "clamped_swiglu", True, torch.bfloat16)
    t = synth.make_layer(cfg, seed=3, device=dev_gen)
    tensors = {}
    for kind in ("gate", "up", "down"):
        rows, K = cfg.rows_K(kind)
        info = tensor_info(f"blk.0.ffn_{kind}_exps.weight", (cfg.n_expert, rows, K), GGMLType.MXFP4)
        tensors[info.name] = (info, t[kind])
        binfo = tensor_info(f"blk.0.ffn_{kind}_exps.bias", (cfg.n_expert, rows), GGMLType.F32)
        tensors[binfo.name] = (binfo, t[kind + "_b"].reshape(-1).view(torch.uint8).clone())
    return cfg, t, tensors


@pytest.mark.parametrize("mode", ["prefetcher", "async", "t64-slab", "gguf-slab"])
def test_stream_expert_ffn_matches_oracle(dev, mode):
    """An expert's gate/up/down through stream_linear windows (compute/blockffn.py:396-449),
    fed by a layer-wide BlockPrefetcher, per-window async copies, or HBM slabs."""
    from nurostream_amd.compute.blockffn import BlockPrefetcher, stream_expert_ffn
    from nurostream_amd.residency.cache import TieredCache
    cfg, t, tensors = _gptoss_small_tensors()
    src = _source(tensors, dev, budget=6 * 64 * 136)
    provider = src
    if mode.endswith("slab"):
        provider = TieredCache(src, device=dev, slab_layout=mode.split("-")[0])
        provider.slab_budget = 1 << 30
        for kind in ("gate", "up", "down"):
            rows, _ = cfg.rows_K(kind)
            for e in range(cfg.n_expert):
                assert provider.admit_slab(f"blk.0.ffn_{kind}_exps.weight", e * rows, (e + 1) * rows)
    x = torch.randn(2, cfg.n_embd)
    act = lambda g, u: OM.clamped_swiglu(g, u)  # noqa: E731

    def act_t(g, u):
        gc = torch.clamp(g, max=7.0)
        uc = torch.clamp(u, -7.0, 7.0)
        return (uc + 1) * (gc * torch.sigmoid(1.702 * gc))

    ex = OM.ExpertSet(OQ.MXFP4, cfg.n_embd, cfg.n_ff, {k: t[k].numpy() for k in ("gate", "up", "down")},
                      {k: t[k + "_b"].numpy() for k in ("gate", "up", "down")})
    for e in (0, 5):
        plan = [(f"blk.0.ffn_{k}_exps.weight", e * r, (e + 1) * r)
                for k, r in (("gate", cfg.n_ff), ("up", cfg.n_ff), ("down", cfg.n_embd))]
        pf = BlockPrefetcher(provider, plan, block_rows=64, depth=4) if mode == "prefetcher" else None
        try:
            y = stream_expert_ffn(provider, "blk.0.", e, x.to(dev), cfg.n_ff, cfg.n_embd, act_t, block_rows=64,
                                  device=dev, bias=True, lookahead=2, prefetcher=pf)
        finally:
            if pf is not None:
                pf.close()
        torch.cuda.synchronize()
        ref = OM.expert_ffn(ex, e, x.numpy(), act, block_rows=64)
        tol = MFMA_TOL if mode == "t64-slab" else 2e-5  # t64 slabs run on the block-scaled MFMA
        assert rel_max(to_np(y), ref) < tol, (mode, e)
    assert src.arena.used == 0
