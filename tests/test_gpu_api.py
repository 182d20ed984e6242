"""NeuroStream.load over a GGUF file (api.py:66-237, 342-388): the FFN stack
with all expert slabs in HBM (fused layers), none (the streamed neuron path),
and after pin_hot_experts, against the oracle."""
from __future__ import annotations

import pytest
import torch

from api_cases import oracle_stack, write_gptoss_gguf
from helpers import MFMA_TOL, rel_max, to_np
from moe_cases import _small

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gguf_file(tmp_path_factory):
    cfg = _small("gptoss-small")
    path = tmp_path_factory.mktemp("gguf") / "tiny-gpt-oss.gguf"
    layers = write_gptoss_gguf(path, cfg, n_layers=2, seed=17)
    return path, cfg, layers


def _x(cfg, T):
    from nurostream_amd import synth
    return synth.activations(T, cfg.n_embd, seed=60 + T, device="cpu")


@pytest.mark.parametrize("T", [1, 3])
def test_load_all_slabs_resident_runs_fused_layers(dev, gguf_file, T):
    from nurostream_amd.api import NeuroStream
    path, cfg, layers = gguf_file
    ns = NeuroStream.load(path, device="cuda", slab_budget="1GB", mem_budget="64MB")
    assert ns.cfg.n_layer == 2 and ns.cfg.n_expert == cfg.n_expert and ns.cfg.n_ffn_expert == cfg.n_ff
    assert ns.cache.slab_bytes > 0
    x = _x(cfg, T)
    y = ns.model.ffn_stack(x.to(dev))
    assert all(ns.model._fused_layer(li) is not None for li in range(2))
    assert rel_max(to_np(y), oracle_stack(cfg, layers, x.numpy())) < 2 * MFMA_TOL
    assert ns.model.router_stats.tokens_routed == 2 * T


@pytest.mark.parametrize("T", [1, 4])
def test_load_streamed_neuron_path(dev, gguf_file, T):
    from nurostream_amd.api import NeuroStream
    path, cfg, layers = gguf_file
    ns = NeuroStream.load(path, device="cuda", mem_budget="8MB", block_rows=64, expert_lookahead=4)
    assert ns.cache.slab_bytes == 0
    x = _x(cfg, T)
    y = ns.model.ffn_stack(x.to(dev))
    torch.cuda.synchronize()
    assert rel_max(to_np(y), oracle_stack(cfg, layers, x.numpy())) < 2e-5
    assert ns.arena.used == 0
    st = ns.model.router_stats
    assert st.tokens_routed == 2 * T and sum(st.hits.values()) == 2 * T * cfg.top_k


def test_pin_hot_experts_admits_whole_experts(dev, gguf_file):
    from nurostream_amd.api import NeuroStream
    path, cfg, layers = gguf_file
    per_expert = sum(cfg.expert_bytes(k) for k in ("gate", "up", "down"))
    ns = NeuroStream.load(path, device="cuda", mem_budget="8MB", block_rows=64)
    ns.cache.slab_budget = int(3.5 * per_expert)  # room for three whole experts
    x = _x(cfg, 6)
    ref = oracle_stack(cfg, layers, x.numpy())
    ns.model.ffn_stack(x.to(dev))
    hot = [k for k, _ in ns.model.router_stats.hits.most_common(3)]
    assert ns.pin_hot_experts() == 3
    assert ns.cache.slab_bytes == 3 * per_expert
    for layer, e in hot:
        assert all(ns.cache.has_slab(f"blk.{layer}.ffn_{k}_exps.weight", e * r, (e + 1) * r)
                   for k, r in (("gate", cfg.n_ff), ("up", cfg.n_ff), ("down", cfg.n_embd)))
    assert ns.pin_hot_experts() == 0  # nothing else fits whole
    y = ns.model.ffn_stack(x.to(dev))  # slab hits (t64 MFMA) mixed with streamed blocks
    assert rel_max(to_np(y), ref) < 2 * MFMA_TOL
    with pytest.raises(NotImplementedError):
        next(ns.generate("hello"))
