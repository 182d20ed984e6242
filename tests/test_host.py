"""Host-side logic of the path, on the CPU: geometry, GGUF container, arena,
block planning and stream_linear over float weights, residency bookkeeping,
and the rule that quantized compute never falls back to the CPU."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from nurostream_amd import _native as N
from nurostream_amd.compute import blockffn as B
from nurostream_amd.format.gguf import (GGMLType, GGUFFile, GGUFWriter, nbytes_for, row_geometry,
                                        tensor_info)
from nurostream_amd.io.arena import Arena, BudgetExceeded
from nurostream_amd.io.source import HostSource
from nurostream_amd.residency.cache import TieredCache


@pytest.mark.parametrize("dtype,K,row_bytes", [(GGMLType.MXFP4, 2880, 1530), (GGMLType.Q4_K, 4096, 2304),
                                              (GGMLType.Q4_K, 1536, 864), (GGMLType.Q4_0, 4096, 2304),
                                              (GGMLType.Q8_0, 32, 34), (GGMLType.F32, 8, 32)])
def test_row_bytes_at_baseline_shapes(dtype, K, row_bytes):
    """Row sizes of the BASELINE tensors (format/gguf.py:39-68, io/source.py:38-62)."""
    assert nbytes_for(dtype, K) == row_bytes
    info = tensor_info("w", (3, 5, K), dtype)
    assert row_geometry(info) == (15, K, row_bytes)
    assert row_geometry(info) is row_geometry(info)  # memoised on the instance


def test_gguf_container_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    w = rng.integers(0, 256, nbytes_for(GGMLType.MXFP4, 4 * 64), dtype=np.uint8)
    b = rng.standard_normal(7).astype(np.float32)
    path = tmp_path / "t.gguf"
    wr = GGUFWriter(path, "gpt-oss")
    wr.add("gpt-oss.expert_count", 4)
    wr.add("gpt-oss.rope.scale", 0.5)
    wr.add("tokenizer.ggml.tokens", ["a", "bc"])
    wr.add_tensor("blk.0.ffn_gate_exps.weight", (4, 64), GGMLType.MXFP4, w.tobytes())
    wr.add_tensor("blk.0.bias", (7,), GGMLType.F32, b.tobytes())
    wr.write()
    f = GGUFFile(path)
    assert f.arch() == "gpt-oss"
    assert f.cfg("expert_count") == 4
    info = f.tensors["blk.0.ffn_gate_exps.weight"]
    assert info.dtype == GGMLType.MXFP4 and info.torch_shape == (4, 64)
    for name, data in (("blk.0.ffn_gate_exps.weight", w.tobytes()), ("blk.0.bias", b.tobytes())):
        off = f.file_offset(f.tensors[name])
        assert off % 32 == 0
        with open(path, "rb") as fh:
            fh.seek(off)
            assert fh.read(len(data)) == data


def test_arena_budget_rules():
    a = Arena(100)
    a.acquire(60)
    with pytest.raises(BudgetExceeded):
        a.acquire(101)  # larger than the whole budget
    with pytest.raises(TimeoutError):
        a.acquire(50, timeout=0.01)
    a.release(60)
    a.acquire(100, timeout=0)
    assert a.used == 100 and a.stats.peak_bytes == 100
    a.release(100)
    assert a.used == 0


@pytest.mark.parametrize("budget_rows,block_rows,depth", [(2, 512, 2), (9, 4, 8), (100, 512, 4), (1, 8, 2), (3, 1, 1)])
def test_budget_clamp_keeps_depth_plus_one_blocks(budget_rows, block_rows, depth):
    """depth copies in flight plus the one being consumed fit the arena (blockffn.py:123-132,313-325)."""
    rb = 17
    br, d, ok = B._budget_clamp(budget_rows * rb, rb, block_rows, depth)
    if budget_rows < 2:
        assert not ok
        return
    assert ok and 1 <= br <= block_rows and 1 <= d <= depth
    assert (d + 1) * br <= budget_rows or d == 1


def _f32_source(rows, K, budget, seed=0):
    w = torch.from_numpy(np.random.default_rng(seed).standard_normal((rows, K)).astype(np.float32))
    info = tensor_info("w", (rows, K), GGMLType.F32)
    return w, HostSource({"w": (info, w.reshape(-1).view(torch.uint8).clone())}, Arena(budget))


@pytest.mark.parametrize("block_rows", [1, 7, 8, 64, 4096])
@pytest.mark.parametrize("depth", [1, 2, 4, 8])
def test_stream_linear_blocks_depths_and_leases(block_rows, depth):
    """Same result for every block size and lookahead; every lease returned; peak within budget
    (tests/test_gpt_oss.py:176-226, tests/test_tuning.py:78-88)."""
    rows, K = 67, 32
    w, src = _f32_source(rows, K, budget=10 * K * 4)
    x = torch.from_numpy(np.random.default_rng(1).standard_normal((3, K)).astype(np.float32))
    seen = []
    out = B.stream_linear(src, "w", x, block_rows=block_rows, lookahead=depth,
                          callback=lambda n, s, e, y: seen.append((s, e)))
    torch.testing.assert_close(out, x @ w.T, rtol=1e-5, atol=1e-5)
    assert src.arena.used == 0
    assert src.arena.stats.peak_bytes <= src.arena.budget
    assert seen[0][0] == 0 and seen[-1][1] == rows
    assert all(a[1] == b[0] for a, b in zip(seen, seen[1:]))


def test_stream_linear_window_and_errors():
    rows, K = 40, 16
    w, src = _f32_source(rows, K, budget=1 << 20)
    x = torch.randn(2, K)
    out = B.stream_linear(src, "w", x, block_rows=7, row_start=5, row_end=29)
    torch.testing.assert_close(out, x @ w[5:29].T)
    assert B.stream_linear(src, "w", x, row_start=50, row_end=60).shape == (2, 0)
    torch.testing.assert_close(B.stream_linear(src, "w", x, row_start=-3, row_end=400), x @ w.T)
    with pytest.raises(ValueError):
        B.stream_linear(src, "w", x, block_rows=0)
    with pytest.raises(ValueError):
        B.stream_linear(src, "w", torch.randn(2, K + 1))


def test_stream_linear_releases_leases_on_error():
    """An exception mid-stream cancels the queued copies and returns their leases."""
    w, src = _f32_source(64, 16, budget=1 << 20)

    def boom(name, s, e, y):
        if s >= 16:
            raise RuntimeError("stop")

    with pytest.raises(RuntimeError, match="stop"):
        B.stream_linear(src, "w", torch.randn(1, 16), block_rows=8, lookahead=4, callback=boom)
    assert src.arena.used == 0


def test_block_prefetcher_shared_queue():
    """One layer-wide queue serves several windows in plan order, with the same outputs."""
    w, src = _f32_source(48, 16, budget=1 << 20)
    x = torch.randn(2, 16)
    plan = [("w", 0, 20), ("w", 30, 48)]
    with B.BlockPrefetcher(src, plan, block_rows=8, depth=2) as pf:
        assert pf.enabled
        a = B.stream_linear(src, "w", x, block_rows=8, row_start=0, row_end=20, prefetcher=pf)
        b = B.stream_linear(src, "w", x, block_rows=8, row_start=30, row_end=48, prefetcher=pf)
    torch.testing.assert_close(a, x @ w[0:20].T)
    torch.testing.assert_close(b, x @ w[30:48].T)
    assert src.arena.used == 0


def _q8_kat_source(rows=4):
    """Q8_0 rows of d = 1.0 and bytes 1..32, the reference's slab fixture (tests/test_tuning.py:104-133)."""
    row = torch.cat((torch.tensor([1.0], dtype=torch.float16).view(torch.uint8), torch.arange(1, 33, dtype=torch.uint8)))
    info = tensor_info("expert", (1, rows, 32), GGMLType.Q8_0)
    return row, HostSource({"expert": (info, row.repeat(rows))}, Arena(4096))


def test_slab_serves_subranges_without_source_reads():
    """Admitted slabs answer any sub-range of their rows from the slab (cache.py:260-276)."""
    row, src = _q8_kat_source()
    cache = TieredCache(src, device="cpu", slab_layout="gguf")
    cache.slab_budget = 4 * 34
    assert cache.admit_slab("expert", 0, 4)
    reads = src.reads
    assert cache.has_slab("expert", 1, 3) and not cache.has_slab("expert", 3, 5)
    for lo, hi in ((0, 1), (1, 3), (2, 4), (0, 4)):
        raw, dtype = cache.raw_rows("expert", lo, hi)
        assert dtype == GGMLType.Q8_0
        assert torch.equal(raw, row.repeat(hi - lo))
    assert src.reads == reads and cache.stats.slab_misses == 0
    cache2 = TieredCache(src, device="cpu", slab_layout="gguf")
    cache2.slab_budget = 4 * 34 - 1
    assert not cache2.admit_slab("expert", 0, 4)  # over the slab budget
    f32 = TieredCache(_f32_source(4, 8, 1 << 20)[1], device="cpu")
    f32.slab_budget = 1 << 20
    assert not f32.admit_slab("w", 0, 4)  # float tensors are never slabbed


def test_fused_residents_leave_the_tier_together():
    """fuse_vram lays q, k and v out in one buffer; evicting any of them (to
    make room, or by replacing it) takes the whole group and the shared
    buffer, so the tier's byte count matches the storage still alive."""
    rows, K = 4, 32
    blk = torch.cat((torch.tensor([1.0], dtype=torch.float16).view(torch.uint8), torch.arange(1, 33, dtype=torch.uint8)))
    names = ("blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.0.attn_v.weight")
    tensors = {n: (tensor_info(n, (rows, K), GGMLType.Q8_0), blk.repeat(rows)) for n in names + ("blk.0.o.weight",)}
    src = HostSource(tensors, Arena(1 << 20))
    one = rows * 34
    cache = TieredCache(src, device="cpu", vram_budget=3 * one)
    for n in names:
        assert cache.admit_vram(n)
    buf, t = cache.fuse_vram(names)
    assert t == GGMLType.Q8_0 and buf.numel() == 3 * one and cache.stats.vram_bytes == 3 * one
    assert cache.admit_vram("blk.0.o.weight")  # needs room: the LRU resident is q, grouped with k and v
    assert not any(cache.is_resident(n) for n in names)
    assert cache._fused == {} and cache.stats.vram_bytes == one
    # replacing a member also dissolves its group
    cache2 = TieredCache(src, device="cpu", vram_budget=4 * one)
    for n in names:
        assert cache2.admit_vram(n)
    cache2.fuse_vram(names)
    cache2._hbm.put(names[1], cache2._hbm.items[names[1]])
    assert cache2._fused == {} and cache2.is_resident(names[1]) and not cache2.is_resident(names[0])
    assert cache2._hbm.held == one


def test_quantized_compute_never_falls_back_to_cpu():
    """Block formats compute on the GPU only: CPU tensors raise instead of taking a CPU path."""
    from nurostream_amd.compute.kernels import can_fuse, fused_gemv
    from nurostream_amd.compute.quant import dequantize
    raw = torch.zeros(34 * 4, dtype=torch.uint8)
    x = torch.ones(1, 32)
    assert not can_fuse(GGMLType.Q8_0, x)
    with pytest.raises(N.NativeError):
        dequantize(raw, GGMLType.Q8_0, 128)
    with pytest.raises(N.NativeError):
        fused_gemv(raw, GGMLType.Q8_0, x, 4, 32)
    with pytest.raises(TypeError):
        dequantize(raw.view(torch.int8), GGMLType.Q8_0, 128)
    with pytest.raises(N.NativeError):
        dequantize(torch.zeros(210, dtype=torch.uint8), GGMLType.Q6_K, 256)
    with pytest.raises(NotImplementedError):
        dequantize(raw, GGMLType.Q5_K, 128)


def test_router_stats_contract():
    """moe/router.py:26-56: hits per (layer, expert), top_experts, skew, summary; record() counts ids."""
    from nurostream_amd.moe.router import RouterStats
    st = RouterStats()
    assert st.skew() == 0.0
    st.record(0, torch.tensor([[3, 1], [3, 2], [3, 1]]))
    st.record(1, torch.tensor([[0, 5]]))
    assert st.tokens_routed == 4 and st.expert_reads == 3 + 2
    assert st.hits[(0, 3)] == 3 and st.hits[(0, 1)] == 2 and st.hits[(1, 5)] == 1
    assert st.top_experts(0, 2) == [(3, 3), (1, 2)]
    # 5 (layer, expert) entries: the busiest 20% (one entry, 3 hits) of 8 routings
    assert st.skew() == pytest.approx(3 / 8)
    assert "4 tokens" in st.summary() and "5 expert reads" in st.summary()


def test_parse_size_and_api_on_cpu(tmp_path):
    """api.py:30-37 sizes; NeuroStream.load parses the GGUF on any device, but
    its expert path computes on the GPU only (no CPU fallback)."""
    import sys
    from nurostream_amd.api import NeuroStream, parse_size
    assert parse_size("2GB") == 2 << 30 and parse_size("1.5G") == 3 << 29 and parse_size("512M") == 512 << 20
    assert parse_size(" 64K ") == 64 << 10 and parse_size(123) == 123 and parse_size("7") == 7
    with pytest.raises(ValueError):
        parse_size("lots")
    sys.path.insert(0, str(__import__("pathlib").Path(__file__).parent))
    from api_cases import write_gptoss_gguf
    from nurostream_amd import synth
    cfg = synth.MoEConfig("s", GGMLType.MXFP4, 8, 2, 64, 64, "gptoss", "clamped_swiglu", True, torch.bfloat16)
    path = tmp_path / "t.gguf"
    write_gptoss_gguf(path, cfg, n_layers=1, seed=1)
    ns = NeuroStream.load(path, device="cpu")
    assert (ns.cfg.n_layer, ns.cfg.n_embd, ns.cfg.n_expert, ns.cfg.n_expert_used, ns.cfg.n_ffn_expert) == (1, 64, 8, 2, 64)
    with pytest.raises(NotImplementedError):  # no attention tensors in this GGUF
        next(ns.generate([1, 2, 3]))
    with pytest.raises(NotImplementedError):  # text prompts need the tokenizer
        next(ns.generate("hello"))
    with pytest.raises(N.NativeError):
        ns.model._ffn_block(torch.randn(1, 64), 0)
