"""NeuroStream's host-side surface on the CPU (api.py:30-37, 179-191,
336-341, 399-441): parse_size, sampling, report() after streamed reads, and
close() / the context manager; plus the Arena's first-come-first-served
order and the BlockPrefetcher's handling of blocks the caller passed."""
from __future__ import annotations

import threading
import time

import numpy as np
import pytest
import torch

from nurostream_amd.api import NeuroStream, parse_size
from nurostream_amd.compute import blockffn as B
from nurostream_amd.format.gguf import GGMLType, GGUFWriter
from nurostream_amd.io.arena import Arena, BudgetExceeded


def test_parse_size_forms():
    assert parse_size(123) == 123
    assert parse_size("2GB") == 2 << 30
    assert parse_size("1.5G") == 3 << 29
    assert parse_size("512M") == 512 << 20
    assert parse_size("512MiB") == 512 << 20
    assert parse_size("64k") == 64 << 10
    assert parse_size(" 4096 ") == 4096
    assert parse_size("1T") == 1 << 40
    for bad in ("", "GB", "abc", "-1G", "1.2.3M", "5X"):
        with pytest.raises(ValueError):
            parse_size(bad)


def test_sample_greedy_and_nucleus():
    logits = torch.tensor([0.0, 3.0, 1.0, 2.9])
    assert NeuroStream._sample(logits, 0.0, 0.9) == 1
    torch.manual_seed(0)
    # top_p below the largest probability: only the most likely token remains
    p = torch.softmax(logits, -1)
    assert all(NeuroStream._sample(logits, 1.0, float(p.max()) * 0.5) == 1 for _ in range(50))
    # top_p covering the two largest: only tokens 1 and 3 are ever drawn
    two = float(torch.sort(p, descending=True).values[:2].sum())
    drawn = {NeuroStream._sample(logits, 1.0, two - 1e-6) for _ in range(200)}
    assert drawn <= {1, 3} and len(drawn) == 2
    # top_p = 1 samples the full softmax
    drawn = {NeuroStream._sample(logits, 1.0, 1.0) for _ in range(400)}
    assert drawn == {0, 1, 2, 3}


def test_arena_serves_waiters_in_arrival_order():
    """A large request that arrived first is granted before later small ones."""
    a = Arena(100)
    a.acquire(90)
    order = []

    def take(n, tag):
        a.acquire(n, timeout=5)
        order.append(tag)

    big = threading.Thread(target=take, args=(60, "big"))
    big.start()
    time.sleep(0.05)
    small = threading.Thread(target=take, args=(5, "small"))
    small.start()
    time.sleep(0.05)
    assert order == []  # 10 bytes are free, but the earlier request waits first
    a.release(30)
    time.sleep(0.05)
    assert order == [] and a.used == 60  # still: the big request does not fit yet, the small one queues behind it
    a.release(60)
    big.join(5)
    small.join(5)
    assert sorted(order) == ["big", "small"] and a.used == 65
    assert a.stats.n_waits == 2 and a.stats.peak_bytes == 90
    with pytest.raises(BudgetExceeded):
        a.acquire(101)
    a.reset()
    assert a.used == 0 and "arena" in a.summary()


def _gguf(path, rows=48, K=32, n_expert=2):
    """A gpt-oss GGUF whose expert tensors are F32 (streamable on the CPU)."""
    g = torch.Generator().manual_seed(3)
    w = torch.randn(n_expert * rows, K, generator=g)
    wr = GGUFWriter(path, "gpt-oss")
    for k, v in (("block_count", 1), ("embedding_length", K), ("expert_count", n_expert),
                 ("expert_used_count", 1), ("expert_feed_forward_length", rows)):
        wr.add(f"gpt-oss.{k}", v)
    wr.add_tensor("blk.0.ffn_gate_exps.weight", (n_expert, rows, K), GGMLType.F32, w.numpy().tobytes())
    wr.write()
    return w


def test_report_after_streamed_reads_and_close(tmp_path):
    path = tmp_path / "m.gguf"
    w = _gguf(path)
    with NeuroStream.load(path, device="cpu", mem_budget="64KB", block_rows=8, n_workers=2) as ns:
        name = "blk.0.ffn_gate_exps.weight"
        x = torch.randn(2, 32)
        plan = [(name, 0, 48), (name, 48, 96)]
        with B.BlockPrefetcher(ns.cache, plan, block_rows=8, depth=3) as pf:
            y = torch.cat([B.stream_linear(ns.cache, name, x, block_rows=8, row_start=lo, row_end=hi,
                                           prefetcher=pf) for _, lo, hi in plan], dim=1)
        torch.testing.assert_close(y, x @ w.T, rtol=1e-5, atol=1e-5)
        ns.model.router_stats.record(0, torch.tensor([[1], [0]]))
        rep = ns.report()
        lines = {k.strip(): v for k, v in (line.split(" : ", 1) for line in rep.splitlines())}
        assert set(lines) >= {"model", "device", "arena", "io", "cache", "router", "generate"}
        assert "m.gguf" in lines["model"] and "gpt-oss" in lines["model"]
        st = ns.source.stats
        assert st.requests >= 12 and st.bytes_read >= w.numel() * 4
        assert f"reads: {st.requests}" in lines["io"]
        assert "2 tokens" in lines["router"] and "2 expert reads" in lines["router"]
        assert ns.arena.used == 0 and ns.arena.stats.peak_bytes > 0
    # closed by the context manager: the reader is gone, close() again is harmless
    assert ns.source.reader._handle is None
    ns.close()


def test_prefetcher_drops_blocks_the_caller_passed(tmp_path):
    """A block asked for before it was submitted is read by the caller and
    never read later; every lease comes back."""
    path = tmp_path / "m.gguf"
    w = _gguf(path)
    from nurostream_amd.io.stream import DiskSource
    src = DiskSource(path, Arena(1 << 20), n_workers=2)
    name = "blk.0.ffn_gate_exps.weight"
    x = torch.randn(1, 32)
    with B.BlockPrefetcher(src, [(name, 0, 96)], block_rows=8, depth=1) as pf:
        assert pf.take(name, 40) is None  # not submitted yet: dropped from the plan
        got = pf.take(name, 0)
        assert got is not None
        src.arena.release(got[1])
        seen = []
        for start in range(8, 96, 8):
            r = pf.take(name, start)
            if r is not None:
                seen.append(start)
                src.arena.release(r[1])
        assert 40 not in seen and len(seen) == 10
    assert src.arena.used == 0
    out = B.stream_linear(src, name, x, block_rows=8)
    torch.testing.assert_close(out, x @ w.T, rtol=1e-5, atol=1e-5)
    src.close()
