"""The disk reader and the disk-backed source on the CPU (no GPU): bytes,
chunking across staging buffers, short reads, time-outs, counters, and the
StreamingSource contract (io/reader.py, io/stream.py) under stream_linear
and BlockPrefetcher with an F32 tensor (the reference's float path)."""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from nurostream_amd.compute import blockffn as B
from nurostream_amd.format.gguf import GGMLType, GGUFWriter, row_geometry
from nurostream_amd.io.arena import Arena
from nurostream_amd.io.reader import DiskReader
from nurostream_amd.io.stream import DiskSource


@pytest.fixture
def blob(tmp_path):
    data = np.random.default_rng(0).integers(0, 256, (1 << 20) + 37, dtype=np.uint8)
    path = tmp_path / "blob.bin"
    data.tofile(path)
    return path, data


@pytest.mark.parametrize("direct", [False, True])
def test_reader_bytes_across_chunks(blob, direct):
    """Spans at odd offsets and sizes, several staging buffers long, come back byte for byte."""
    path, data = blob
    rng = random.Random(1)
    with DiskReader(path, n_workers=4, direct=direct, slot_bytes=16 << 10, n_slots=6) as r:
        spans = [(0, 1), (1, 4095), (4095, 4097), (len(data) - 37, 37), (0, len(data))]
        spans += [(o, rng.randint(0, 200_000)) for o in (rng.randint(0, len(data) - 200_001) for _ in range(40))]
        futs = [(o, n, r.submit(o, n)) for o, n in spans]
        rng.shuffle(futs)
        for o, n, f in futs:
            got = r.wait(f).numpy()
            assert got.shape == (n,) and np.array_equal(got, data[o:o + n]), (o, n)
        assert np.array_equal(r.read(12345, 77777).numpy(), data[12345:12345 + 77777])
        st = r.stats
        assert st.requests == len(spans) + 1
        assert st.bytes_read == sum(n for _, n in spans) + 77777
        assert st.prefetch_hits + st.prefetch_misses == len(spans)
        assert st.wall_seconds >= 0 and st.throughput_gbps >= 0 and "GB/s" in st.summary()


def test_reader_short_read_is_eof_error(blob):
    path, data = blob
    with DiskReader(path, n_workers=2) as r:
        with pytest.raises(EOFError):
            r.read(len(data) - 10, 11)
        with pytest.raises(EOFError):
            r.wait(r.submit(len(data) + 5, 1))
        assert np.array_equal(r.read(0, 10).numpy(), data[:10])  # the reader still works


def test_reader_timeout_and_close(blob):
    """A reader without workers never reads: waits time out and the ticket stays pending; close drops it."""
    path, _ = blob
    r = DiskReader(path, n_workers=0)
    f = r.submit(0, 100)
    assert not f.done()
    with pytest.raises(TimeoutError):
        r.wait(f, timeout=0.01)
    assert not f.retired
    r.close()
    r.close()  # idempotent
    with pytest.raises(RuntimeError):
        r.submit(0, 1)


def test_reader_errors(tmp_path):
    with pytest.raises(OSError):
        DiskReader(tmp_path / "missing.bin")
    with pytest.raises(OSError):
        DiskReader(tmp_path)  # a directory
    (tmp_path / "x.bin").write_bytes(b"abc")
    with pytest.raises(ValueError):
        DiskReader(tmp_path / "x.bin", slot_bytes=4096)  # below the minimum staging size
    with DiskReader(tmp_path / "x.bin") as r:
        assert r.read(0, 0).numel() == 0
        assert bytes(r.read(1, 2).numpy()) == b"bc"


def _f32_gguf(path, rows, K, seed=0):
    w = np.random.default_rng(seed).standard_normal((rows, K)).astype(np.float32)
    gw = GGUFWriter(path, "gpt-oss")
    gw.add_tensor("w", (rows, K), GGMLType.F32, w.reshape(-1).view(np.uint8))
    gw.add_tensor("q", (8, 64), GGMLType.Q4_0,
                  np.random.default_rng(seed + 1).integers(0, 256, 8 * 2 * 18, dtype=np.uint8))
    gw.write()
    return torch.from_numpy(w)


@pytest.mark.parametrize("block_rows", [1, 7, 64])
@pytest.mark.parametrize("depth", [1, 4])
def test_disk_source_under_stream_linear(tmp_path, block_rows, depth):
    """stream_linear's async path over the disk source: same result for every block size and
    depth, every lease returned, peak within budget (tests/test_gpt_oss.py:176-226)."""
    rows, K = 67, 32
    w = _f32_gguf(tmp_path / "m.gguf", rows, K)
    src = DiskSource(tmp_path / "m.gguf", Arena(10 * K * 4), n_workers=3)
    x = torch.from_numpy(np.random.default_rng(1).standard_normal((3, K)).astype(np.float32))
    out = B.stream_linear(src, "w", x, block_rows=block_rows, lookahead=depth)
    torch.testing.assert_close(out, x @ w.T, rtol=1e-5, atol=1e-5)
    assert src.arena.used == 0 and src.arena.stats.peak_bytes <= src.arena.budget
    assert src.stats.bytes_read >= rows * K * 4
    src.close()


def test_disk_source_prefetcher_and_contract(tmp_path):
    rows, K = 40, 16
    w = _f32_gguf(tmp_path / "m.gguf", rows, K)
    path = tmp_path / "m.gguf"
    src = DiskSource(path, Arena(1 << 20), n_workers=2)
    info = src.gguf.tensors["q"]
    raw_file = np.fromfile(path, dtype=np.uint8)
    off = src.gguf.file_offset(info)
    _, _, rb = row_geometry(info)
    # raw_rows / raw_bytes are the file's bytes, clamped like the reference
    assert np.array_equal(src.raw_rows("q", 2, 5).numpy(), raw_file[off + 2 * rb:off + 5 * rb])
    assert src.raw_rows("q", 6, 100).numel() == 2 * rb
    assert np.array_equal(src.raw_bytes("q").numpy(), raw_file[off:off + info.nbytes])
    torch.testing.assert_close(src.fetch("w"), w)
    torch.testing.assert_close(src.fetch_rows("w", 3, 9), w[3:9])
    # submit_rows charges the arena until the caller releases it
    fut, nbytes = src.submit_rows("w", 0, 10)
    assert src.arena.used == nbytes == 10 * K * 4
    torch.testing.assert_close(src.reader.wait(fut).view(torch.float32).reshape(10, K), w[:10])
    src.arena.release(nbytes)
    # prefetch: whole tensors, at most half the budget, absent names skipped
    q = src.prefetch(["w", "missing", "q"])
    assert q == rows * K * 4 + info.nbytes and src.arena.used == q
    assert np.array_equal(src.raw_bytes("q").numpy(), raw_file[off:off + info.nbytes])
    src.drop_inflight()
    assert src.arena.used == 0
    # a plan through the shared BlockPrefetcher
    x = torch.randn(2, K)
    plan = [("w", 0, 20), ("w", 20, 40)]
    with B.BlockPrefetcher(src, plan, block_rows=6, depth=2) as pf:
        out = torch.cat([B.stream_linear(src, "w", x, block_rows=6, row_start=lo, row_end=hi, prefetcher=pf)
                         for _, lo, hi in plan], dim=1)
    torch.testing.assert_close(out, x @ w.T, rtol=1e-5, atol=1e-5)
    assert src.arena.used == 0
    src.close()
