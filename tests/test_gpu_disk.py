"""GPU parity of the disk path: nsx_reader reads into device memory (pinned
staging, copies on the reader's stream), and DiskSource under stream_linear,
BlockPrefetcher and stream_expert_ffn, against the file bytes and the oracle."""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from helpers import rel_max, to_np
from oracle import moe as OM
from oracle import quant as OQ

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("direct", [True, False])
def test_disk_reader_device_reads(dev, tmp_path, direct):
    """Spans at odd offsets, split over 1 MiB staging buffers and 8 workers, land in device
    memory byte for byte; the caller's stream is ordered after the copies (no host sync)."""
    from nurostream_amd.io.reader import DiskReader
    data = np.random.default_rng(3).integers(0, 256, (24 << 20) + 4093, dtype=np.uint8)
    path = tmp_path / "blob.bin"
    data.tofile(path)
    rng = random.Random(4)
    with DiskReader(path, n_workers=8, device=dev, direct=direct, slot_bytes=1 << 20, n_slots=12) as r:
        spans = [(0, len(data)), (1, 3), (4097, (3 << 20) + 5)]
        spans += [(o, rng.randint(1, 2_500_000)) for o in (rng.randint(0, len(data) - 2_500_001) for _ in range(40))]
        futs = [(o, n, r.submit(o, n)) for o, n in spans]
        sums = []
        for o, n, f in futs:
            t = r.wait(f)
            assert t.is_cuda and t.numel() == n
            sums.append(t[::4099].to(torch.int64).sum())  # consumed on the current stream right away
        got = torch.stack(sums).cpu().numpy()
        want = np.array([int(data[o:o + n][::4099].astype(np.int64).sum()) for o, n, _ in futs])
        np.testing.assert_array_equal(got, want)
        o, n, f = futs[2]
        assert np.array_equal(f.tensor.cpu().numpy(), data[o:o + n])
        st = r.stats
        assert st.bytes_read == sum(n for _, n in spans) and st.requests == len(spans)


def _write_gguf(path, tensors):
    from nurostream_amd.format.gguf import GGUFWriter
    gw = GGUFWriter(path, "gpt-oss")
    for name, (info, raw) in tensors.items():
        gw.add_tensor(name, info.torch_shape, info.dtype, raw.numpy().reshape(-1))
    gw.write()


def test_disk_config1_q4_0_stream_linear(dev, tmp_path):
    """BASELINE config 1 read from a GGUF file on disk: Q4_0 4096 x 4096, block_rows 512, depth 2."""
    from nurostream_amd import synth
    from nurostream_amd.compute.blockffn import stream_linear
    from nurostream_amd.format.gguf import GGMLType, tensor_info
    from nurostream_amd.io.arena import Arena
    from nurostream_amd.io.stream import DiskSource
    raw = synth.matrix_bytes(GGMLType.Q4_0, 4096, 4096, synth.generator(0, "cpu"), "cpu")
    x = synth.activations(1, 4096, seed=0, device="cpu")
    _write_gguf(tmp_path / "c1.gguf", {"w": (tensor_info("w", (4096, 4096), GGMLType.Q4_0), raw)})
    with DiskSource(tmp_path / "c1.gguf", Arena(4 * 512 * 2304), n_workers=8, device=dev) as src:
        y = stream_linear(src, "w", x.to(dev), block_rows=512, device=dev, lookahead=2)
        torch.cuda.synchronize()
        ref = OQ.gemv(raw.numpy(), OQ.Q4_0, x.numpy(), 4096, 4096, f64=True)
        assert rel_max(to_np(y), ref) < 2e-5
        assert src.arena.used == 0 and src.arena.stats.peak_bytes <= src.arena.budget
        assert src.stats.bytes_read == 4096 * 2304


def test_disk_stream_expert_ffn_prefetcher(dev, tmp_path):
    """A GPT-OSS-shaped MXFP4 expert's gate/up/down streamed from disk through a layer-wide
    BlockPrefetcher (compute/blockffn.py:278-449) against the oracle."""
    from nurostream_amd import synth
    from nurostream_amd.compute.blockffn import BlockPrefetcher, stream_expert_ffn
    from nurostream_amd.format.gguf import GGMLType, tensor_info
    from nurostream_amd.io.arena import Arena
    from nurostream_amd.io.stream import DiskSource
    cfg = synth.MoEConfig("s", GGMLType.MXFP4, 8, 4, 256, 192, "gptoss", "clamped_swiglu", True, torch.bfloat16)
    t = synth.make_layer(cfg, seed=3, device="cpu")
    tensors = {}
    for kind in ("gate", "up", "down"):
        rows, K = cfg.rows_K(kind)
        info = tensor_info(f"blk.0.ffn_{kind}_exps.weight", (cfg.n_expert, rows, K), GGMLType.MXFP4)
        tensors[info.name] = (info, t[kind])
        binfo = tensor_info(f"blk.0.ffn_{kind}_exps.bias", (cfg.n_expert, rows), GGMLType.F32)
        tensors[binfo.name] = (binfo, t[kind + "_b"].reshape(-1).view(torch.uint8).clone())
    _write_gguf(tmp_path / "l.gguf", tensors)

    def act_t(g, u):
        gc = torch.clamp(g, max=7.0)
        uc = torch.clamp(u, -7.0, 7.0)
        return (uc + 1) * (gc * torch.sigmoid(1.702 * gc))

    ex = OM.ExpertSet(OQ.MXFP4, cfg.n_embd, cfg.n_ff, {k: t[k].numpy() for k in ("gate", "up", "down")},
                      {k: t[k + "_b"].numpy() for k in ("gate", "up", "down")})
    x = torch.randn(2, cfg.n_embd)
    with DiskSource(tmp_path / "l.gguf", Arena(6 * 64 * 136), n_workers=4, device=dev) as src:
        for e in (0, 5):
            plan = [(f"blk.0.ffn_{k}_exps.weight", e * r, (e + 1) * r)
                    for k, r in (("gate", cfg.n_ff), ("up", cfg.n_ff), ("down", cfg.n_embd))]
            with BlockPrefetcher(src, plan, block_rows=64, depth=4) as pf:
                y = stream_expert_ffn(src, "blk.0.", e, x.to(dev), cfg.n_ff, cfg.n_embd, act_t, block_rows=64,
                                      device=dev, bias=True, lookahead=2, prefetcher=pf)
            torch.cuda.synchronize()
            ref = OM.expert_ffn(ex, e, x.numpy(), lambda g, u: OM.clamped_swiglu(g, u), block_rows=64)
            assert rel_max(to_np(y), ref) < 2e-5, e
        assert src.arena.used == 0
        st = src.stats
        assert st.prefetch_hits + st.prefetch_misses > 0
