"""Weight sources: where raw GGUF bytes come from before the cache.

`row_geometry` is the reference's (io/source.py:38-62). `HostSource` is the
build's replacement for the disk-backed StreamingSource (io/stream.py): the
raw tensors sit in pinned host RAM and `submit_rows` starts an asynchronous
host-to-device copy on a side stream, charged to the arena until the caller
releases it -- the same (future, nbytes) contract as
StreamingSource.submit_rows (io/stream.py:200-216). `BlockReader.wait` plays
AsyncReader.wait (io/reader.py:127-139): it orders the caller's stream after
the copy on the GPU (no host-side block) and counts prefetch hits/misses.
`GGUFSource` serves the same protocol from a GGUF file on disk.
"""
from __future__ import annotations

import mmap
import threading
import time
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from ..format.gguf import GGUFFile, TensorInfo, row_geometry  # noqa: F401  (re-export)
from .arena import Arena


@dataclass
class IOStats:
    requests: int = 0
    bytes_read: int = 0
    stall_seconds: float = 0.0
    prefetch_hits: int = 0
    prefetch_misses: int = 0

    @property
    def prefetch_rate(self) -> float:
        t = self.prefetch_hits + self.prefetch_misses
        return 0.0 if t == 0 else self.prefetch_hits / t

    def summary(self) -> str:
        return (f"{self.bytes_read / 1e9:.2f}GB in {self.requests} reads | "
                f"stall {self.stall_seconds:.2f}s | prefetch {self.prefetch_rate:.1%}")


class BlockFuture:
    """One in-flight row block: a device (or host) tensor and its copy event."""

    __slots__ = ("tensor", "event", "cancelled")

    def __init__(self, tensor: torch.Tensor, event=None) -> None:
        self.tensor = tensor
        self.event = event
        self.cancelled = False

    def done(self) -> bool:
        return self.event is None or self.event.query()

    def result(self) -> torch.Tensor:
        if self.event is not None and self.tensor.is_cuda:
            cur = torch.cuda.current_stream(self.tensor.device)
            cur.wait_event(self.event)
            self.tensor.record_stream(cur)
        return self.tensor

    def cancel(self) -> bool:
        # the copy is already queued; the buffer returns to the allocator when dropped
        self.cancelled = True
        return False


class BlockReader:
    """`wait(fut)` for BlockFuture, with hit/stall accounting."""

    def __init__(self) -> None:
        self.stats = IOStats()
        self._lock = threading.Lock()

    def wait(self, fut: BlockFuture) -> torch.Tensor:
        hit = fut.done()
        with self._lock:
            if hit:
                self.stats.prefetch_hits += 1
            else:
                self.stats.prefetch_misses += 1
        return fut.result()


class _Index:
    def __init__(self, tensors: dict[str, TensorInfo]) -> None:
        self.tensors = tensors


class HostSource:
    """Raw GGUF tensors in host RAM, copied to the device a row block at a time.

    `tensors` maps name -> (TensorInfo, uint8 host tensor of info.nbytes).
    With `device` on a GPU the host bytes are pinned once, at construction,
    and every submitted block is copied on a dedicated side stream.
    """

    def __init__(self, tensors: dict, arena: Arena, device: str | torch.device | None = None,
                 pin: bool = True) -> None:
        self.arena = arena
        self.reader = BlockReader()
        self.device = torch.device(device) if device is not None else torch.device("cpu")
        infos, raw = {}, {}
        cuda = self.device.type == "cuda"
        for name, (info, data) in tensors.items():
            data = data.reshape(-1)
            if data.dtype != torch.uint8 or data.numel() != info.nbytes:
                raise ValueError(f"{name}: expected {info.nbytes} uint8 bytes")
            if cuda and pin and not data.is_pinned():
                data = data.pin_memory()
            infos[name], raw[name] = info, data
        self.gguf = _Index(infos)
        self._raw = raw
        self.reads = 0
        self._copy_stream = torch.cuda.Stream(self.device) if cuda else None

    def _span(self, name: str, start: int, end: int):
        info = self.gguf.tensors[name]
        n_rows, _, rb = row_geometry(info)
        start, end = max(0, start), min(n_rows, end)
        return self._raw[name], start * rb, max(0, end - start) * rb

    def raw_bytes(self, name: str) -> torch.Tensor:
        self.reads += 1
        return self._raw[name]

    def raw_rows(self, name: str, start: int, end: int) -> torch.Tensor:
        self.reads += 1
        data, off, n = self._span(name, start, end)
        return data[off:off + n]

    def fetch_rows(self, name, start, end, device="cpu", dtype=torch.float32):
        from ..compute.quant import dequantize

        info = self.gguf.tensors[name]
        _, elems, rb = row_geometry(info)
        raw = self.raw_rows(name, start, end)
        rows = raw.numel() // rb if rb else 0
        nbytes = raw.numel()
        self.arena.acquire(nbytes)
        try:
            return dequantize(raw.to(device), info.dtype, rows * elems, out_dtype=dtype).reshape(rows, elems)
        finally:
            self.arena.release(nbytes)

    def fetch(self, name, device="cpu", dtype=torch.float32):
        from ..compute.quant import dequantize

        info = self.gguf.tensors[name]
        raw = self.raw_bytes(name).to(device)
        return dequantize(raw, info.dtype, info.n_elements, out_dtype=dtype).reshape(info.torch_shape)

    def submit_rows(self, name: str, start: int, end: int, *, timeout: float | None = None):
        """Start copying rows [start, end); returns (BlockFuture, nbytes). Caller releases."""
        data, off, nbytes = self._span(name, start, end)
        self.arena.acquire(nbytes, timeout=timeout)
        try:
            self.reads += 1
            self.reader.stats.requests += 1
            self.reader.stats.bytes_read += nbytes
            src = data[off:off + nbytes]
            if self._copy_stream is None:
                return BlockFuture(src), nbytes
            cur = torch.cuda.current_stream(self.device)
            dst = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            self._copy_stream.wait_stream(cur)  # dst's allocation is ordered on `cur`
            with torch.cuda.stream(self._copy_stream):
                dst.copy_(src, non_blocking=True)
                ev = torch.cuda.Event()
                ev.record(self._copy_stream)
            dst.record_stream(self._copy_stream)
            return BlockFuture(dst, ev), nbytes
        except BaseException:
            self.arena.release(nbytes)
            raise


class GGUFSource(HostSource):
    """HostSource over the tensors of a GGUF file (memory-mapped, then pinned
    per tensor on first use is avoided: every tensor is copied once into
    pinned RAM at open, which bounds nothing but keeps submit_rows async)."""

    def __init__(self, path: str | Path, arena: Arena, device=None, names=None) -> None:
        g = GGUFFile(path)
        fh = open(g.path, "rb")
        mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
        try:
            tensors = {}
            for name, info in g.tensors.items():
                if names is not None and name not in names:
                    continue
                view = np.frombuffer(mm, dtype=np.uint8, count=info.nbytes, offset=g.file_offset(info))
                tensors[name] = (info, torch.from_numpy(view.copy()))
                del view  # no export of the map may outlive it
        finally:
            mm.close()
            fh.close()
        super().__init__(tensors, arena, device)
        self.gguf = g
        self.gguf.tensors = {n: t for n, t in g.tensors.items() if n in tensors}
