"""Disk-backed weight source (the io/stream.py seam).

`DiskSource` serves the reference's StreamingSource protocol
(io/stream.py:35-227) from a GGUF file through `DiskReader`:
- `submit_rows(name, lo, hi, timeout=None) -> (future, nbytes)`: the arena
  is charged first and released if the submit fails; the caller releases it
  after `reader.wait(fut)`.
- `raw_rows` / `raw_bytes` / `fetch_rows` / `fetch`: blocking reads under
  the arena budget.
- `prefetch(names)` / `prefetch_layer`: whole-tensor reads ahead of use,
  never more than half the budget and never waiting for it, skipping names
  already in flight or absent.
- `drop_inflight`, `close`.

On a GPU source the submitted rows land in device memory (the reader copies
each chunk out of pinned staging as it arrives), so `BlockPrefetcher` and
`stream_linear` consume them like the pinned-RAM `HostSource`'s blocks. The
blocking reads return host tensors, as the reference's do.
"""
from __future__ import annotations

from pathlib import Path

import torch

from ..format.gguf import GGUFFile, row_geometry
from .arena import Arena, BudgetExceeded
from .reader import DEFAULT_WORKERS, DiskReader, ReadFuture

# The GGUF tensor names of one transformer block that prefetch_layer reads
# ahead (the block's non-expert tensors; io/stream.py:22-33 lists the same
# names): attention and norms, then the dense FFN or the MoE router.
_BLOCK_COMMON = ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "attn_q_norm", "attn_k_norm",
                 "ffn_norm")
DENSE_SUFFIXES = tuple(f"{n}.weight" for n in _BLOCK_COMMON + ("ffn_gate", "ffn_up", "ffn_down"))
MOE_SUFFIXES = tuple(f"{n}.weight" for n in _BLOCK_COMMON + ("ffn_gate_inp",))


class DiskSource:
    """WeightSource over a GGUF file on disk, bounded by an Arena."""

    def __init__(self, path: str | Path, arena: Arena, n_workers: int = 16, device=None,
                 direct: bool = True) -> None:
        self.gguf = GGUFFile(path)
        self.arena = arena
        self.device = torch.device(device) if device is not None else torch.device("cpu")
        self.reader = DiskReader(self.gguf.path, n_workers=n_workers, device=self.device, direct=direct)
        self._inflight: dict[str, tuple[ReadFuture, int]] = {}

    @property
    def stats(self):
        return self.reader.stats

    # -- prefetch -------------------------------------------------------------

    def prefetch(self, names) -> int:
        """Read whole tensors ahead of use (io/stream.py:94-124); returns the
        bytes queued. Names already queued or absent from the file are
        skipped; speculative reads take at most half the arena and never wait
        for it (a lease that is not free now ends the batch: the rest is read
        on demand)."""
        wanted = []
        for name in dict.fromkeys(names):
            info = self.gguf.tensors.get(name)
            if info is not None and name not in self._inflight:
                wanted.append((name, info))
        cap, queued = self.arena.budget // 2, 0
        for name, info in wanted:
            if queued + info.nbytes > cap:
                break
            try:
                self.arena.acquire(info.nbytes, timeout=0)
            except (TimeoutError, BudgetExceeded):
                break
            try:
                fut = self.reader.submit(self.gguf.file_offset(info), info.nbytes)
            except BaseException:
                self.arena.release(info.nbytes)
                raise
            self._inflight[name] = (fut, info.nbytes)
            queued += info.nbytes
        return queued

    def prefetch_layer(self, layer: int, moe: bool = False) -> int:
        suffixes = MOE_SUFFIXES if moe else DENSE_SUFFIXES
        return self.prefetch(f"blk.{layer}.{s}" for s in suffixes)

    def drop_inflight(self) -> None:
        """Release everything still queued (io/stream.py:130-135)."""
        for fut, nbytes in list(self._inflight.values()):
            fut.cancel()
            self.arena.release(nbytes)
        self._inflight.clear()

    # -- access ---------------------------------------------------------------

    def _span(self, name: str, start: int, end: int):
        info = self.gguf.tensors[name]
        n_rows, row_elems, row_bytes = row_geometry(info)
        start, end = max(0, start), min(n_rows, end)
        n = max(0, end - start)
        return info, self.gguf.file_offset(info) + start * row_bytes, n * row_bytes, n, row_elems

    def raw_bytes(self, name: str) -> torch.Tensor:
        """A tensor's quantized bytes (host), resolving a pending prefetch (io/stream.py:139-155)."""
        pending = self._inflight.pop(name, None)
        if pending is not None:
            fut, nbytes = pending
            try:
                raw = self.reader.wait(fut)
            finally:
                self.arena.release(nbytes)
            return raw.cpu() if raw.is_cuda else raw
        info = self.gguf.tensors[name]
        self.arena.acquire(info.nbytes)
        try:
            return self.reader.read(self.gguf.file_offset(info), info.nbytes)
        finally:
            self.arena.release(info.nbytes)

    def fetch(self, name: str, device="cpu", dtype: torch.dtype = torch.float32) -> torch.Tensor:
        from ..compute.quant import dequantize
        info = self.gguf.tensors[name]
        raw = self.raw_bytes(name).to(device, non_blocking=True)
        return dequantize(raw, info.dtype, info.n_elements, out_dtype=dtype).reshape(info.torch_shape)

    def fetch_rows(self, name: str, start: int, end: int, device="cpu",
                   dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """Row range = neuron range, dequantized (io/stream.py:161-186)."""
        from ..compute.quant import dequantize
        info, off, nbytes, n, row_elems = self._span(name, start, end)
        if n == 0:
            return torch.empty((0, row_elems), dtype=dtype, device=device)
        self.arena.acquire(nbytes)
        try:
            raw = self.reader.read(off, nbytes).to(device, non_blocking=True)
            return dequantize(raw, info.dtype, n * row_elems, out_dtype=dtype).reshape(n, row_elems)
        finally:
            self.arena.release(nbytes)

    def raw_rows(self, name: str, start: int, end: int) -> torch.Tensor:
        """Quantized bytes of a row range (host), read under the arena budget (io/stream.py:188-198)."""
        _, off, nbytes, _, _ = self._span(name, start, end)
        self.arena.acquire(nbytes)
        try:
            return self.reader.read(off, nbytes)
        finally:
            self.arena.release(nbytes)

    def submit_rows(self, name: str, start: int, end: int, *, timeout: float | None = None):
        """Start reading rows [start, end); (future, nbytes). The caller releases (io/stream.py:200-216)."""
        _, off, nbytes, _, _ = self._span(name, start, end)
        self.arena.acquire(nbytes, timeout=timeout)
        try:
            fut = self.reader.submit(off, nbytes)
        except BaseException:
            self.arena.release(nbytes)
            raise
        return fut, nbytes

    def close(self) -> None:
        self.drop_inflight()
        self.reader.close()

    def __enter__(self) -> "DiskSource":
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()
