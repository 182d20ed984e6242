"""Row-window streaming: stream_linear, BlockPrefetcher, stream_expert_ffn.

Behaviour of neurostream/compute/blockffn.py, kept call-compatible:
  stream_linear      :57-241   x @ W[row_start:row_end].T a block of rows at a
                               time; resident / slab windows skip async I/O;
                               async pipelines hold depth+1 leases and clamp
                               block_rows and depth to the arena budget; the
                               next read is submitted before the current block
                               computes; leftover leases are released in
                               `finally`.
  BlockPrefetcher    :278-393  one layer-wide queue of `depth` blocks across
                               every (tensor, window) of a plan; held windows
                               are never queued; a failed submit is retried;
                               a block the caller passes before it was
                               submitted is dropped from the plan.
  stream_expert_ffn  :396-449  gate/up windows + bias row, activation, down
                               window + bias row.
The block product itself is a HIP kernel: `fused_gemv` on raw GGUF bytes or
t64 tiles for up to 16 tokens, else a HIP dequantize plus a matmul.
"""
from __future__ import annotations

from collections import deque
from typing import Callable

import torch

from ..format.gguf import row_geometry
from . import kernels as K
from .quant import dequantize

NeuronCallback = Callable[[str, int, int, torch.Tensor], None]

DEFAULT_BLOCK_ROWS = 1024
DEFAULT_LOOKAHEAD = 2


def _block_product(raw, dtype, x, rows: int, row_elems: int, device, out_dtype, fuse: bool):
    """x @ dequant(raw).T for one block of `rows` rows."""
    if isinstance(raw, torch.Tensor) and raw.device != torch.device(device):
        raw = raw.to(device, non_blocking=True)
    if fuse:
        return K.fused_gemv(raw, dtype, x, rows, row_elems, out_dtype=out_dtype)
    if isinstance(raw, K.T64Rows):
        raw = raw.to_gguf()
    w = dequantize(raw, dtype, rows * row_elems, out_dtype=out_dtype).reshape(rows, row_elems)
    return x.to(out_dtype) @ w.T


def _budget_clamp(budget: int, row_bytes: int, block_rows: int, depth: int):
    """(block_rows, depth, ok): fit depth+1 blocks in the arena, or give up on async."""
    rows_in_budget = budget // max(1, row_bytes)
    if rows_in_budget < 2:
        return 1, depth, False
    block_rows = min(block_rows, max(1, rows_in_budget // (depth + 1)))
    while depth > 1 and (depth + 1) * block_rows > rows_in_budget:
        depth -= 1
    return block_rows, depth, True


def stream_linear(provider, name: str, x: torch.Tensor, block_rows: int = DEFAULT_BLOCK_ROWS,
                  device="cpu", dtype: torch.dtype = torch.float32, callback: NeuronCallback | None = None,
                  out: torch.Tensor | None = None, row_start: int = 0, row_end: int | None = None,
                  lookahead: int = DEFAULT_LOOKAHEAD, prefetcher: "BlockPrefetcher | None" = None):
    """x @ W[row_start:row_end].T, streaming those rows a block at a time. x: (T, in) -> (T, window)."""
    info = provider.gguf.tensors[name]
    n_rows, row_elems, row_bytes = row_geometry(info)
    if block_rows <= 0:
        raise ValueError("block_rows must be positive")
    if x.shape[-1] != row_elems:
        raise ValueError(f"{name}: x has {x.shape[-1]} features, W rows span {row_elems}")
    row_start = max(0, row_start)
    row_end = n_rows if row_end is None else min(n_rows, row_end)
    window = max(0, row_end - row_start)
    if out is None:
        out = torch.empty((x.shape[0], window), device=device, dtype=dtype)
    if window == 0:
        return out

    src = getattr(provider, "source", provider)
    resident = getattr(provider, "is_resident", lambda _n: False)(name)
    if not resident:
        has_slab = getattr(provider, "has_slab", None)
        resident = bool(has_slab and has_slab(name, row_start, row_end))
    can_async = not resident and hasattr(src, "submit_rows") and hasattr(src, "reader")
    depth = max(1, lookahead)
    if can_async:
        block_rows, depth, can_async = _budget_clamp(src.arena.budget, row_bytes, block_rows, depth)

    fuse = K.can_fuse(info.dtype, x)
    shared = prefetcher if (prefetcher is not None and prefetcher.enabled) else None
    if shared is not None:
        can_async = False
        bounds = shared.bounds(row_start, row_end)
    else:
        bounds = [(lo, min(lo + block_rows, row_end)) for lo in range(row_start, row_end, block_rows)]
    reader = (src._reader_for(name) if hasattr(src, "_reader_for") else src.reader) if can_async else None
    pending: deque = deque()
    queued = 0
    try:
        if can_async:
            for lo, hi in bounds[:depth]:
                pending.append(src.submit_rows(name, lo, hi))
                queued += 1
        for start, end in bounds:
            rows = end - start
            got = shared.take(name, start) if shared is not None else None
            if got is not None:
                raw, nbytes = got
                try:
                    block_out = _block_product(raw, info.dtype, x, rows, row_elems, device, dtype, fuse)
                finally:
                    shared.src.arena.release(nbytes)
            elif can_async:
                fut, nbytes = pending.popleft()
                raw = reader.wait(fut)
                if queued < len(bounds):  # refill before computing: keep `depth` copies in flight
                    nlo, nhi = bounds[queued]
                    pending.append(src.submit_rows(name, nlo, nhi))
                    queued += 1
                try:
                    block_out = _block_product(raw, info.dtype, x, rows, row_elems, device, dtype, fuse)
                finally:
                    src.arena.release(nbytes)
            elif fuse and hasattr(provider, "raw_rows"):
                hit = provider.raw_rows(name, start, end)
                if hit is not None:
                    block_out = K.fused_gemv(hit[0], hit[1], x, rows, row_elems, out_dtype=dtype)
                else:
                    w = provider.fetch_rows(name, start, end, device=device, dtype=dtype)
                    block_out = x.to(dtype) @ w.T
            else:
                w = provider.fetch_rows(name, start, end, device=device, dtype=dtype)
                block_out = x.to(w.dtype) @ w.T
            out[:, start - row_start:end - row_start] = block_out
            if callback is not None:
                callback(name, start, end, block_out)
    finally:
        for fut, nbytes in pending:  # queued but never consumed: do not strand the lease
            fut.cancel()
            src.arena.release(nbytes)
    return out


class BlockPrefetcher:
    """A read-ahead queue over a whole layer's plan of row windows.

    `plan` is [(tensor name, row_lo, row_hi)] in the order the caller will
    consume the windows (e.g. every chosen expert's gate, up and down). The
    windows are cut into blocks of `block_rows` rows, skipping windows the
    provider already holds (resident tensors, admitted slabs), and up to
    `depth` block reads are kept submitted at once across window boundaries,
    so the queue drains once per layer rather than once per projection. Each
    submitted block holds an arena lease until the caller, having taken it
    with `take`, releases it; `block_rows` and `depth` are clamped so that
    depth + 1 blocks fit the arena (the one being computed still holds its
    lease), else the prefetcher disables itself.

    The contract of the reference's BlockPrefetcher
    (compute/blockffn.py:278-393): `enabled`, `block_rows`, `depth`,
    `bounds(lo, hi)`, `take(name, start) -> (raw, nbytes) | None`, `close()`
    and the context manager. A submit that fails (arena full) leaves the block
    first in line for the next top-up; a block the caller asks for before it
    was submitted is dropped from the plan (the caller reads it itself), so
    it is never read late.
    """

    def __init__(self, provider, plan, block_rows: int, depth: int = DEFAULT_LOOKAHEAD) -> None:
        self.provider = provider
        self.src = getattr(provider, "source", provider)
        self.block_rows = max(1, int(block_rows))
        self.depth = max(1, int(depth))
        self.enabled = hasattr(self.src, "submit_rows") and hasattr(self.src, "reader")
        self._blocks: list[tuple[str, int, int]] = []  # every block to read, in consumption order
        self._where: dict[tuple[str, int], int] = {}  # (name, start) -> index in _blocks
        self._cursor = 0  # first block not yet submitted
        self._skipped: set[int] = set()  # blocks the caller went past before they were submitted
        self._live: dict[tuple[str, int], tuple] = {}  # submitted, not yet taken: (future, nbytes)
        if not self.enabled or not plan:
            return
        widest = max(row_geometry(provider.gguf.tensors[name])[2] for name, _, _ in plan)
        self.block_rows, self.depth, self.enabled = _budget_clamp(self.src.arena.budget, widest, self.block_rows,
                                                                  self.depth)
        if not self.enabled:
            return
        br = self.block_rows
        for name, lo, hi in plan:
            if not self._held(name, lo, hi):
                self._blocks += [(name, s, min(s + br, hi)) for s in range(lo, hi, br)]
        self._where = {(name, lo): i for i, (name, lo, _) in enumerate(self._blocks)}
        self._top_up()

    def _held(self, name: str, lo: int, hi: int) -> bool:
        """The provider already holds these rows: no read is ever queued for them."""
        if getattr(self.provider, "is_resident", lambda _n: False)(name):
            return True
        has_slab = getattr(self.provider, "has_slab", None)
        return bool(has_slab is not None and has_slab(name, lo, hi))

    def _top_up(self) -> None:
        while len(self._live) < self.depth and self._cursor < len(self._blocks):
            i = self._cursor
            if i in self._skipped:
                self._cursor += 1
                continue
            name, lo, hi = self._blocks[i]
            try:
                handle = self.src.submit_rows(name, lo, hi)
            except Exception:  # arena full or reader refused: retried at the next top-up
                return
            self._live[(name, lo)] = handle
            self._cursor += 1

    def bounds(self, lo: int, hi: int) -> list[tuple[int, int]]:
        """The blocks of window [lo, hi), cut as the plan cut them."""
        br = self.block_rows
        return [(s, min(s + br, hi)) for s in range(lo, hi, br)]

    def take(self, name: str, start: int):
        """(raw bytes, nbytes) of the block of `name` starting at `start`, once
        its read is done; the caller releases the nbytes lease. None when the
        block was not read ahead (the caller reads it). The queue is topped up
        before returning, so reads stay in flight while the caller computes."""
        key = (name, start)
        handle = self._live.pop(key, None)
        if handle is None:
            i = self._where.get(key)
            if i is not None and i >= self._cursor:
                self._skipped.add(i)
            return None
        fut, nbytes = handle
        reader = self.src._reader_for(name) if hasattr(self.src, "_reader_for") else self.src.reader
        try:
            raw = reader.wait(fut)
        except BaseException:
            self.src.arena.release(nbytes)
            raise
        self._top_up()
        return raw, nbytes

    def close(self) -> None:
        """Cancel the reads still queued and return their leases."""
        live, self._live = self._live, {}
        for fut, nbytes in live.values():
            fut.cancel()
            self.src.arena.release(nbytes)
        self._cursor = len(self._blocks)

    def __enter__(self) -> "BlockPrefetcher":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def stream_expert_ffn(provider, prefix: str, expert: int, x: torch.Tensor, rows_per_expert: int,
                      n_embd: int, activation, block_rows: int = DEFAULT_BLOCK_ROWS, device="cpu",
                      dtype: torch.dtype = torch.float32, bias: bool = False,
                      lookahead: int = DEFAULT_LOOKAHEAD, callback: NeuronCallback | None = None,
                      prefetcher: BlockPrefetcher | None = None) -> torch.Tensor:
    """One routed expert's FFN, a block of neurons at a time."""
    def project(kind, value, lo, span):
        name = prefix + f"ffn_{kind}_exps"
        y = stream_linear(provider, name + ".weight", value, block_rows, device, dtype, callback,
                          row_start=lo, row_end=lo + span, lookahead=lookahead, prefetcher=prefetcher)
        if bias:
            y = y + provider.fetch_rows(name + ".bias", expert, expert + 1, device=device, dtype=dtype)
        return y

    gate = project("gate", x, expert * rows_per_expert, rows_per_expert)
    up = project("up", x, expert * rows_per_expert, rows_per_expert)
    a = activation(gate, up)
    del gate, up
    return project("down", a, expert * n_embd, n_embd)
