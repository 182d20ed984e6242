"""Tiered weight residency: VRAM-Q / VRAM-F / RAM, plus per-expert slabs.

Contract of the reference's TieredCache (neurostream/residency/cache.py:81-457):
  * VRAM-Q: raw quantized bytes on the GPU, expanded per access (default);
    VRAM-F: float tensors (F32/F16/BF16) cached in the compute dtype;
    RAM: raw bytes in host memory (pinned here, so uploads are asynchronous).
  * LRU eviction inside each tier, pins exempt (`pin`, `_evict`).
  * Expert slabs: `admit_slab(name, lo, hi)` keeps one expert's row range on
    the GPU under `slab_budget`; `_slab_for` resolves any sub-range of an
    admitted slab, so neuron-block streaming hits it (cache.py:260-276).
  * `raw_rows` / `fetch_rows` / `raw_quantized` / `has_slab` / `is_resident`
    and the CacheStats counters.
MI355X-specific: with `slab_layout="t64"` (the default on a GPU for MXFP4),
an admitted slab is re-laid into 64-row tiles by one HIP kernel, so decode
GEMVs load one 128-bit vector per lane per block. `raw_rows` then returns a
`T64Rows` window that `fused_gemv` and `dequantize_rows` accept; the GGUF
bytes are recoverable exactly (`T64Rows.to_gguf`).
"""
from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass

import torch

from ..compute.kernels import T64Rows, t64_pack
from ..compute.quant import dequantize
from ..format.gguf import FLOAT_TYPES, GGMLType, row_geometry


@dataclass
class CacheStats:
    vram_hits: int = 0
    ram_hits: int = 0
    misses: int = 0
    vram_bytes: int = 0
    ram_bytes: int = 0
    evictions: int = 0
    dequant_calls: int = 0
    slab_hits: int = 0
    slab_misses: int = 0

    @property
    def slab_rate(self) -> float:
        t = self.slab_hits + self.slab_misses
        return 0.0 if t == 0 else self.slab_hits / t

    @property
    def hit_rate(self) -> float:
        t = self.vram_hits + self.ram_hits + self.misses
        return 0.0 if t == 0 else (self.vram_hits + self.ram_hits) / t

    def summary(self) -> str:
        return (f"vram {self.vram_bytes / 1e9:.2f}GB/{self.vram_hits} hits | "
                f"ram {self.ram_bytes / 1e9:.2f}GB/{self.ram_hits} hits | "
                f"miss {self.misses} | evict {self.evictions} | hit-rate {self.hit_rate:.1%}")


@dataclass
class _Entry:
    payload: torch.Tensor
    nbytes: int
    ready: bool  # True: float tensor in compute dtype; False: raw quantized bytes
    dtype: GGMLType | None = None
    n_elements: int = 0
    shape: tuple = ()
    layout: str = "gguf"  # "gguf" raw bytes or "t64" tiles (slabs only)
    rows: int = 0


def dequantize_rows(raw, dtype, rows: int, row_elems: int, out_dtype=torch.float32) -> torch.Tensor:
    """(rows, row_elems) floats from raw GGUF bytes or a T64Rows window."""
    if isinstance(raw, T64Rows):
        raw = raw.to_gguf()
    return dequantize(raw, dtype, rows * row_elems, out_dtype=out_dtype).reshape(rows, row_elems)


class TieredCache:
    def __init__(self, source, device="cpu", compute_dtype=torch.float32, vram_budget: int = 0,
                 ram_budget: int = 0, slab_layout: str | None = None) -> None:
        self.source = source
        self.gguf = source.gguf
        self.device = torch.device(device)
        self.compute_dtype = compute_dtype
        self.vram_budget = vram_budget
        self.ram_budget = ram_budget
        self.slab_budget = 0
        self.slab_bytes = 0
        if slab_layout is None:
            slab_layout = "t64" if self.device.type == "cuda" else "gguf"
        if slab_layout not in ("t64", "gguf"):
            raise ValueError(f"slab_layout must be 't64' or 'gguf', not {slab_layout!r}")
        self.slab_layout = slab_layout
        self._slab: OrderedDict[str, _Entry] = OrderedDict()
        self._slab_spans: dict[str, list[tuple[int, int]]] = {}
        self._vram: OrderedDict[str, _Entry] = OrderedDict()
        self._ram: OrderedDict[str, _Entry] = OrderedDict()
        self._pinned: set[str] = set()
        self.stats = CacheStats()

    # -- sizing / placement ------------------------------------------------

    def vram_cost(self, name: str) -> int:
        info = self.gguf.tensors[name]
        if info.dtype in FLOAT_TYPES:
            return info.n_elements * self.compute_dtype.itemsize
        return info.nbytes

    def pin(self, names) -> None:
        self._pinned.update(names)

    def _evict(self, store, need: int, budget: int, is_vram: bool) -> None:
        used = self.stats.vram_bytes if is_vram else self.stats.ram_bytes
        while used + need > budget and store:
            victim = next((n for n in store if n not in self._pinned), None)
            if victim is None:
                return  # everything left is pinned
            e = store.pop(victim)
            if is_vram:
                self.stats.vram_bytes -= e.nbytes
            else:
                self.stats.ram_bytes -= e.nbytes
            self.stats.evictions += 1
            used -= e.nbytes

    def admit_vram(self, name: str) -> bool:
        if name in self._vram:
            return True
        info = self.gguf.tensors[name]
        need = self.vram_cost(name)
        if need > self.vram_budget:
            return False
        self._evict(self._vram, need, self.vram_budget, True)
        if self.stats.vram_bytes + need > self.vram_budget:
            return False
        raw = self.source.raw_bytes(name)
        if info.dtype in FLOAT_TYPES:
            t = dequantize(raw.to(self.device), info.dtype, info.n_elements,
                           out_dtype=self.compute_dtype).reshape(info.torch_shape)
            entry = _Entry(t, need, True)
        else:
            entry = _Entry(raw.to(self.device), need, False, info.dtype, info.n_elements, info.torch_shape)
        self._vram[name] = entry
        self.stats.vram_bytes += need
        return True

    def admit_ram(self, name: str) -> bool:
        if name in self._ram:
            return True
        info = self.gguf.tensors[name]
        need = info.nbytes
        if need > self.ram_budget:
            return False
        self._evict(self._ram, need, self.ram_budget, False)
        if self.stats.ram_bytes + need > self.ram_budget:
            return False
        raw = self.source.raw_bytes(name)
        if raw.is_cuda:
            raw = raw.cpu()
        if self.device.type == "cuda" and not raw.is_pinned():
            raw = raw.pin_memory()
        self._ram[name] = _Entry(raw, need, False, info.dtype, info.n_elements, info.torch_shape)
        self.stats.ram_bytes += need
        return True

    # -- access --------------------------------------------------------------

    def is_resident(self, name: str) -> bool:
        return name in self._vram or name in self._ram

    def _expand(self, e: _Entry) -> torch.Tensor:
        if e.ready:
            return e.payload
        self.stats.dequant_calls += 1
        raw = e.payload.to(self.device, non_blocking=True)
        return dequantize(raw, e.dtype, e.n_elements, out_dtype=self.compute_dtype).reshape(e.shape)

    def get(self, name: str) -> torch.Tensor:
        for store, attr in ((self._vram, "vram_hits"), (self._ram, "ram_hits")):
            e = store.get(name)
            if e is not None:
                store.move_to_end(name)
                setattr(self.stats, attr, getattr(self.stats, attr) + 1)
                return self._expand(e)
        self.stats.misses += 1
        return self.source.fetch(name, device=self.device, dtype=self.compute_dtype)

    def _slab_for(self, name: str, start: int, end: int):
        """(entry, slab_start) of an admitted slab covering rows [start, end)."""
        for lo, hi in self._slab_spans.get(name, ()):
            if lo <= start and end <= hi:
                key = f"{name}#{lo}:{hi}"
                e = self._slab.get(key)
                if e is not None:
                    self._slab.move_to_end(key)
                    return e, lo
        return None

    def _slab_view(self, e: _Entry, base: int, start: int, end: int, row_bytes: int, K: int):
        if e.layout == "t64":
            return T64Rows(e.payload, e.dtype, e.rows, K, start - base, end - base)
        return e.payload[(start - base) * row_bytes:(end - base) * row_bytes]

    def fetch_rows(self, name, start, end, device=None, dtype=None) -> torch.Tensor:
        device = self.device if device is None else device
        dtype = self.compute_dtype if dtype is None else dtype
        info = self.gguf.tensors[name]
        n_rows, row_elems, row_bytes = row_geometry(info)
        found = self._slab_for(name, start, end)
        if found is not None:
            slab, base = found
            self.stats.vram_hits += 1
            self.stats.slab_hits += 1
            self.stats.dequant_calls += 1
            raw = self._slab_view(slab, base, start, end, row_bytes, row_elems)
            return dequantize_rows(raw, slab.dtype, end - start, row_elems, dtype).to(device)
        e = self._vram.get(name) or self._ram.get(name)
        if e is None:
            self.stats.misses += 1
            return self.source.fetch_rows(name, start, end, device=device, dtype=dtype)
        if name in self._vram:
            self._vram.move_to_end(name)
            self.stats.vram_hits += 1
        else:
            self._ram.move_to_end(name)
            self.stats.ram_hits += 1
        start, end = max(0, start), min(n_rows, end)
        if start >= end:
            return torch.empty((0, row_elems), dtype=dtype, device=device)
        if e.ready:
            return e.payload.reshape(-1, row_elems)[start:end].to(device, dtype)
        raw = e.payload[start * row_bytes:end * row_bytes]
        if raw.device != torch.device(device):
            raw = raw.to(device, non_blocking=True)
        self.stats.dequant_calls += 1
        return dequantize_rows(raw, e.dtype, end - start, row_elems, dtype)

    def raw_quantized(self, name: str):
        e = self._vram.get(name)
        if e is not None:
            if e.ready:
                return None
            self._vram.move_to_end(name)
            self.stats.vram_hits += 1
            return e.payload, e.dtype
        e = self._ram.get(name)
        if e is None or e.ready:
            return None
        self._ram.move_to_end(name)
        self.stats.ram_hits += 1
        return e.payload.to(self.device, non_blocking=True), e.dtype

    def admit_slab(self, name: str, start: int, end: int, layout: str | None = None) -> bool:
        """Keep rows [start, end) of `name` on the GPU, still quantized."""
        info = self.gguf.tensors[name]
        if info.dtype in FLOAT_TYPES or self.is_resident(name):
            return False
        key = f"{name}#{start}:{end}"
        if key in self._slab:
            return True
        n_rows, row_elems, row_bytes = row_geometry(info)
        need = (end - start) * row_bytes
        if self.slab_bytes + need > self.slab_budget:
            return False
        layout = layout or self.slab_layout
        if layout == "t64" and (info.dtype != GGMLType.MXFP4 or self.device.type != "cuda"):
            layout = "gguf"
        raw = self.source.raw_rows(name, start, end).to(self.device)
        payload = t64_pack(raw, info.dtype, end - start, row_elems) if layout == "t64" else raw
        self._slab[key] = _Entry(payload, need, False, info.dtype, layout=layout, rows=end - start)
        self._slab_spans.setdefault(name, []).append((start, end))
        self.slab_bytes += need
        return True

    def has_slab(self, name: str, start: int, end: int) -> bool:
        return self._slab_for(name, start, end) is not None

    def slab_entry(self, name: str, start: int, end: int):
        """(payload tensor, layout) of the slab admitted exactly as [start, end), or None."""
        e = self._slab.get(f"{name}#{start}:{end}")
        return None if e is None else (e.payload, e.layout)

    def raw_rows(self, name: str, start: int, end: int):
        """(raw bytes or T64Rows on the device, GGMLType) for a row range, or None."""
        info = self.gguf.tensors[name]
        if info.dtype in FLOAT_TYPES:
            return None
        _, row_elems, row_bytes = row_geometry(info)
        found = self._slab_for(name, start, end)
        if found is not None:
            slab, base = found
            self.stats.vram_hits += 1
            self.stats.slab_hits += 1
            return self._slab_view(slab, base, start, end, row_bytes, row_elems), slab.dtype
        if self._slab:
            self.stats.slab_misses += 1
        lo, hi = start * row_bytes, end * row_bytes
        e = self._vram.get(name)
        if e is not None and not e.ready:
            self._vram.move_to_end(name)
            self.stats.vram_hits += 1
            return e.payload[lo:hi], e.dtype
        e = self._ram.get(name)
        if e is not None and not e.ready:
            self._ram.move_to_end(name)
            self.stats.ram_hits += 1
            return e.payload[lo:hi].to(self.device, non_blocking=True), e.dtype
        self.stats.misses += 1
        raw = self.source.raw_rows(name, start, end)
        return raw.to(self.device, non_blocking=True), info.dtype

    def submit_rows(self, name: str, start: int, end: int):
        if self.is_resident(name):
            return None
        return self.source.submit_rows(name, start, end)

    def clear(self) -> None:
        self._slab.clear()
        self._slab_spans.clear()
        self._vram.clear()
        self._ram.clear()
        self.slab_bytes = 0
        self.stats = CacheStats()
        if self.device.type == "cuda":
            torch.cuda.empty_cache()
