"""Where each weight lives: HBM tiers, a host-RAM tier and per-expert slabs.

The provider the streaming seam reads from (the protocol of the reference's
TieredCache, neurostream/residency/cache.py:81-457: `gguf`, `source`,
`is_resident`, `has_slab`, `raw_rows`, `fetch_rows`, `get`,
`raw_quantized`, `admit_vram` / `admit_ram` / `admit_slab`, `submit_rows`,
`pin`, `clear`, and the `CacheStats` counters).

Organisation in this build:
  * two `_Tier`s -- HBM and host RAM -- each a byte-budgeted LRU of
    `_Resident` records. A record of a block-quantized tensor keeps its raw
    GGUF bytes (the VRAM-Q / RAM policy: 4.5 bits a weight instead of 32);
    an F32 / F16 / BF16 tensor is kept in the compute dtype (VRAM-F), since
    for it that costs nothing. RAM records are pinned host memory, so their
    uploads are asynchronous. Names passed to `pin` are never evicted.
  * a `_SlabIndex` of admitted expert row ranges, kept sorted per tensor so
    the slab covering any sub-range of it is found by bisection (neuron-block
    streaming asks for sub-ranges of an admitted expert window).
  * MI355X: a slab of an MXFP4 tensor on the GPU is re-laid into 64-row
    tiles (`slab_layout="t64"`, one HIP pack kernel at admission) so that the
    expert kernels load one 128-bit vector per lane per block; `raw_rows`
    then hands out `T64Rows` windows, which `fused_gemv` and `dequantize_rows`
    accept, and `T64Rows.to_gguf` recovers the GGUF bytes exactly.
"""
from __future__ import annotations

import bisect
from collections import OrderedDict
from dataclasses import dataclass

import torch

from ..compute.kernels import T64Rows, t64_pack
from ..compute.quant import dequantize
from ..format.gguf import FLOAT_TYPES, GGMLType, row_geometry


@dataclass
class CacheStats:
    """Access counters (the reference's CacheStats fields)."""
    vram_hits: int = 0      # accesses served from HBM (whole tensors or slabs)
    ram_hits: int = 0       # accesses served from the host-RAM tier
    misses: int = 0         # accesses that went to the source
    vram_bytes: int = 0     # bytes held by the HBM tier (slabs excluded)
    ram_bytes: int = 0      # bytes held by the RAM tier
    evictions: int = 0
    dequant_calls: int = 0
    slab_hits: int = 0
    slab_misses: int = 0    # row requests on a cache with slabs that no slab covered

    @staticmethod
    def _ratio(num: int, den: int) -> float:
        return num / den if den else 0.0

    @property
    def slab_rate(self) -> float:
        return self._ratio(self.slab_hits, self.slab_hits + self.slab_misses)

    @property
    def hit_rate(self) -> float:
        return self._ratio(self.vram_hits + self.ram_hits, self.vram_hits + self.ram_hits + self.misses)

    def summary(self) -> str:
        return (f"cache: HBM {self.vram_bytes / 2**30:.2f} GiB ({self.vram_hits} hits), "
                f"RAM {self.ram_bytes / 2**30:.2f} GiB ({self.ram_hits} hits), {self.misses} misses, "
                f"{self.evictions} evictions, hit rate {100 * self.hit_rate:.1f}%, "
                f"slabs {self.slab_hits}/{self.slab_hits + self.slab_misses}")


@dataclass
class _Resident:
    data: torch.Tensor         # float tensor (expanded) or raw bytes / t64 tiles
    nbytes: int                # bytes charged to the tier or the slab budget
    expanded: bool             # True: `data` is already in the compute dtype
    ggml_type: GGMLType | None = None
    n_elements: int = 0
    shape: tuple = ()
    layout: str = "gguf"       # slabs: "gguf" bytes or "t64" tiles
    rows: int = 0              # slabs: rows held


class _Tier:
    """A byte-budgeted LRU of residents; `protected` names are never evicted.

    Residents laid out in one shared buffer (TieredCache.fuse_vram) form a
    group that leaves together: evicting or replacing any member evicts
    every member, so the bytes the tier counts are the bytes still alive,
    and `on_group_gone(group)` lets the owner drop the shared buffer."""

    def __init__(self, budget: int, on_group_gone=None) -> None:
        self.budget = int(budget)
        self.held = 0
        self.items: OrderedDict[str, _Resident] = OrderedDict()
        self.groups: dict[str, tuple] = {}  # member name -> its group (a tuple of names)
        self.on_group_gone = on_group_gone

    def lookup(self, name: str) -> _Resident | None:
        r = self.items.get(name)
        if r is not None:
            self.items.move_to_end(name)  # most recently used last
        return r

    def group(self, names: tuple) -> None:
        for n in names:
            self.groups[n] = names

    def _drop(self, name: str) -> int:
        """Remove `name` and, when it is grouped, the rest of its group: how many residents left."""
        group = self.groups.get(name)
        gone = 0
        for m in (group or (name,)):
            self.groups.pop(m, None)
            r = self.items.pop(m, None)
            if r is not None:
                self.held -= r.nbytes
                gone += 1
        if group is not None and self.on_group_gone is not None:
            self.on_group_gone(group)
        return gone

    def make_room(self, need: int, protected: set) -> int:
        """Evict least recently used residents (a group whole) until `need`
        more bytes fit; returns how many were evicted (it may still not fit if
        the rest is protected)."""
        evicted = 0
        for name in [n for n in self.items if n not in protected]:
            if self.held + need <= self.budget:
                break
            if name not in self.items or any(m in protected for m in self.groups.get(name, ())):
                continue
            evicted += self._drop(name)
        return evicted

    def put(self, name: str, r: _Resident) -> None:
        if name in self.items:  # a replaced member takes its group (and shared buffer) with it
            self._drop(name)
        self.items[name] = r
        self.held += r.nbytes


class _SlabIndex:
    """Admitted row ranges per tensor, sorted by start row."""

    def __init__(self) -> None:
        self.by_name: dict[str, list[tuple[int, int, _Resident]]] = {}
        self.nbytes = 0

    def add(self, name: str, lo: int, hi: int, r: _Resident) -> None:
        spans = self.by_name.setdefault(name, [])
        bisect.insort(spans, (lo, hi, r), key=lambda s: (s[0], s[1]))
        self.nbytes += r.nbytes

    def exact(self, name: str, lo: int, hi: int) -> _Resident | None:
        for a, b, r in self.by_name.get(name, ()):
            if (a, b) == (lo, hi):
                return r
        return None

    def covering(self, name: str, lo: int, hi: int):
        """(resident, its first row) of a slab holding all of rows [lo, hi), or None."""
        spans = self.by_name.get(name)
        if not spans:
            return None
        i = bisect.bisect_right(spans, lo, key=lambda s: s[0])  # spans starting at or before lo
        for a, b, r in reversed(spans[:i]):
            if hi <= b:
                return r, a
        return None

    def __bool__(self) -> bool:
        return bool(self.by_name)


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
        if slab_layout is None:
            slab_layout = "t64" if self.device.type == "cuda" else "gguf"
        if slab_layout not in ("t64", "gguf"):
            raise ValueError(f"slab_layout must be 't64' or 'gguf', not {slab_layout!r}")
        self.slab_layout = slab_layout
        self.slab_budget = 0  # bytes of expert slabs admit_slab may hold (set by the loader)
        self._fused: dict[tuple, torch.Tensor] = {}
        self._hbm = _Tier(vram_budget, on_group_gone=self._unfuse)
        self._ram = _Tier(ram_budget)
        self._slabs = _SlabIndex()
        self._protected: set[str] = set()
        self.stats = CacheStats()

    # budgets and holdings (the reference's attribute names)
    @property
    def vram_budget(self) -> int:
        return self._hbm.budget

    @vram_budget.setter
    def vram_budget(self, v: int) -> None:
        self._hbm.budget = int(v)

    @property
    def ram_budget(self) -> int:
        return self._ram.budget

    @ram_budget.setter
    def ram_budget(self, v: int) -> None:
        self._ram.budget = int(v)

    @property
    def slab_bytes(self) -> int:
        return self._slabs.nbytes

    # -- placement -------------------------------------------------------------

    def vram_cost(self, name: str) -> int:
        """HBM bytes `name` takes once admitted: float tensors in the compute
        dtype, block-quantized ones as their raw bytes."""
        info = self.gguf.tensors[name]
        if info.dtype in FLOAT_TYPES:
            return info.n_elements * self.compute_dtype.itemsize
        return info.nbytes

    def pin(self, names) -> None:
        """Never evict these tensors from either tier."""
        self._protected.update(names)

    def _admit(self, tier: _Tier, name: str, need: int, make) -> bool:
        if name in tier.items:
            return True
        if need > tier.budget:
            return False
        self.stats.evictions += tier.make_room(need, self._protected)
        if tier.held + need > tier.budget:
            return False
        tier.put(name, make())
        self._sync_bytes()
        return True

    def _sync_bytes(self) -> None:
        self.stats.vram_bytes, self.stats.ram_bytes = self._hbm.held, self._ram.held

    def admit_vram(self, name: str) -> bool:
        """Hold `name` whole in HBM (VRAM-F for float tensors, VRAM-Q for the rest)."""
        info = self.gguf.tensors[name]
        need = self.vram_cost(name)

        def make():
            raw = self.source.raw_bytes(name).to(self.device)
            if info.dtype in FLOAT_TYPES:
                t = dequantize(raw, info.dtype, info.n_elements, out_dtype=self.compute_dtype)
                return _Resident(t.reshape(info.torch_shape), need, True)
            return _Resident(raw, need, False, info.dtype, info.n_elements, info.torch_shape)
        return self._admit(self._hbm, name, need, make)

    def admit_ram(self, name: str) -> bool:
        """Hold `name`'s raw bytes in host RAM (pinned when the compute device is a GPU)."""
        info = self.gguf.tensors[name]

        def make():
            raw = self.source.raw_bytes(name)
            raw = raw.cpu() if raw.is_cuda else raw
            if self.device.type == "cuda" and not raw.is_pinned():
                raw = raw.pin_memory()
            return _Resident(raw, info.nbytes, False, info.dtype, info.n_elements, info.torch_shape)
        return self._admit(self._ram, name, info.nbytes, make)

    def admit_slab(self, name: str, start: int, end: int, layout: str | None = None) -> bool:
        """Keep rows [start, end) of a block-quantized tensor in HBM, still
        quantized (one expert's window of a stacked tensor), within slab_budget."""
        info = self.gguf.tensors[name]
        if info.dtype in FLOAT_TYPES or self.is_resident(name):
            return False
        if self._slabs.exact(name, start, end) is not None:
            return True
        _, row_elems, row_bytes = row_geometry(info)
        need = (end - start) * row_bytes
        if self._slabs.nbytes + need > self.slab_budget:
            return False
        layout = layout or self.slab_layout
        if info.dtype != GGMLType.MXFP4 or self.device.type != "cuda":
            layout = "gguf"  # the tile layout exists for MXFP4 on the GPU only
        raw = self.source.raw_rows(name, start, end).to(self.device)
        data = t64_pack(raw, info.dtype, end - start, row_elems) if layout == "t64" else raw
        self._slabs.add(name, start, end, _Resident(data, need, False, info.dtype, layout=layout, rows=end - start))
        return True

    # -- lookups ---------------------------------------------------------------

    def is_resident(self, name: str) -> bool:
        return name in self._hbm.items or name in self._ram.items

    def has_slab(self, name: str, start: int, end: int) -> bool:
        return self._slabs.covering(name, start, end) is not None

    def slab_entry(self, name: str, start: int, end: int):
        """(data tensor, layout) of the slab admitted as exactly [start, end), or None."""
        r = self._slabs.exact(name, start, end)
        return None if r is None else (r.data, r.layout)

    def vram_raw(self, name: str):
        """(raw bytes, GGMLType) of a block-quantized tensor held whole in the
        HBM tier, or None -- never a copy from another tier."""
        r = self._hbm.lookup(name)
        if r is None or r.expanded:
            return None
        self.stats.vram_hits += 1
        return r.data, r.ggml_type

    def fuse_vram(self, names):
        """Lay block-quantized tensors held whole in the HBM tier out back to
        back in one buffer, so one GEMV can run over all their rows (the q, k
        and v projections of an attention layer): returns (buffer, GGMLType),
        or None unless every name is such a tensor and they share one type.
        Each resident then becomes a view into the buffer and the separate
        copies are freed, so the tier holds the same bytes as before."""
        names = tuple(names)
        rs = [self._hbm.items.get(n) for n in names]
        if any(r is None or r.expanded for r in rs) or len({r.ggml_type for r in rs}) != 1:
            return None
        buf = self._fused.get(names)
        if buf is not None and all(r.data.untyped_storage().data_ptr() == buf.untyped_storage().data_ptr()
                                   for r in rs):
            return buf, rs[0].ggml_type
        buf = torch.cat([r.data.reshape(-1) for r in rs])
        off = 0
        for r in rs:
            n = r.data.numel()
            r.data = buf[off:off + n]
            off += n
        self._fused[names] = buf
        self._hbm.group(names)  # the members share `buf`: they leave the tier together
        return buf, rs[0].ggml_type

    def _unfuse(self, names: tuple) -> None:
        self._fused.pop(names, None)

    def _tiered(self, name: str):
        """(resident, "vram" | "ram") with the hit counted, or (None, None)."""
        r = self._hbm.lookup(name)
        if r is not None:
            self.stats.vram_hits += 1
            return r, "vram"
        r = self._ram.lookup(name)
        if r is not None:
            self.stats.ram_hits += 1
            return r, "ram"
        return None, None

    def _expand(self, r: _Resident) -> torch.Tensor:
        if r.expanded:
            return r.data
        self.stats.dequant_calls += 1
        raw = r.data.to(self.device, non_blocking=True)
        return dequantize(raw, r.ggml_type, r.n_elements, out_dtype=self.compute_dtype).reshape(r.shape)

    def get(self, name: str) -> torch.Tensor:
        """The whole tensor in the compute dtype on the compute device."""
        r, _ = self._tiered(name)
        if r is not None:
            return self._expand(r)
        self.stats.misses += 1
        return self.source.fetch(name, device=self.device, dtype=self.compute_dtype)

    @staticmethod
    def _slab_window(r: _Resident, first: int, start: int, end: int, row_bytes: int, K: int):
        if r.layout == "t64":
            return T64Rows(r.data, r.ggml_type, r.rows, K, start - first, end - first)
        return r.data[(start - first) * row_bytes:(end - first) * row_bytes]

    def raw_rows(self, name: str, start: int, end: int):
        """(raw bytes or a T64Rows window on the device, GGMLType) of rows
        [start, end), from a slab, a tier or the source; None for float tensors."""
        info = self.gguf.tensors[name]
        if info.dtype in FLOAT_TYPES:
            return None
        _, row_elems, row_bytes = row_geometry(info)
        hit = self._slabs.covering(name, start, end)
        if hit is not None:
            r, first = hit
            self.stats.vram_hits += 1
            self.stats.slab_hits += 1
            return self._slab_window(r, first, start, end, row_bytes, row_elems), r.ggml_type
        if self._slabs:
            self.stats.slab_misses += 1
        r, tier = self._tiered(name)
        if r is not None and not r.expanded:
            part = r.data[start * row_bytes:end * row_bytes]
            return (part if tier == "vram" else part.to(self.device, non_blocking=True)), r.ggml_type
        if r is None:
            self.stats.misses += 1
        return self.source.raw_rows(name, start, end).to(self.device, non_blocking=True), info.dtype

    def fetch_rows(self, name, start, end, device=None, dtype=None) -> torch.Tensor:
        """Rows [start, end) dequantized to `dtype` on `device` (the window is
        clipped to the tensor)."""
        device = self.device if device is None else torch.device(device)
        dtype = self.compute_dtype if dtype is None else dtype
        info = self.gguf.tensors[name]
        n_rows, row_elems, row_bytes = row_geometry(info)
        hit = self._slabs.covering(name, start, end)
        if hit is not None:
            r, first = hit
            self.stats.vram_hits += 1
            self.stats.slab_hits += 1
            self.stats.dequant_calls += 1
            window = self._slab_window(r, first, start, end, row_bytes, row_elems)
            return dequantize_rows(window, r.ggml_type, end - start, row_elems, dtype).to(device)
        r, _ = self._tiered(name)
        if r is None:
            self.stats.misses += 1
            return self.source.fetch_rows(name, start, end, device=device, dtype=dtype)
        start, end = max(0, start), min(n_rows, end)
        if start >= end:
            return torch.empty((0, row_elems), dtype=dtype, device=device)
        if r.expanded:
            return r.data.reshape(-1, row_elems)[start:end].to(device, dtype)
        raw = r.data[start * row_bytes:end * row_bytes].to(device, non_blocking=True)
        self.stats.dequant_calls += 1
        return dequantize_rows(raw, r.ggml_type, end - start, row_elems, dtype)

    def raw_quantized(self, name: str):
        """(raw bytes on the compute device, GGMLType) of a block-quantized
        tensor held in a tier -- RAM-tier bytes are uploaded for the call --
        or None."""
        r, tier = self._tiered(name)
        if r is None or r.expanded:
            return None
        return (r.data if tier == "vram" else r.data.to(self.device, non_blocking=True)), r.ggml_type

    def submit_rows(self, name: str, start: int, end: int):
        """Queue a block read at the source, unless the tensor is held in a tier."""
        if self.is_resident(name):
            return None
        return self.source.submit_rows(name, start, end)

    def clear(self) -> None:
        """Drop every resident and slab and reset the counters (budgets stay)."""
        self._hbm = _Tier(self._hbm.budget, on_group_gone=self._unfuse)
        self._ram = _Tier(self._ram.budget)
        self._slabs = _SlabIndex()
        self._fused = {}
        self.stats = CacheStats()
        if self.device.type == "cuda":
            torch.cuda.empty_cache()
