"""GPT-OSS MoE FFN stack on one MI355X (model/gpt_oss.py:61-177 of the reference).

`GptOssFFNStack` holds one MoELayer per layer (VRAM-resident expert slabs)
and chains them the way the reference's decoder wraps its FFN blocks:
h = rms_norm(x, post_attention_norm) (compute/ops.py:14-20), out = moe(h),
x = x + out (gpt_oss.py:126,177). Attention is not on the MoE path and is
not modelled: layer l + 1 reads layer l's output directly.

`forward` runs the whole chain on the device with no host synchronisation:
per layer one MoE layer call (device-side routing), the residual add and
the next layer's norm folded into the next router kernel (up to two tokens,
nsx_moe_forward_norm) or into the layer's own last launch (nsx_moe_forward_addnorm),
the same bits as a separate nsx_add_rmsnorm. `_route` and
`_ffn_block` keep the reference's per-layer signatures; `_route` returns the
chosen experts as a host list (a device-to-host copy, as the reference's
torch.unique(...).tolist() at gpt_oss.py:121).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from ..compute.ops import add_rms_norm
from ..moe.fused import MoELayer
from ..moe.router import RouterStats


def clamped_swiglu(gate: torch.Tensor, up: torch.Tensor, alpha: float = 1.702, limit: float = 7.0) -> torch.Tensor:
    """model/gpt_oss.py:61-70 on torch tensors (the activation callable of
    stream_expert_ffn): (clamp(up, -l, l) + 1) * g * sigmoid(alpha * g), g = min(gate, l)."""
    g = torch.clamp(gate, max=limit)
    u = torch.clamp(up, -limit, limit)
    return (u + 1) * (g * torch.sigmoid(alpha * g))


@dataclass
class StackConfig:
    n_layer: int
    n_embd: int
    n_expert: int
    n_expert_used: int
    n_ffn_expert: int
    rms_eps: float = 1e-5


class GptOssFFNStack:
    """The routed-expert FFN blocks of a GPT-OSS decoder, all resident."""

    def __init__(self, layers: list[MoELayer], norm_weights: list[torch.Tensor | None] | None = None,
                 eps: float = 1e-5) -> None:
        if not layers:
            raise ValueError("an FFN stack needs at least one layer")
        l0 = layers[0]
        self.layers = layers
        self.cfg = StackConfig(len(layers), l0.n_embd, l0.n_expert, l0.top_k, l0.n_ff, eps)
        self.device = l0.device
        self.norm_weights = norm_weights or [None] * len(layers)
        if len(self.norm_weights) != len(layers):
            raise ValueError("one post-attention norm weight (or None) per layer")
        self.router_stats = RouterStats()
        self._bufs: dict[int, tuple] = {}
        self._alt: dict[int, torch.Tensor] = {}  # the residual stream's second buffer, per T
        # one token runs as a decode chain (no router launch after the first layer) where every layer can
        self.decode_chain = True
        self._chain: bool | None = None
        self._share: torch.Tensor | None = None

    def _buffers(self, T: int):
        b = self._bufs.get(T)
        if b is None:
            n, L, k = self.cfg.n_embd, self.cfg.n_layer, self.cfg.n_expert_used
            b = (torch.empty(T, n, device=self.device), torch.empty(T, n, device=self.device),
                 torch.empty(L, T, k, dtype=torch.int32, device=self.device),
                 torch.empty(L, T, k, dtype=torch.float32, device=self.device))
            self._bufs[T] = b
            for layer in self.layers:
                layer.workspace(T)
        return b

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """x: (T, n_embd) fp32 residual stream in; returns it after every
        layer's FFN block (into `out` when given). Device-only: no host sync.
        Between layers x += out and h = rms_norm(x) of the next layer run inside
        that layer's router kernel where the layer allows it
        (MoELayer.forward_norm, the residual stream then alternating between two
        buffers), else inside this layer's last launch (MoELayer.forward_addnorm,
        in place); both the same bits as add_rms_norm."""
        x = x.reshape(-1, self.cfg.n_embd)
        T = x.shape[0]
        h, y, ids, wts = self._buffers(T)
        if T == 1 and self.decode_chain and self._chain_ok():
            return self._forward_chain(x, out, y, ids, wts)
        alt = self._alt.get(T)
        if alt is None:
            alt = self._alt[T] = torch.empty(T, self.cfg.n_embd, device=self.device)
        res = torch.empty_like(x) if out is None else out
        eps = self.cfg.rms_eps
        add_rms_norm(x.float().contiguous(), None, self.norm_weights[0], eps, out=h, sum_out=res)
        cur, other = res, alt
        n = len(self.layers)
        pending = False  # y holds the last layer's output, not yet added to cur
        for li, layer in enumerate(self.layers):  # x += out; h = rms_norm(x); out = layer(h)
            if pending:  # this layer's add + norm inside its router kernel
                layer.forward_norm(cur, y, self.norm_weights[li], eps, x_out=other, out=y, ids=ids[li],
                                   weights=wts[li])
                cur, other = other, cur
            elif li + 1 < n and not self.layers[li + 1].norm_folds(T):
                # the next layer's add + norm in this layer's last launch (h is its input, then the next one's)
                layer.forward_addnorm(h, cur, self.norm_weights[li + 1], eps, x_out=cur, h_out=h, ids=ids[li],
                                      weights=wts[li])
                continue
            else:
                layer.forward(h, out=y, ids=ids[li], weights=wts[li])
            pending = True
        if cur is res:
            res.add_(y)
        else:
            torch.add(cur, y, out=res)
        return res

    __call__ = forward

    def _chain_ok(self) -> bool:
        if self._chain is None:
            sizes = [layer.chain_share_bytes() for layer in self.layers]
            self._chain = min(sizes) >= 0
            if self._chain:
                self._share = torch.empty(max(sizes), dtype=torch.uint8, device=self.device)
        return self._chain

    def _forward_chain(self, x, out, y, ids, wts) -> torch.Tensor:
        """One token through every layer as a decode chain (MoELayer.chain_t1):
        the residual stream updated in place in `out`, and after the first layer
        no router launch -- each down kernel leaves the next layer's router
        shares in one buffer, which that layer's gate/up kernel reads (matches
        the separate norm to rounding: the rms is summed in another order)."""
        res = torch.empty_like(x) if out is None else out
        res.copy_(x)
        eps, n = self.cfg.rms_eps, len(self.layers)
        for li, layer in enumerate(self.layers):
            nxt = self.layers[li + 1] if li + 1 < n else None
            layer.chain_t1(res, self.norm_weights[li], eps, self._share if li else None, nxt,
                           None if nxt is None else self.norm_weights[li + 1], None if nxt is None else self._share,
                           y, ids[li], wts[li])
        return res

    def last_routing(self, T: int) -> tuple[torch.Tensor, torch.Tensor]:
        """(ids (L, T, k), weights (L, T, k)) of the last forward over T tokens."""
        _, _, ids, wts = self._buffers(T)
        return ids, wts

    # -- the reference's per-layer seams (gpt_oss.py:116-177) -------------------

    def _route(self, h: torch.Tensor, layer: int):
        """(chosen experts ascending (host list), ids (T, k), weights (T, k)), gpt_oss.py:116-121."""
        from ..moe.fused import router_topk
        lay = self.layers[layer]
        ids, wts, _ = router_topk(h, lay.router_w, lay.router_b, lay.top_k, "gptoss")
        return torch.unique(ids).tolist(), ids, wts

    def _ffn_block(self, x: torch.Tensor, layer: int) -> torch.Tensor:
        """x + moe(rms_norm(x)) for one layer, gpt_oss.py:123-177 (device
        routing; the router statistics are taken from the layer's ids)."""
        x = x.reshape(-1, self.cfg.n_embd).float().contiguous()
        h = add_rms_norm(x, None, self.norm_weights[layer], self.cfg.rms_eps)
        out, ids, _ = self.layers[layer].forward(h)
        self.router_stats.record(layer, ids)
        return x + out

    @classmethod
    def synthetic(cls, cfg, n_layers: int, seed: int, device, layout: str = "t64", dispatch: str = "auto"):
        """n_layers independently seeded layers of `cfg`
        (router seed = f(seed, layer)), expert slabs resident in HBM."""
        from .. import synth
        from ..compute.kernels import t64_pack_stacked
        layers = []
        for li in range(n_layers):
            t = synth.make_layer(cfg, seed=seed, device=device, layer=li)
            if layout == "t64":
                mats = {k: t64_pack_stacked(t[k], cfg.ggml_type, cfg.n_expert, *cfg.rows_K(k))
                        for k in ("gate", "up", "down")}
            else:
                mats = {k: t[k] for k in ("gate", "up", "down")}
            layers.append(MoELayer(ggml_type=cfg.ggml_type, n_expert=cfg.n_expert, top_k=cfg.top_k,
                                   n_embd=cfg.n_embd, n_ff=cfg.n_ff, router_w=t["router_w"], router_b=t["router_b"],
                                   gate=mats["gate"], up=mats["up"], down=mats["down"], gate_b=t["gate_b"],
                                   up_b=t["up_b"], down_b=t["down_b"], layout=layout,
                                   router_mode=cfg.router_mode, act=cfg.act, dispatch=dispatch))
            del t, mats
        return cls(layers)


class _HostBlockStore:
    """One layer's expert matrices (t64 tiles) split into row blocks, a seeded
    share of which lives in pinned host RAM instead of HBM.

    Per projection: `dev` holds the HBM-resident blocks and `host` the others,
    each packed in (expert, block) order. An expert with no host block is one
    contiguous run of `dev` and is used in place; the others are assembled
    per step into a staging slot."""

    def __init__(self, full: dict, rows: dict, K: dict, n_expert: int, block_rows: int, host_fraction: float,
                 rng, device) -> None:
        from .. import _native as N
        if block_rows <= 0 or block_rows % 64:
            raise ValueError(f"block_rows {block_rows}: a positive multiple of the 64-row tile")
        lib = N.load()
        self.kinds = tuple(full)
        import numpy as np
        self.per, self.blocks, self.dev, self.host, self.where, self.whole = {}, {}, {}, {}, {}, {}
        self.tiles, self.block_bytes = {}, {}
        self.segs = {}
        self.host_bytes = 0
        for kind in self.kinds:
            per = lib.nsx_t64_bytes(39, rows[kind], K[kind])
            rb = per // (-(-rows[kind] // 64) * 64)  # bytes per (padded) row
            spans = [(r0, min(rows[kind], r0 + block_rows)) for r0 in range(0, rows[kind], block_rows)]
            # byte extent of a block of rows [r0, r1): whole 64-row tiles
            ext = [(r0 * rb, (-(-r1 // 64) * 64) * rb) for r0, r1 in spans]
            host = rng.random((n_expert, len(spans))) < host_fraction
            nd = int(sum((b1 - b0) for e in range(n_expert) for i, (b0, b1) in enumerate(ext) if not host[e, i]))
            nh = int(sum((b1 - b0) for e in range(n_expert) for i, (b0, b1) in enumerate(ext) if host[e, i]))
            dev = torch.empty(max(nd, 16), dtype=torch.uint8, device=device)
            hst = torch.empty(max(nh, 16), dtype=torch.uint8, pin_memory=True)
            where, od, oh = {}, 0, 0
            src = full[kind]
            for e in range(n_expert):
                for i, (b0, b1) in enumerate(ext):
                    n = b1 - b0
                    blk = src[e * per + b0:e * per + b1]
                    if host[e, i]:
                        hst[oh:oh + n].copy_(blk)
                        where[(e, i)] = ("host", oh, b0, n)
                        oh += n
                    else:
                        dev[od:od + n].copy_(blk)
                        where[(e, i)] = ("dev", od, b0, n)
                        od += n
            self.per[kind], self.blocks[kind] = per, len(spans)
            self.tiles[kind] = -(-rows[kind] // 64)
            self.block_bytes[kind] = block_rows * rb  # every block but the last spans this many bytes
            self.dev[kind], self.host[kind], self.where[kind] = dev, hst, where
            self.whole[kind] = [not host[e].any() for e in range(n_expert)]
            self.host_bytes += nh
            # per expert with host blocks: (host src addresses, dst offsets in a slot, bytes) and the
            # same for its HBM blocks (gather), as int64 arrays ready for the C calls
            hp, dp = hst.data_ptr(), dev.data_ptr()
            segs = {}
            for e in range(n_expert):
                if self.whole[kind][e]:
                    continue
                h_, g_ = [], []
                for i in range(len(spans)):
                    loc, off, b0, n = where[(e, i)]
                    (h_ if loc == "host" else g_).append((hp + off if loc == "host" else dp + off, b0, n))
                segs[e] = tuple(np.array(v, dtype=np.int64).reshape(-1, 3) for v in (h_, g_))
            self.segs[kind] = segs
        torch.cuda.synchronize(device)

    def address(self, kind: str, e: int) -> int | None:
        """Device address of expert e's whole matrix when all of it is in HBM."""
        if not self.whole[kind][e]:
            return None
        return self.dev[kind].data_ptr() + self.where[kind][(e, 0)][1]

    def tile_table(self, kind: str, device) -> torch.Tensor:
        """int64 device tensor: the address of every 64-row tile of every
        expert, in HBM or (device-mapped) in the pinned host blocks."""
        from .. import _native as N
        import ctypes as C
        lib = N.load()
        hdev = C.c_uint64(0)
        N.check(lib.nsx_host_device_address(self.host[kind].data_ptr(), C.byref(hdev)), "host device address")
        per, n_expert = self.per[kind], len(self.whole[kind])
        tiles = self.tiles[kind]
        tb = per // tiles
        dbase, hbase = self.dev[kind].data_ptr(), int(hdev.value)
        tab = []
        for e in range(n_expert):
            for t in range(tiles):
                loc, off, b0, n = self.where[kind][(e, (t * tb) // self.block_bytes[kind])]
                assert b0 <= t * tb and t * tb + tb <= b0 + n
                tab.append((dbase if loc == "dev" else hbase) + off + t * tb - b0)
        return torch.tensor(tab, dtype=torch.int64, device=device)

    def host_bytes_of(self, kind: str, e: int) -> int:
        """Bytes of expert e's matrix held in pinned host RAM."""
        return sum(n for (ee, _), (loc, _, _, n) in self.where[kind].items() if ee == e and loc == "host")


class _CopyFuture:
    """One block's DMA copy in flight: `done` polls its event, `result` orders
    the caller's stream after it on the GPU (no host wait) and returns the
    block's device address."""

    __slots__ = ("event", "address")

    def __init__(self, event, address: int) -> None:
        self.event, self.address = event, address

    def done(self) -> bool:
        return self.event.query()

    def result(self) -> int:
        torch.cuda.current_stream().wait_event(self.event)
        return self.address

    def cancel(self) -> bool:  # the copy is queued on the GPU already; its slot is the caller's
        return False


class _TileBlockSource:
    """One layer's host-resident expert blocks behind the block-source protocol
    BlockPrefetcher consumes (compute/blockffn.py:278-393 of the reference:
    `gguf.tensors` with row geometry, `has_slab`, `submit_rows(name, lo, hi)
    -> (future, nbytes)` under an arena lease, `reader.wait`, `arena`).

    Tensor names are the projections ("gate", "up", "down"); rows are the
    stacked experts' rows (expert e owns rows [e*out, (e+1)*out), as
    io/source.py:38-62), and a row's bytes are its share of the t64 tiles, so
    a block of 512 rows is 8 whole tiles. Windows whose blocks all sit in HBM
    count as held slabs. A submitted block is copied from pinned host RAM by
    DMA on the next of the stack's copy streams, straight to the address the
    caller put in `dest[(name, lo)]` (its place in a staging slot), so no
    block is copied twice; its future is that copy's event."""

    def __init__(self, store: _HostBlockStore, rows: dict, K: dict, block_rows: int, arena, streams) -> None:
        from ..format.gguf import GGMLType, TensorInfo
        from ..io.source import BlockReader, _Index
        self.store, self.rows, self.block_rows = store, rows, block_rows
        self.arena, self.streams = arena, streams
        self.reader = BlockReader()
        n_expert = len(store.whole[store.kinds[0]])
        infos = {}
        for kind in store.kinds:
            padded = store.tiles[kind] * 64
            rb = store.per[kind] // padded
            n_rows = n_expert * rows[kind]
            infos[kind] = TensorInfo(kind, (K[kind], n_rows), GGMLType.MXFP4, 0, n_expert * store.per[kind],
                                     geom=(n_rows, K[kind], rb))
        self.gguf = _Index(infos)
        self.dest: dict = {}
        self._next = 0
        self.bytes_copied = 0

    def _block(self, name: str, lo: int, hi: int):
        rows = self.rows[name]
        e, r0 = divmod(lo, rows)
        i = r0 // self.block_rows
        if r0 % self.block_rows or hi != e * rows + min(rows, (i + 1) * self.block_rows):
            raise ValueError(f"{name}: rows [{lo}, {hi}) are not one {self.block_rows}-row block of one expert")
        return e, i

    def is_resident(self, name: str) -> bool:
        return False

    def has_slab(self, name: str, lo: int, hi: int) -> bool:
        rows, br = self.rows[name], self.block_rows
        where = self.store.where[name]
        for r in range(lo, hi, br):
            e, r0 = divmod(r, rows)
            if where[(e, r0 // br)][0] != "dev":
                return False
        return True

    def submit_rows(self, name: str, start: int, end: int, *, timeout: float | None = None):
        """DMA-copy one host block to dest[(name, start)]: (future, nbytes); the caller releases."""
        from .. import _native as N
        e, i = self._block(name, start, end)
        loc, off, _b0, n = self.store.where[name][(e, i)]
        if loc != "host":
            raise ValueError(f"{name} rows [{start}, {end}) are in HBM: nothing to read")
        dst = self.dest[(name, start)]
        self.arena.acquire(n, timeout=timeout)
        try:
            cs = self.streams[self._next % len(self.streams)]
            self._next += 1
            seg = (C.c_uint64 * 1)(self.store.host[name].data_ptr() + off)
            dd = (C.c_uint64 * 1)(dst)
            nb = (C.c_int64 * 1)(n)
            N.check(N.load().nsx_copy_blocks_async(1, seg, dd, nb, cs.cuda_stream, None), "copy_blocks_async")
            ev = torch.cuda.Event()
            ev.record(cs)
            self.reader.stats.requests += 1
            self.reader.stats.bytes_read += n
            self.bytes_copied += n
            return _CopyFuture(ev, dst), n
        except BaseException:
            self.arena.release(n)
            raise


class GptOssHostStreamedStack(GptOssFFNStack):
    """BASELINE config 5b: the FFN stack with a seeded share (25%) of the
    experts' row blocks in pinned host RAM. Three ways to reach them:

    mode "read": every layer gets tile tables (MoELayer.set_tile_tables) that
    point each 64-row tile at HBM or at its pinned host block; the expert
    kernels read the host tiles over PCIe themselves. A step needs no host
    synchronisation and no staging copy, so it is one graph like the
    resident stack.

    mode "stage": per layer and step the router's ids come to the host
    (model/gpt_oss.py:121 does the same to pick its windows); every chosen
    expert matrix with host blocks is assembled in a staging slot -- its host
    blocks as DMA copies from pinned RAM (nsx_copy_blocks_async, all of the
    layer's blocks queued at once over COPY_STREAMS copy streams), its HBM
    blocks as one gather kernel (nsx_gather_copy) -- and the layer's expert
    address table points at the slots for this step.

    mode "prefetch": as "stage", but the host blocks go through the
    reference's prefetcher seam (compute/blockffn.py:278-393, one per layer as
    model/gpt_oss.py:133-160 builds it): a plan of the chosen experts' host
    blocks in the order the layer consumes them (ascending expert; gate, up,
    down), read `depth` blocks ahead by BlockPrefetcher over the layer's
    _TileBlockSource, each block a DMA copy on a copy stream into its slot
    under an arena lease of depth + 1 blocks, taken in plan order.

    Either way the experts run in the same fused kernels as the resident
    stack, with the same arithmetic: outputs are identical to it."""

    COPY_STREAMS = 4
    MODES = ("stage", "read", "prefetch")

    def __init__(self, layers, stores, eps: float = 1e-5, mode: str = "stage", block_rows: int = 512,
                 depth: int = 4) -> None:
        super().__init__(layers, eps=eps)
        self.stores = stores
        self.block_rows, self.depth = block_rows, depth
        self.bytes_from_host = 0
        self._tile_tabs = None
        self._slots = None
        self._sources = None
        self.arena = None
        self.mode = None
        self.set_mode(mode)

    def set_mode(self, mode: str) -> None:
        """Switch how the host blocks are reached; each mode's tables, slots
        and sources are built on first use and kept."""
        if mode not in self.MODES:
            raise ValueError(f"mode {mode!r}: one of {self.MODES}")
        if mode == "read":
            if self._tile_tabs is None:
                self._tile_tabs = [tuple(st.tile_table(k, self.device) for k in ("gate", "up", "down"))
                                   for st in self.stores]
            for layer, tabs in zip(self.layers, self._tile_tabs):
                layer.set_tile_tables(*tabs)
        else:
            for layer in self.layers:  # the expert address tables again, rewritten per step
                layer.set_tile_tables(None, None, None)
            self._make_slots()
            if mode == "prefetch":
                self._make_sources()
        self.mode = mode

    def _make_slots(self) -> None:
        if self._slots is not None:
            return
        stores = self.stores
        n_slots = min(self.cfg.n_expert, 64)
        self._slots = {k: torch.empty(n_slots * stores[0].per[k], dtype=torch.uint8, device=self.device)
                       for k in stores[0].kinds}
        self._tables = [{k: torch.empty(self.cfg.n_expert, dtype=torch.int64, pin_memory=True)
                         for k in stores[0].kinds} for _ in self.layers]
        # per step every entry starts at valid full-size memory: the expert itself or slot 0
        self._default = [{k: torch.tensor([st.address(k, e) or self._slots[k].data_ptr()
                                           for e in range(self.cfg.n_expert)], dtype=torch.int64)
                          for k in st.kinds} for st in stores]
        # host blocks spread over several copy streams (default priority), so
        # several DMA engines share the PCIe link
        self._copy_streams = [torch.cuda.Stream(self.device) for _ in range(self.COPY_STREAMS)]

    def _make_sources(self) -> None:
        if self._sources is not None:
            return
        from ..io.arena import Arena
        stores, depth = self.stores, self.depth
        rows = {k: (self.cfg.n_ffn_expert if k in ("gate", "up") else self.cfg.n_embd) for k in stores[0].kinds}
        K = {k: (self.cfg.n_embd if k in ("gate", "up") else self.cfg.n_ffn_expert) for k in stores[0].kinds}
        widest = max(st.block_bytes[k] for st in stores for k in st.kinds)
        # depth blocks in flight plus the one being taken (BlockPrefetcher's depth + 1 rule)
        self.arena = Arena((depth + 1) * widest)
        self._sources = [_TileBlockSource(st, rows, K, self.block_rows, self.arena,
                                          self._copy_streams[:max(1, min(depth, self.COPY_STREAMS))])
                         for st in stores]

    def _assign_slots(self, li: int, chosen):
        """Point the layer's expert tables at staging slots for the chosen
        experts that have host blocks: (host blocks [(kind, expert, block
        index, host address, slot address, bytes)], HBM segments (n, 3) int64
        of (source, slot address, bytes) to gather)."""
        import numpy as np
        st = self.stores[li]
        hblocks, gseg = [], []
        for kind in st.kinds:
            table = self._tables[li][kind]
            slot_base, per, bb = self._slots[kind].data_ptr(), st.per[kind], st.block_bytes[kind]
            n_slots = self._slots[kind].numel() // per
            table.copy_(self._default[li][kind])
            used = 0
            for e in chosen:
                seg = st.segs[kind].get(e)
                if seg is None:
                    continue
                if used >= n_slots:
                    raise RuntimeError(f"more than {n_slots} staged experts in one layer")
                dst = slot_base + used * per
                used += 1
                hs, gs = seg
                hblocks += [(kind, e, int(b0) // bb, int(src), dst + int(b0), int(n)) for src, b0, n in hs]
                if len(gs):
                    a = gs.copy()
                    a[:, 1] += dst
                    gseg.append(a)
                table[e] = dst
        G = np.concatenate(gseg) if gseg else np.zeros((0, 3), np.int64)
        return hblocks, G

    def _publish_tables(self, li: int) -> None:
        layer = self.layers[li]
        for kind, dev_table in (("gate", layer.gate_ptrs), ("up", layer.up_ptrs), ("down", layer.down_ptrs)):
            dev_table.copy_(self._tables[li][kind], non_blocking=True)

    def _stage(self, li: int, chosen) -> None:
        import numpy as np
        from .. import _native as N
        lib = N.load()
        hblocks, G = self._assign_slots(li, chosen)
        H = np.array([(src, dst, n) for _, _, _, src, dst, n in hblocks], dtype=np.int64).reshape(-1, 3)
        s = N.stream_ptr(self.device)
        col = lambda a, j: np.ascontiguousarray(a[:, j]).ctypes.data_as(C.c_void_p)  # noqa: E731
        with torch.cuda.device(self.device):
            cur = torch.cuda.current_stream(self.device)
            ns = len(self._copy_streams)
            for i, cs in enumerate(self._copy_streams[:len(H)]):
                part = H[i::ns]
                cs.wait_stream(cur)  # the slots are free once the work queued so far is done
                N.check(lib.nsx_copy_blocks_async(len(part), col(part, 0), col(part, 1), col(part, 2),
                                                  cs.cuda_stream, None), "copy_blocks_async")
            N.check(lib.nsx_gather_copy(len(G), col(G, 0), col(G, 1), col(G, 2), s), "gather_copy")
            for cs in self._copy_streams[:len(H)]:
                cur.wait_stream(cs)
            self._publish_tables(li)
        self.bytes_from_host += int(H[:, 2].sum()) if len(H) else 0

    def _prefetch(self, li: int, chosen) -> None:
        """The host blocks of the chosen experts through BlockPrefetcher, in
        the order the layer consumes them; the HBM blocks of the same experts
        gathered into their slots by one kernel."""
        import numpy as np
        from .. import _native as N
        from ..compute.blockffn import BlockPrefetcher
        src = self._sources[li]
        hblocks, G = self._assign_slots(li, chosen)
        order = {"gate": 0, "up": 1, "down": 2}
        hblocks.sort(key=lambda b: (b[1], order[b[0]], b[2]))  # ascending expert; gate, up, down
        br = self.block_rows
        plan, dest = [], {}
        for kind, e, i, _src, dst, _n in hblocks:
            rows = src.rows[kind]
            lo = e * rows + i * br
            plan.append((kind, lo, e * rows + min(rows, (i + 1) * br)))
            dest[(kind, lo)] = dst
        src.dest = dest
        s = N.stream_ptr(self.device)
        col = lambda a, j: np.ascontiguousarray(a[:, j]).ctypes.data_as(C.c_void_p)  # noqa: E731
        with torch.cuda.device(self.device):
            cur = torch.cuda.current_stream(self.device)
            for cs in src.streams:
                cs.wait_stream(cur)  # the slots are free once the work queued so far is done
            N.check(N.load().nsx_gather_copy(len(G), col(G, 0), col(G, 1), col(G, 2), s), "gather_copy")
            b0 = src.bytes_copied
            with BlockPrefetcher(src, plan, block_rows=br, depth=self.depth) as pf:
                if plan and not pf.enabled:
                    raise RuntimeError("the prefetcher's arena cannot hold depth + 1 blocks")
                for name, lo, hi in plan:
                    got = pf.take(name, lo)
                    if got is None:  # not read ahead: read it now, in order
                        fut, n = src.submit_rows(name, lo, hi)
                        src.reader.wait(fut)
                    else:
                        _, n = got
                    src.arena.release(n)  # the block is in its slot (ordered on `cur`): the lease ends
            self._publish_tables(li)
        self.bytes_from_host += src.bytes_copied - b0

    def prefetch_stats(self) -> dict:
        """Prefetch mode: blocks read, prefetch hits (copy already done when
        taken) and the arena's peak lease, over every call so far."""
        if not self._sources:
            return {}
        req = sum(s.reader.stats.requests for s in self._sources)
        hits = sum(s.reader.stats.prefetch_hits for s in self._sources)
        return {"blocks": req, "hits": hits, "arena_budget": self.arena.budget,
                "arena_peak": self.arena.stats.peak_bytes}

    def host_bytes_of_routing(self, ids) -> int:
        """Bytes read from pinned host RAM for a step routed as `ids` (per layer
        (T, k) expert ids): every chosen expert's host blocks, once per layer."""
        total = 0
        for li, st in enumerate(self.stores):
            for e in torch.unique(ids[li]).tolist():
                total += sum(st.host_bytes_of(k, e) for k in st.kinds)
        return total

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """As GptOssFFNStack.forward; in "stage" and "prefetch" modes one host
        synchronisation per layer (routing)."""
        if self.mode == "read":
            return GptOssFFNStack.forward(self, x, out)
        from ..moe.fused import router_topk
        x = x.reshape(-1, self.cfg.n_embd)
        T = x.shape[0]
        h, y, ids, wts = self._buffers(T)
        res = torch.empty_like(x) if out is None else out
        eps = self.cfg.rms_eps
        add_rms_norm(x.float().contiguous(), None, self.norm_weights[0], eps, out=h, sum_out=res)
        stage = self._prefetch if self.mode == "prefetch" else self._stage
        for li, layer in enumerate(self.layers):
            rid, _, _ = router_topk(h, layer.router_w, layer.router_b, layer.top_k, "gptoss")
            chosen = torch.unique(rid).tolist()  # device -> host, as the reference
            stage(li, chosen)
            layer.forward(h, out=y, ids=ids[li], weights=wts[li])
            if li + 1 < len(self.layers):
                add_rms_norm(res, y, self.norm_weights[li + 1], eps, out=h, sum_out=res)
            else:
                res.add_(y)
        return res

    __call__ = forward

    @classmethod
    def synthetic(cls, cfg, n_layers: int, seed: int, device, host_fraction: float = 0.25, block_rows: int = 512,
                  dispatch: str = "auto", mode: str = "stage", depth: int = 4):
        """BASELINE config 5b: the layers of GptOssFFNStack.synthetic with a
        seeded host_fraction of their block_rows-row blocks in pinned RAM
        (prefetch mode: read `depth` blocks ahead)."""
        import numpy as np
        from .. import synth
        from ..compute.kernels import t64_pack_stacked
        layers, stores = [], []
        for li in range(n_layers):
            t = synth.make_layer(cfg, seed=seed, device=device, layer=li)
            full = {k: t64_pack_stacked(t[k], cfg.ggml_type, cfg.n_expert, *cfg.rows_K(k))
                    for k in ("gate", "up", "down")}
            for k in ("gate", "up", "down"):
                t[k] = None
            rng = np.random.default_rng(synth.layer_seed(seed, li) + 99991)
            st = _HostBlockStore(full, {k: cfg.rows_K(k)[0] for k in full}, {k: cfg.rows_K(k)[1] for k in full},
                                 cfg.n_expert, block_rows, host_fraction, rng, device)
            del full
            views = {}
            for k in st.kinds:
                per = st.per[k]
                views[k] = [st.dev[k][st.where[k][(e, 0)][1]:st.where[k][(e, 0)][1] + per] if st.whole[k][e]
                            else None for e in range(cfg.n_expert)]
            slot0 = {k: torch.empty(st.per[k], dtype=torch.uint8, device=device) for k in st.kinds}
            mats = {k: [v if v is not None else slot0[k] for v in views[k]] for k in st.kinds}
            layers.append(MoELayer(ggml_type=cfg.ggml_type, n_expert=cfg.n_expert, top_k=cfg.top_k,
                                   n_embd=cfg.n_embd, n_ff=cfg.n_ff, router_w=t["router_w"], router_b=t["router_b"],
                                   gate=mats["gate"], up=mats["up"], down=mats["down"], gate_b=t["gate_b"],
                                   up_b=t["up_b"], down_b=t["down_b"], layout="t64",
                                   router_mode=cfg.router_mode, act=cfg.act, dispatch=dispatch))
            stores.append(st)
            del t
        return cls(layers, stores, mode=mode, block_rows=block_rows, depth=depth)


@dataclass
class MoEModelConfig:
    """The MoE-path subset of the reference's model config (model/qwen3.py,
    from_gguf: the same GGUF keys)."""
    n_layer: int
    n_embd: int
    n_expert: int
    n_expert_used: int
    n_ffn_expert: int
    rms_eps: float = 1e-6

    @classmethod
    def from_gguf(cls, g) -> "MoEModelConfig":
        n_ffn = int(g.cfg("feed_forward_length", 0) or 0)
        return cls(n_layer=int(g.cfg("block_count")), n_embd=int(g.cfg("embedding_length")),
                   n_expert=int(g.cfg("expert_count", 0) or 0), n_expert_used=int(g.cfg("expert_used_count", 0) or 0),
                   n_ffn_expert=int(g.cfg("expert_feed_forward_length", 0) or 0) or n_ffn,
                   rms_eps=float(g.cfg("attention.layer_norm_rms_epsilon", 1e-6)))


class GptOssModel:
    """The routed-expert FFN blocks of a GPT-OSS GGUF over a TieredCache
    (model/gpt_oss.py:97-177 of the reference).

    `_ffn_block(x, layer)` = x + moe(rms_norm(x, post_attention_norm)):
      * when every expert of the layer has its three slabs in HBM (t64), one
        fused MoE layer call over the slabs' addresses (no host sync);
      * otherwise the reference's neuron path: route (ids to the host), one
        BlockPrefetcher plan for the layer, stream_expert_ffn per chosen expert
        in ascending id, out[rows] += w_e * y_e -- every block product on the
        HIP GEMV, slab hits in place, the rest streamed through submit_rows.
    """

    def __init__(self, cache, cfg: MoEModelConfig, device, dtype=torch.float32, block_rows: int = 1024,
                 expert_lookahead: int = 2) -> None:
        self.cache = cache
        self.gguf = cache.gguf
        self.cfg = cfg
        self.device = torch.device(device)
        self.dtype = dtype
        self.block_rows = block_rows
        self.expert_lookahead = expert_lookahead
        self.router_stats = RouterStats()
        self.neuron_callback = None
        self._w: dict[str, torch.Tensor] = {}
        self._fused: dict[int, MoELayer] = {}
        self._acfg = None
        self._capturing: list | None = None

    def w(self, name: str) -> torch.Tensor:
        t = self._w.get(name)
        if t is None:
            t = self.cache.get(name).to(self.device, torch.float32)
            self._w[name] = t
        return t

    def has(self, name: str) -> bool:
        return name in self.gguf.tensors

    def _route(self, h: torch.Tensor, layer: int):
        """(chosen (host list, ascending), ids (T, k) int64, weights (T, k)), gpt_oss.py:116-121."""
        from ..moe.fused import router_topk
        p = f"blk.{layer}.ffn_gate_inp"
        bias = self.w(p + ".bias") if self.has(p + ".bias") else None
        ids, wts, _ = router_topk(h, self.w(p + ".weight"), bias, self.cfg.n_expert_used, "gptoss")
        return torch.unique(ids).tolist(), ids.long(), wts

    def _fused_layer(self, layer: int) -> MoELayer | None:
        """A MoELayer over this layer's t64 slabs when all 3 x n_expert are admitted."""
        lay = self._fused.get(layer)
        if lay is not None:
            return lay
        c, p = self.cfg, f"blk.{layer}."
        mats = {}
        for kind, rpe in (("gate", c.n_ffn_expert), ("up", c.n_ffn_expert), ("down", c.n_embd)):
            slabs = []
            for e in range(c.n_expert):
                ent = self.cache.slab_entry(p + f"ffn_{kind}_exps.weight", e * rpe, (e + 1) * rpe)
                if ent is None or ent[1] != "t64":
                    return None
                slabs.append(ent[0])
            mats[kind] = slabs
        bias = lambda n: self.w(n) if self.has(n) else None  # noqa: E731
        rb = bias(p + "ffn_gate_inp.bias")
        lay = MoELayer(ggml_type=self.gguf.tensors[p + "ffn_gate_exps.weight"].dtype, n_expert=c.n_expert,
                       top_k=c.n_expert_used, n_embd=c.n_embd, n_ff=c.n_ffn_expert,
                       router_w=self.w(p + "ffn_gate_inp.weight"), router_b=rb, gate=mats["gate"], up=mats["up"],
                       down=mats["down"], gate_b=bias(p + "ffn_gate_exps.bias"), up_b=bias(p + "ffn_up_exps.bias"),
                       down_b=bias(p + "ffn_down_exps.bias"), layout="t64", router_mode="gptoss",
                       act="clamped_swiglu")
        self._fused[layer] = lay
        return lay

    def _ffn_block(self, x: torch.Tensor, layer: int) -> torch.Tensor:
        from ..compute.blockffn import BlockPrefetcher, stream_expert_ffn
        c, p = self.cfg, f"blk.{layer}."
        x = x.reshape(-1, c.n_embd).to(self.device, torch.float32).contiguous()
        norm = p + "post_attention_norm.weight"
        h = add_rms_norm(x, None, self.w(norm) if self.has(norm) else None, c.rms_eps)
        fused = self._fused_layer(layer)
        if fused is not None:
            out, ids, _ = fused.forward(h)
            if self._capturing is not None:  # no host copy inside a graph capture: recorded after each replay
                self._capturing.append((layer, ids))
            else:
                self.router_stats.record(layer, ids)
            return x + out
        chosen, ids, weights = self._route(h, layer)
        stats = self.router_stats
        stats.tokens_routed += h.shape[0]
        out = torch.zeros_like(h)
        active = []
        for e in chosen:
            mask = ids == e
            rows = mask.any(-1).nonzero(as_tuple=True)[0]
            if rows.numel():
                active.append((e, rows, (weights * mask).sum(-1)[rows, None]))
        plan = [(p + f"ffn_{kind}_exps.weight", e * span, (e + 1) * span) for e, _r, _w in active
                for kind, span in (("gate", c.n_ffn_expert), ("up", c.n_ffn_expert), ("down", c.n_embd))]
        pf = BlockPrefetcher(self.cache, plan, self.block_rows, self.expert_lookahead)
        try:
            for e, rows, wgt in active:
                stats.hits[(layer, e)] += rows.numel()
                stats.expert_reads += 1
                out[rows] += wgt * stream_expert_ffn(self.cache, p, e, h[rows], c.n_ffn_expert, c.n_embd,
                                                     clamped_swiglu, self.block_rows, self.device, torch.float32,
                                                     bias=True, lookahead=self.expert_lookahead,
                                                     callback=self.neuron_callback, prefetcher=pf)
        finally:  # a failed forward must not strand arena leases
            pf.close()
        return x + out

    def ffn_stack(self, x: torch.Tensor) -> torch.Tensor:
        """x after every layer's FFN block."""
        for layer in range(self.cfg.n_layer):
            x = self._ffn_block(x, layer)
        return x

    # -- the step either side of the FFN (model/gpt_oss.py:97-114, 207-228) --

    def attn_config(self):
        from .decode import AttnConfig, yarn_inv_freq
        if self._acfg is None:
            need = ["token_embd.weight", "output_norm.weight"] + [
                f"blk.{li}.{n}" for li in range(self.cfg.n_layer)
                for n in ("attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight")]
            missing = [n for n in need if not self.has(n)]
            if missing or self.gguf.cfg("attention.head_count") is None:
                raise NotImplementedError(
                    f"a decode token needs the embedding, attention and output tensors; this GGUF lacks "
                    f"{missing[:3] or ['attention.head_count']}{' ...' if len(missing) > 3 else ''}")
            self._acfg = AttnConfig.from_gguf(self.gguf)
            self._inv_freq, self._amp = yarn_inv_freq(self._acfg, self.device)
        return self._acfg

    def _resident_raw(self, name: str):
        """(raw device bytes, dtype) of a quantized tensor held whole in the HBM
        tier, or None (a RAM-tier tensor is not: it takes the streamed paths)."""
        return self.cache.vram_raw(name)

    def _linear(self, name: str, x: torch.Tensor) -> torch.Tensor:
        """x @ W.T in fp32 (model/qwen3.py:169-194): the fused GEMV on HBM-resident
        raw rows, else stream_linear by row blocks; float tensors by matmul."""
        from ..compute.blockffn import stream_linear
        from ..compute.kernels import can_fuse, fused_gemv
        from ..format.gguf import FLOAT_TYPES, row_geometry
        info = self.gguf.tensors[name]
        n_rows, K, _ = row_geometry(info)
        if info.dtype in FLOAT_TYPES:
            return x @ self.w(name).T
        hit = self._resident_raw(name)
        if hit is not None and can_fuse(hit[1], x):
            return fused_gemv(hit[0], hit[1], x, n_rows, K, out_dtype=torch.float32)
        return stream_linear(self.cache, name, x, self.block_rows, self.device, torch.float32)

    def _biased_linear(self, name: str, x: torch.Tensor) -> torch.Tensor:
        out = self._linear(name + ".weight", x)
        return out + self.w(name + ".bias") if self.has(name + ".bias") else out

    def embed(self, ids: torch.Tensor) -> torch.Tensor:
        """Rows of token_embd for device int32 ids -> (T, n_embd) fp32 (gather_embeddings, blockffn.py:470-487)."""
        from ..format.gguf import FLOAT_TYPES, row_geometry
        from .decode import dequantize_rows
        name = "token_embd.weight"
        info = self.gguf.tensors[name]
        n_rows, K, _ = row_geometry(info)
        if info.dtype in FLOAT_TYPES:
            return self.w(name).reshape(n_rows, K)[ids.long()]
        hit = self._resident_raw(name)
        if hit is not None:
            return dequantize_rows(hit[0], hit[1], n_rows, K, ids)
        return torch.stack([self.cache.fetch_rows(name, t, t + 1, device=self.device, dtype=torch.float32)[0]
                            for t in ids.tolist()])

    def _qkv_raw(self, layer: int):
        """(raw bytes, dtype, rows) of the layer's q, k and v weights laid out
        back to back in HBM by the cache (TieredCache.fuse_vram: the three
        residents become views of one buffer, no extra bytes) -- one GEMV then
        writes the q | k | v block -- or None when they are not all HBM-tier
        quantized rows of one type."""
        from ..format.gguf import row_geometry
        p = f"blk.{layer}."
        names = [p + n + ".weight" for n in ("attn_q", "attn_k", "attn_v")]
        got = self.cache.fuse_vram(names)
        if got is None:
            return None
        rows = sum(row_geometry(self.gguf.tensors[n])[0] for n in names)
        return got[0], got[1], rows

    def _attention_block(self, x: torch.Tensor, layer: int, kv, pending: torch.Tensor | None = None) -> torch.Tensor:
        """x + o_proj(sink_attention(...)) for the one token at kv.pos (gpt_oss.py:101-114).

        `pending` (the previous FFN output) is added to x first, inside the
        attention norm's kernel (x is updated in place). Then one GEMV for q|k|v,
        the sink attention (sliding window on even layers) with the bias,
        rotary and cache append of the token's q / k / v in the same launch,
        and one GEMV for the output projection with its bias and the
        residual."""
        from ..compute.kernels import can_fuse, fused_gemv
        from ..format.gguf import row_geometry
        from .decode import attn_decode_qkv
        c, p = self.attn_config(), f"blk.{layer}."
        wn = self.w(p + "attn_norm.weight")
        cat = self._qkv_raw(layer)
        if cat is not None and self._norm_fusable(cat[1], x, pending, wn):
            # the attention norm in the QKV GEMV's prologue; x + pending goes to a new residual buffer
            # (the GEMV's other workgroups still read x)
            xs = torch.empty_like(x) if pending is not None else None
            qkv = self._gemv_norm(cat[0], cat[1], cat[2], x, pending, wn, xs).reshape(-1)
            if xs is not None:
                x = xs
        else:
            h = add_rms_norm(x, pending, wn, self.cfg.rms_eps, sum_out=x if pending is not None else None)
            if cat is not None and can_fuse(cat[1], h):
                qkv = fused_gemv(cat[0], cat[1], h, cat[2], h.shape[-1], out_dtype=torch.float32).reshape(-1)
            else:
                qkv = torch.cat([self._linear(p + n + ".weight", h).reshape(-1)
                                 for n in ("attn_q", "attn_k", "attn_v")])
        b = lambda n: self.w(p + n + ".bias") if self.has(p + n + ".bias") else None  # noqa: E731
        sinks = self.w(p + "attn_sinks.weight") if self.has(p + "attn_sinks.weight") else None
        att = attn_decode_qkv(qkv, b("attn_q"), b("attn_k"), b("attn_v"), c, self._inv_freq, self._amp, kv, layer,
                              sinks, c.sliding_window if layer % 2 == 0 else 0).reshape(1, -1)
        o_name = p + "attn_output.weight"
        hit = self._resident_raw(o_name)
        if hit is not None and can_fuse(hit[1], att):
            n_rows, K, _ = row_geometry(self.gguf.tensors[o_name])
            return fused_gemv(hit[0], hit[1], att, n_rows, K, out_dtype=torch.float32, bias=b("attn_output"),
                              resid=x)
        return x + self._biased_linear(p + "attn_output", att)

    def _ffn_pending(self, x: torch.Tensor, layer: int):
        """(x, moe output) for a fused layer -- the residual add is left to the
        next norm kernel -- or (x + ffn(x), None) on the streamed path."""
        fused = self._fused_layer(layer)
        if fused is None:
            return self._ffn_block(x, layer), None
        p = f"blk.{layer}."
        norm = p + "post_attention_norm.weight"
        h = add_rms_norm(x, None, self.w(norm) if self.has(norm) else None, self.cfg.rms_eps)
        out, ids, _ = fused.forward(h)
        if self._capturing is not None:  # no host copy inside a graph capture: recorded after each replay
            self._capturing.append((layer, ids))
        else:
            self.router_stats.record(layer, ids)
        return x, out

    def _norm_fusable(self, dtype, x: torch.Tensor, pending: torch.Tensor | None, wn) -> bool:
        """Whether a one-token GEMV can take the block norm of x (+ pending) in its prologue
        (nsx_fused_gemv_norm: fp32 vectors of K <= 4096 values, x 16-byte aligned)."""
        from ..compute.kernels import can_fuse
        vecs = [x] + [t for t in (pending, wn) if t is not None]
        K = x.shape[-1]
        return (can_fuse(dtype, x) and x.numel() == K and K <= 4096 and x.data_ptr() % 16 == 0
                and all(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous() and t.numel() == K
                        for t in vecs))

    def _gemv_norm(self, raw, dtype, n_rows: int, x, pending, wn, sum_out=None) -> torch.Tensor:
        from ..compute.kernels import fused_gemv_norm
        K = x.shape[-1]
        return fused_gemv_norm(raw, dtype, x.reshape(-1), None if pending is None else pending.reshape(-1), wn,
                               self.cfg.rms_eps, n_rows, K, sum_out=None if sum_out is None else sum_out.reshape(-1))

    def _head(self, x: torch.Tensor, pending: torch.Tensor | None = None) -> torch.Tensor:
        """Logits of the last hidden state (+ pending): output_norm, then output.weight (or the tied embedding)."""
        from ..format.gguf import row_geometry
        name = "output.weight" if self.has("output.weight") else "token_embd.weight"
        wn = self.w("output_norm.weight")
        hit = self._resident_raw(name) if name in self.gguf.tensors else None
        x = x.contiguous()
        if hit is not None and self._norm_fusable(hit[1], x, pending, wn):  # the output norm in the GEMV's prologue
            return self._gemv_norm(hit[0], hit[1], row_geometry(self.gguf.tensors[name])[0], x, pending, wn)
        h = add_rms_norm(x, pending, wn, self.cfg.rms_eps)
        return self._linear(name, h)

    def _decode_one(self, ids: torch.Tensor, kv) -> torch.Tensor:
        """One token (device int32 id) through every layer at kv.pos; kv.pos += 1 on the device."""
        from .decode import advance
        x = self.embed(ids).reshape(1, -1).contiguous()
        pending = None
        for layer in range(self.cfg.n_layer):
            x = self._attention_block(x, layer, kv, pending)
            x, pending = self._ffn_pending(x, layer)
        logits = self._head(x, pending)
        advance(kv)
        return logits

    def forward(self, tokens, kv=None, start_pos: int = 0, last_only: bool = True) -> torch.Tensor:
        """Logits (model/gpt_oss.py:207-228): (1, vocab), or (T, vocab) when not
        last_only. Tokens go through one at a time at positions start_pos..;
        kv is a DeviceKV whose length must be start_pos (a new one sized for
        these tokens when None)."""
        from .decode import DeviceKV
        c = self.attn_config()
        ids = torch.as_tensor(tokens, dtype=torch.int32).reshape(-1).to(self.device)
        T = ids.numel()
        if start_pos + T > c.context_length:
            raise ValueError("prompt and continuation exceed model context length")
        if kv is None:
            kv = DeviceKV(self.cfg.n_layer, c, start_pos + T, self.device)
            if start_pos:
                kv.pos.fill_(start_pos)
                kv.length = start_pos
        if kv.length != start_pos:
            raise ValueError(f"start_pos {start_pos} does not follow the cache's {kv.length} positions")
        if start_pos + T > kv.ctx_max:
            raise ValueError(f"{start_pos + T} positions exceed the cache's capacity of {kv.ctx_max}")
        outs = [self._decode_one(ids[i:i + 1], kv) for i in range(T)]
        return outs[-1] if last_only else torch.cat(outs)


class GptOssDecodeGraph:
    """One decode token of a GptOssModel -- embedding, every layer's attention
    and fused MoE FFN, output norm, LM head and the position step -- captured
    as one HIP graph over a DeviceKV, replayed once per token.

    Needs every quantized dense tensor whole in HBM and every layer's experts
    as t64 slabs (no host synchronisation inside a token)."""

    def __init__(self, model: GptOssModel, kv) -> None:
        from ..format.gguf import FLOAT_TYPES
        from .decode import DeviceKV
        self.model, self.kv = model, kv
        c = model.attn_config()
        for name, info in model.gguf.tensors.items():
            if ".ffn_" in name and "_exps." in name:
                continue
            if info.dtype not in FLOAT_TYPES and model._resident_raw(name) is None:
                raise ValueError(f"{name} is not resident in HBM: a decode graph reads every dense tensor in place")
        for layer in range(model.cfg.n_layer):
            if model._fused_layer(layer) is None:
                raise ValueError(f"layer {layer}: experts are not all t64 slabs in HBM")
        self.ids = torch.zeros(1, dtype=torch.int32, device=model.device)
        # one eager token on a scratch cache runs every lazy setup step before capture
        scratch = DeviceKV(model.cfg.n_layer, c, 1, model.device)
        model._capturing = []
        try:
            model._decode_one(self.ids, scratch)
            torch.cuda.synchronize(model.device)
            model._capturing = []
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.logits = model._decode_one(self.ids, kv)
            kv.length -= 1  # the capture did not run the step
            self._routing = model._capturing
        finally:
            model._capturing = None
        del scratch

    def step(self, token: int, record: bool = True) -> torch.Tensor:
        """Logits (1, vocab) of `token` at the cache's next position (the graph's own buffer)."""
        if self.kv.length >= self.kv.ctx_max:
            raise ValueError(f"the cache's {self.kv.ctx_max} positions are used up")
        self.ids.fill_(int(token))
        self.graph.replay()
        self.kv.length += 1
        if record:
            for layer, ids in self._routing:
                self.model.router_stats.record(layer, ids)
        return self.logits
