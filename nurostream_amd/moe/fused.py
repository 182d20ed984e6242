"""One MoE FFN layer as a single HIP call sequence (router -> experts -> combine).

`MoELayer` wraps nsx_moe_forward (include/nurostream_amd.h): the router's
top-k, the routed experts' gate/up GEMVs with bias and activation, the down
GEMVs with bias and the ascending-expert weighted combine all run on the
device, with expert ids never leaving it (the reference syncs to the host at
model/gpt_oss.py:121 and moe/router.py:183 to pick windows).

Expert weights are either one stacked tensor per projection (expert e at
base + e * expert_bytes: the kernels compute the address, no table lookup) or
a list of separately admitted slabs (a device table of addresses); all three
projections of a layer share one layout (raw GGUF rows or t64 tiles).
"""
from __future__ import annotations

import ctypes as C

import torch

from .. import _native as N
from ..format.gguf import GGMLType, TYPE_LAYOUT

_W_CODE = {torch.float32: int(GGMLType.F32), torch.bfloat16: int(GGMLType.BF16),
           torch.float16: int(GGMLType.F16)}


_DISPATCH = {"auto": 0, "pairs": 1, "grouped": 2, "mfma": 3}  # NSX_DISPATCH_*


def _addr_table(ptrs, device) -> torch.Tensor:
    return torch.tensor([int(p) for p in ptrs], dtype=torch.int64, device=device)


class MoELayer:
    def __init__(self, *, ggml_type, n_expert: int, top_k: int, n_embd: int, n_ff: int,
                 router_w: torch.Tensor, router_b: torch.Tensor | None,
                 gate, up, down, gate_b=None, up_b=None, down_b=None,
                 layout: str = "gguf", router_mode: str = "gptoss", act: str = "clamped_swiglu",
                 alpha: float = 1.702, limit: float = 7.0, dispatch: str = "auto") -> None:
        """gate/up/down: either one stacked uint8 device tensor per projection
        (expert e at offset e * bytes_per_expert) or a list of n_expert device
        tensors (one slab each). dispatch: "pairs" runs each (token, expert)
        pair on its own, "grouped" sorts the pairs by expert and reads each
        active expert once per work item of up to 16 tokens (t64 layout),
        "auto" groups from 3 tokens on (t64). These give identical outputs.
        "mfma" groups stacked Q4_K experts and runs them on the matrix cores
        (within 1e-5 of the others, not identical); "auto" takes it for such
        layers from 104 (token, expert) pairs on (T * top_k)."""
        if dispatch not in _DISPATCH:
            raise ValueError(f"dispatch {dispatch!r} not in {sorted(_DISPATCH)}")
        self.device = router_w.device
        N.require_device(router_w)
        self.ggml_type = GGMLType(ggml_type)
        self.n_expert, self.top_k, self.n_embd, self.n_ff = n_expert, top_k, n_embd, n_ff
        self.layout = layout
        be, bb = TYPE_LAYOUT[self.ggml_type]
        lib = N.load()

        def table(w, rows, K):
            """(tensors to keep alive, device address table or None, base address, stride)."""
            if isinstance(w, (list, tuple)):
                if len(w) != n_expert:
                    raise ValueError(f"{len(w)} expert slabs for {n_expert} experts")
                keep = list(w)
                return keep, _addr_table([t.data_ptr() for t in keep], self.device), None, 0
            if layout == "t64":
                per = lib.nsx_t64_bytes(int(self.ggml_type), rows, K)
            else:
                per = rows * (K // be) * bb
            if w.numel() < per * n_expert:
                raise ValueError(f"stacked tensor of {w.numel()} bytes, need {per * n_expert}")
            return [w], None, w.data_ptr(), per

        self._keep = []
        (k1, self.gate_ptrs, gb, gs), (k2, self.up_ptrs, ub, us), (k3, self.down_ptrs, db, ds) = (
            table(gate, n_ff, n_embd), table(up, n_ff, n_embd), table(down, n_embd, n_ff))
        self._keep += k1 + k2 + k3
        self.router_w = router_w.contiguous()
        self.router_b = None if router_b is None else router_b.float().contiguous()
        self.gate_b = None if gate_b is None else gate_b.float().contiguous()
        self.up_b = None if up_b is None else up_b.float().contiguous()
        self.down_b = None if down_b is None else down_b.float().contiguous()

        L = N.MoeLayerC()
        L.ggml_type = int(self.ggml_type)
        L.layout = N.LAYOUT_T64 if layout == "t64" else N.LAYOUT_GGUF
        L.n_expert, L.top_k, L.n_embd, L.n_ff = n_expert, top_k, n_embd, n_ff
        L.router_mode = N.ROUTE_GPTOSS if router_mode == "gptoss" else N.ROUTE_QWEN3
        L.act = N.ACT_CLAMPED_SWIGLU if act == "clamped_swiglu" else N.ACT_SILU_MUL
        L.alpha, L.limit = alpha, limit
        L.dispatch = _DISPATCH[dispatch]
        self.dispatch = dispatch
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        L.router_w = self.router_w.data_ptr()
        L.router_dtype = _W_CODE[self.router_w.dtype]
        L.router_bias = ptr(self.router_b)
        L.gate_ptrs, L.up_ptrs, L.down_ptrs = ptr(self.gate_ptrs), ptr(self.up_ptrs), ptr(self.down_ptrs)
        L.gate_base, L.up_base, L.down_base = gb, ub, db
        L.gate_stride, L.up_stride, L.down_stride = gs, us, ds
        L.gate_bias, L.up_bias, L.down_bias = ptr(self.gate_b), ptr(self.up_b), ptr(self.down_b)
        self._c = L
        self._ws: dict[int, torch.Tensor] = {}

    def set_tile_tables(self, gate, up, down) -> None:
        """t64 layers: per projection an int64 device tensor of n_expert x
        ceil(rows / 64) tile addresses (tile t of expert e at [e * tiles + t];
        a tile may sit in device-mapped pinned host memory, read over PCIe),
        or None to use the stacked/slab addresses again."""
        if self.layout != "t64":
            raise ValueError("tile tables need the t64 layout")
        tabs = (gate, up, down)
        for name, rows, t in (("gate", self.n_ff, gate), ("up", self.n_ff, up), ("down", self.n_embd, down)):
            if t is not None:
                N.require_device(t)
                if t.dtype != torch.int64 or t.numel() != self.n_expert * (-(-rows // 64)):
                    raise ValueError(f"{name} tile table: int64 with {self.n_expert} x {-(-rows // 64)} entries")
            setattr(self._c, name + "_tiles", None if t is None else t.data_ptr())
        self._tiles = tabs  # keep the tables alive with the layer

    def workspace(self, T: int) -> torch.Tensor:
        ws = self._ws.get(T)
        if ws is None:
            n = N.load().nsx_moe_workspace_bytes(C.byref(self._c), T)
            if n < 0:
                raise ValueError(f"bad layer for T={T}")
            # zeroed once: padding inside the workspace must read as zero
            ws = torch.zeros(max(n, 256), dtype=torch.uint8, device=self.device)
            self._ws[T] = ws
        return ws

    def _check_buffers(self, T: int, out: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor) -> None:
        """The native call writes through raw pointers: each output must be a
        contiguous tensor of exactly the expected shape and dtype on this
        layer's device, or a ValueError is raised before anything runs."""
        for name, t, shape, dtype in (("out", out, (T, self.n_embd), torch.float32),
                                      ("ids", ids, (T, self.top_k), torch.int32),
                                      ("weights", weights, (T, self.top_k), torch.float32)):
            if not isinstance(t, torch.Tensor):
                raise ValueError(f"{name} must be a tensor")
            if t.device != self.device:
                raise ValueError(f"{name} is on {t.device}, the layer on {self.device}")
            if t.dtype != dtype or tuple(t.shape) != shape or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous {dtype} tensor of shape {shape}, got "
                                 f"{t.dtype} {tuple(t.shape)}{'' if t.is_contiguous() else ' (strided)'}")

    def _prepare(self, h: torch.Tensor, out, ids, weights):
        N.require_device(h)
        h = h.reshape(-1, self.n_embd)
        if h.dtype != torch.float32:
            h = h.float()
        h = h.contiguous()
        if h.device != self.device:
            raise ValueError(f"h is on {h.device}, the layer on {self.device}")
        T = h.shape[0]
        if out is None:
            out = torch.empty((T, self.n_embd), dtype=torch.float32, device=self.device)
        if ids is None:
            ids = torch.empty((T, self.top_k), dtype=torch.int32, device=self.device)
        if weights is None:
            weights = torch.empty((T, self.top_k), dtype=torch.float32, device=self.device)
        self._check_buffers(T, out, ids, weights)
        return h, T, out, ids, weights

    def forward_static(self, h: torch.Tensor, out: torch.Tensor | None = None, ids: torch.Tensor | None = None,
                       weights: torch.Tensor | None = None):
        """forward() through nsx_moe_forward_static: no workspace, no device
        allocation by the library (the workspace is its per-GPU static array,
        shared by every such call on the GPU). The same outputs as forward()."""
        h, T, out, ids, weights = self._prepare(h, out, ids, weights)
        with torch.cuda.device(self.device):
            N.check(N.load().nsx_moe_forward_static(C.byref(self._c), h.data_ptr(), T, out.data_ptr(),
                                                    ids.data_ptr(), weights.data_ptr(), N.stream_ptr(self.device)),
                    "moe_forward_static")
        return out, ids, weights

    def forward(self, h: torch.Tensor, out: torch.Tensor | None = None, ids: torch.Tensor | None = None,
                weights: torch.Tensor | None = None):
        """h: (T, n_embd) fp32 -> (out (T, n_embd) fp32, ids (T, k) int32, weights (T, k) fp32)."""
        h, T, out, ids, weights = self._prepare(h, out, ids, weights)
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            N.check(N.load().nsx_moe_forward(C.byref(self._c), h.data_ptr(), T, out.data_ptr(), ids.data_ptr(),
                                             weights.data_ptr(), ws.data_ptr(), ws.numel(),
                                             N.stream_ptr(self.device)), "moe_forward")
        return out, ids, weights

    __call__ = forward

    def norm_folds(self, T: int) -> bool:
        """Whether forward_norm runs the block's input norm inside the router
        kernel for T tokens: t64 layout, n_embd <= 4096, and T <= 2 (nsx_moe_forward_norm
        takes T < 16, but from three tokens on the router reads x and r twice and a separate
        norm launch measures faster)."""
        return self.layout == "t64" and T <= 2 and self.n_embd <= 4096

    def forward_norm(self, x: torch.Tensor, r: torch.Tensor, norm_w: torch.Tensor | None, eps: float,
                     x_out: torch.Tensor, out: torch.Tensor, ids: torch.Tensor | None = None,
                     weights: torch.Tensor | None = None):
        """One stacked block (model/gpt_oss.py:123-177): x_out = x + r and
        forward(rms_norm(x + r) * norm_w) into out, the norm computed inside the
        router kernel (norm_folds(T)) -- the bits of add_rms_norm + forward.
        x, r, x_out: (T, n_embd) contiguous fp32; x_out must not overlap x or r;
        out may be r."""
        N.require_device(x, r, x_out)
        T = x.shape[0]
        for name, t in (("x", x), ("r", r), ("x_out", x_out)):
            if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != (T, self.n_embd) \
                    or t.device != self.device:
                raise ValueError(f"{name} must be a contiguous fp32 ({T}, {self.n_embd}) tensor on {self.device}")
        if ids is None:
            ids = torch.empty((T, self.top_k), dtype=torch.int32, device=self.device)
        if weights is None:
            weights = torch.empty((T, self.top_k), dtype=torch.float32, device=self.device)
        self._check_buffers(T, out, ids, weights)
        w = None
        if norm_w is not None:
            w = norm_w.to(device=self.device, dtype=torch.float32).contiguous()
            if w.numel() != self.n_embd:
                raise ValueError(f"norm weight of {w.numel()} values, n_embd is {self.n_embd}")
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            N.check(N.load().nsx_moe_forward_norm(C.byref(self._c), x.data_ptr(), r.data_ptr(),
                                                  None if w is None else w.data_ptr(), float(eps), T,
                                                  x_out.data_ptr(), out.data_ptr(), ids.data_ptr(),
                                                  weights.data_ptr(), ws.data_ptr(), ws.numel(),
                                                  N.stream_ptr(self.device)), "moe_forward_norm")
        return out, ids, weights

    def forward_addnorm(self, h: torch.Tensor, x: torch.Tensor, norm_w: torch.Tensor | None, eps: float,
                        x_out: torch.Tensor, h_out: torch.Tensor, ids: torch.Tensor | None = None,
                        weights: torch.Tensor | None = None):
        """One stacked block whose output feeds the next (model/gpt_oss.py:123-177):
        x_out = x + forward(h) and h_out = rms_norm(x_out) * norm_w, the next
        block's input -- the bits of forward + add_rms_norm; on the grouped path the
        combine, the add and the norm are one launch (the MoE output is not kept).
        h, x, x_out, h_out: (T, n_embd) contiguous fp32; x_out may be x, h_out may be
        h but must not overlap x or x_out. Returns (ids, weights)."""
        N.require_device(h, x, x_out, h_out)
        T = x.shape[0]
        for name, t in (("h", h), ("x", x), ("x_out", x_out), ("h_out", h_out)):
            if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != (T, self.n_embd) \
                    or t.device != self.device:
                raise ValueError(f"{name} must be a contiguous fp32 ({T}, {self.n_embd}) tensor on {self.device}")
        if ids is None:
            ids = torch.empty((T, self.top_k), dtype=torch.int32, device=self.device)
        if weights is None:
            weights = torch.empty((T, self.top_k), dtype=torch.float32, device=self.device)
        self._check_buffers(T, h_out, ids, weights)
        w = None
        if norm_w is not None:
            w = norm_w.to(device=self.device, dtype=torch.float32).contiguous()
            if w.numel() != self.n_embd:
                raise ValueError(f"norm weight of {w.numel()} values, n_embd is {self.n_embd}")
        ws = self.workspace(T)
        with torch.cuda.device(self.device):
            N.check(N.load().nsx_moe_forward_addnorm(C.byref(self._c), h.data_ptr(), T, x.data_ptr(),
                                                     None if w is None else w.data_ptr(), float(eps),
                                                     x_out.data_ptr(), h_out.data_ptr(), ids.data_ptr(),
                                                     weights.data_ptr(), ws.data_ptr(), ws.numel(),
                                                     N.stream_ptr(self.device)), "moe_forward_addnorm")
        return ids, weights

    def chain_share_bytes(self) -> int:
        """Bytes of a router-share buffer for chain_t1, or -1 when this layer
        cannot run in the decode chain (t64 on the per-pair kernels, n_embd a
        multiple of 16 up to 3072, a multiple of 4 experts up to 128)."""
        return int(N.load().nsx_moe_chain_share_bytes(C.byref(self._c)))

    def chain_t1(self, x: torch.Tensor, norm_w: torch.Tensor | None, eps: float, share_in: torch.Tensor | None,
                 next_layer: "MoELayer | None", next_norm_w: torch.Tensor | None, share_out: torch.Tensor | None,
                 out: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, phases: int = 3) -> None:
        """One stacked block of a decode chain (T = 1; model/gpt_oss.py:123-177):
        x += forward(rms_norm(x) * norm_w) in place, out/ids/weights as forward.
        share_in None: the block routes from x (norm, router, gate/up launches);
        else it holds this block's router shares, written by the previous
        block's call, and no router launch runs. With next_layer the down kernel
        also writes that block's shares to share_out (may be share_in). x, out:
        (1, n_embd) contiguous fp32; share buffers: uint8 or fp32 device tensors
        of chain_share_bytes() (nsx_moe_chain_t1). phases: N.CHAIN_GATE_UP,
        N.CHAIN_DOWN or both (one launch alone reads what the other left, for
        timing)."""
        N.require_device(x, out)
        for name, t in (("x", x), ("out", out)):
            if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != self.n_embd or t.device != self.device:
                raise ValueError(f"{name} must be a contiguous fp32 tensor of {self.n_embd} values on {self.device}")
        self._check_buffers(1, out.view(1, -1), ids, weights)

        def vec(w):
            if w is None:
                return None
            w = w.to(device=self.device, dtype=torch.float32).contiguous()
            if w.numel() != self.n_embd:
                raise ValueError(f"norm weight of {w.numel()} values, n_embd is {self.n_embd}")
            return w

        def share(buf, layer):
            if buf is None:
                return None
            need = layer.chain_share_bytes()
            if need < 0:
                raise NotImplementedError("this layer does not run in the decode chain")
            if buf.device != self.device or not buf.is_contiguous() or buf.numel() * buf.element_size() < need:
                raise ValueError(f"share buffer must be a contiguous device tensor of >= {need} bytes")
            return buf

        w, nw = vec(norm_w), vec(next_norm_w)
        si = share(share_in, self)
        so = share(share_out, next_layer) if next_layer is not None else None
        if next_layer is not None and so is None:
            raise ValueError("a next layer needs share_out")
        ws = self.workspace(1)
        ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        with torch.cuda.device(self.device):
            N.check(N.load().nsx_moe_chain_t1(C.byref(self._c), x.data_ptr(), ptr(w), float(eps), ptr(si),
                                              None if next_layer is None else C.byref(next_layer._c), ptr(nw),
                                              ptr(so), out.data_ptr(), ids.data_ptr(), weights.data_ptr(),
                                              ws.data_ptr(), ws.numel(), int(phases), N.stream_ptr(self.device)),
                    "moe_chain_t1")

    def phase(self, phase: int, h: torch.Tensor, out: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
              workspace: torch.Tensor | None = None) -> None:
        """Run one phase (_native.PHASE_*) of forward(); later phases read what
        earlier ones left in `workspace` (default: this layer's for h's T)."""
        N.require_device(h, out, ids, weights)
        h = h.reshape(-1, self.n_embd)
        if h.dtype != torch.float32 or not h.is_contiguous():
            raise TypeError("phase() takes a contiguous fp32 h")
        T = h.shape[0]
        self._check_buffers(T, out, ids, weights)
        ws = self.workspace(T) if workspace is None else workspace
        need = N.load().nsx_moe_workspace_bytes(C.byref(self._c), T)
        if ws.device != self.device or ws.dtype != torch.uint8 or not ws.is_contiguous() or ws.numel() < need:
            raise ValueError(f"workspace must be a contiguous uint8 tensor of >= {need} bytes on {self.device}")
        with torch.cuda.device(self.device):
            N.check(N.load().nsx_moe_phase(C.byref(self._c), int(phase), h.data_ptr(), T, out.data_ptr(),
                                           ids.data_ptr(), weights.data_ptr(), ws.data_ptr(), ws.numel(),
                                           N.stream_ptr(self.device)), f"moe_phase {phase}")

    def new_workspace(self, T: int) -> torch.Tensor:
        """A separate zeroed workspace for T tokens (for phase runs that overlap)."""
        n = N.load().nsx_moe_workspace_bytes(C.byref(self._c), T)
        if n < 0:
            raise ValueError(f"bad layer for T={T}")
        return torch.zeros(max(n, 256), dtype=torch.uint8, device=self.device)


def router_topk(h: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, top_k: int,
                mode: str = "gptoss"):
    """Fused router on the device: (ids int32 (T,k), weights fp32 (T,k), logits fp32 (T,E))."""
    N.require_device(h, w)
    h = h.reshape(-1, w.shape[-1]).float().contiguous()
    w = w.contiguous()
    T, E = h.shape[0], w.shape[0]
    dev = h.device
    ids = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    wts = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    lib = N.load()
    b = None if bias is None else bias.float().contiguous()
    with torch.cuda.device(dev):
        N.check(lib.nsx_router_topk(h.data_ptr(), T, h.shape[1], w.data_ptr(), _W_CODE[w.dtype],
                                    None if b is None else b.data_ptr(), E, top_k,
                                    N.ROUTE_GPTOSS if mode == "gptoss" else N.ROUTE_QWEN3,
                                    ids.data_ptr(), wts.data_ptr(), logits.data_ptr(), N.stream_ptr(dev)),
                "router_topk")
    return ids, wts, logits
