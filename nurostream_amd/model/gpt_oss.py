"""GPT-OSS MoE FFN stack on one MI355X (model/gpt_oss.py:61-177 of the reference).

`GptOssFFNStack` holds one MoELayer per layer (VRAM-resident expert slabs)
and chains them the way the reference's decoder wraps its FFN blocks:
h = rms_norm(x, post_attention_norm) (compute/ops.py:14-20), out = moe(h),
x = x + out (gpt_oss.py:126,177). Attention is not on the MoE path and is
not modelled: layer l + 1 reads layer l's output directly.

`forward` runs the whole chain on the device with no host synchronisation:
per layer one fused residual-add + norm kernel (nsx_add_rmsnorm) and one
MoE layer call (nsx_moe_forward, device-side routing). `_route` and
`_ffn_block` keep the reference's per-layer signatures; `_route` returns the
chosen experts as a host list (a device-to-host copy, as the reference's
torch.unique(...).tolist() at gpt_oss.py:121).
"""
from __future__ import annotations

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
        layer's FFN block (into `out` when given). Device-only: no host sync."""
        x = x.reshape(-1, self.cfg.n_embd)
        T = x.shape[0]
        h, y, ids, wts = self._buffers(T)
        res = torch.empty_like(x) if out is None else out
        eps = self.cfg.rms_eps
        add_rms_norm(x.float().contiguous(), None, self.norm_weights[0], eps, out=h, sum_out=res)
        for li, layer in enumerate(self.layers):
            layer.forward(h, out=y, ids=ids[li], weights=wts[li])
            if li + 1 < len(self.layers):  # x += out; h = rms_norm(x) of the next layer
                add_rms_norm(res, y, self.norm_weights[li + 1], eps, out=h, sum_out=res)
            else:
                res.add_(y)
        return res

    __call__ = forward

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
