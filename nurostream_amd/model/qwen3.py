"""The MoE FFN side of a Qwen3 model over a weight cache (model/qwen3.py of the reference).

`Qwen3MoE` supplies exactly what moe.router.moe_ffn reads from its `model`
argument (cfg, w, cache, gguf, device, dtype, has, _linear -- the attributes
the reference's Qwen3Model carries, model/qwen3.py:169-194), so the
reference's sparse-FFN loop runs unchanged on the HIP kernels: routing on
the device, expert products on the fused GEMV or t64 slabs, non-resident
experts streamed through the cache's source.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from ..compute.blockffn import DEFAULT_BLOCK_ROWS, stream_linear
from ..moe.router import RouterStats, moe_ffn


@dataclass
class Qwen3MoEConfig:
    n_embd: int
    n_expert: int
    n_expert_used: int
    n_ffn_expert: int
    rms_eps: float = 1e-6


class Qwen3MoE:
    def __init__(self, cache, cfg: Qwen3MoEConfig, device, dtype=torch.float32,
                 block_rows: int = DEFAULT_BLOCK_ROWS) -> None:
        self.cache = cache
        self.gguf = cache.gguf
        self.cfg = cfg
        self.device = torch.device(device)
        self.dtype = dtype
        self.block_rows = block_rows
        self.router_stats = RouterStats()
        self._w: dict[str, torch.Tensor] = {}

    def w(self, name: str) -> torch.Tensor:
        """A float tensor (router, norms) in the compute dtype, kept after first use."""
        t = self._w.get(name)
        if t is None:
            t = self.cache.get(name).to(self.device, self.dtype)
            self._w[name] = t
        return t

    def has(self, name: str) -> bool:
        return name in self.gguf.tensors

    def _linear(self, name: str, x: torch.Tensor) -> torch.Tensor:
        """x @ W.T through the streaming seam (model/qwen3.py:169-194)."""
        return stream_linear(self.cache, name, x, block_rows=self.block_rows, device=self.device, dtype=self.dtype)

    def ffn(self, h: torch.Tensor, layer: int) -> torch.Tensor:
        return moe_ffn(self, h, layer)
