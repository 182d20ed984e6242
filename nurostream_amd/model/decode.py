"""The step either side of the MoE FFN of a GPT-OSS decode token, on the GPU.

Python seams over libnsx (model/gpt_oss.py of the reference):
- `AttnConfig`: the attention / rope keys of a GPT-OSS GGUF (the
  GptOssConfig / Qwen3Config from_gguf keys, model/gpt_oss.py:22-38,
  model/qwen3.py:56-76).
- `yarn_inv_freq`: the inverse frequencies and amplitude of yarn_tables
  (gpt_oss.py:42-58), in torch fp32 as the reference computes them. The
  kernels then take cos/sin of pos * inv_freq on the device.
- `DeviceKV`: KVCache (model/qwen3.py:79-106) with a fixed capacity in HBM
  and the token position in device memory, so one decode token can be
  captured as a graph and replayed.
- `rope_kv_append`, `attn_decode`, `dequantize_rows`: the kernels;
  `attn_decode_qkv` does the first two in one launch.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .. import _native as N
from ..format.gguf import FLOAT_TYPES, GGMLType


@dataclass
class AttnConfig:
    n_head: int
    n_head_kv: int
    head_dim: int
    vocab_size: int
    rope_base: float
    context_length: int
    sliding_window: int = 128
    rope_factor: float = 32.0
    original_context: int = 4096
    beta_fast: float = 32.0
    beta_slow: float = 1.0

    @property
    def n_rep(self) -> int:
        return self.n_head // self.n_head_kv

    @classmethod
    def from_gguf(cls, g) -> "AttnConfig":
        n_embd = int(g.cfg("embedding_length"))
        n_head = int(g.cfg("attention.head_count"))
        return cls(n_head=n_head, n_head_kv=int(g.cfg("attention.head_count_kv", n_head)),
                   head_dim=int(g.cfg("attention.key_length", n_embd // n_head)),
                   vocab_size=g.tensors["token_embd.weight"].torch_shape[0],
                   rope_base=float(g.cfg("rope.freq_base", 10000.0)),
                   context_length=int(g.cfg("context_length", 4096)),
                   sliding_window=int(g.cfg("attention.sliding_window", 128)),
                   rope_factor=float(g.cfg("rope.scaling.factor", 32.0)),
                   original_context=int(g.cfg("rope.scaling.original_context_length", 4096)),
                   beta_fast=float(g.cfg("rope.scaling.yarn_beta_fast", 32.0)),
                   beta_slow=float(g.cfg("rope.scaling.yarn_beta_slow", 1.0)))


def yarn_inv_freq(cfg: AttnConfig, device) -> tuple[torch.Tensor, float]:
    """(inverse frequencies (head_dim/2,) fp32 on `device`, amplitude) -- gpt_oss.py:42-58."""
    half = cfg.head_dim // 2
    dims = torch.arange(half, dtype=torch.float32)
    inv = 1.0 / cfg.rope_base ** (dims / half)
    factor = cfg.rope_factor
    if factor != 1:
        def correction(rotations):
            return cfg.head_dim * math.log(cfg.original_context / (rotations * 2 * math.pi)) / (2 * math.log(cfg.rope_base))
        low = max(correction(cfg.beta_fast), 0)  # the untruncated (non-integer) range of GPT-OSS
        high = min(correction(cfg.beta_slow), cfg.head_dim - 1)
        ramp = ((dims - low) / (high - low if high != low else 0.001)).clamp(0, 1)
        inv = inv * (1 - ramp) + inv / factor * ramp
    amplitude = 1 + 0.1 * math.log(factor) if factor > 1 else 1.0
    return inv.to(device), float(amplitude)


class DeviceKV:
    """Per-layer K/V history in HBM, [n_kv][ctx_max][head_dim] fp32 each, and
    the next token's position as a device int32 (`pos`) with a host mirror
    (`length`)."""

    def __init__(self, n_layer: int, cfg: AttnConfig, ctx_max: int, device) -> None:
        if ctx_max < 1:
            raise ValueError("ctx_max must be positive")
        self.device = torch.device(device)
        self.ctx_max = int(ctx_max)
        shape = (cfg.n_head_kv, self.ctx_max, cfg.head_dim)
        self.k = [torch.zeros(shape, dtype=torch.float32, device=self.device) for _ in range(n_layer)]
        self.v = [torch.zeros(shape, dtype=torch.float32, device=self.device) for _ in range(n_layer)]
        self.pos = torch.zeros(1, dtype=torch.int32, device=self.device)
        nb = N.load().nsx_attn_workspace_bytes(cfg.n_head, cfg.head_dim, self.ctx_max)
        if nb < 0:
            raise NotImplementedError(f"attention kernels need head_dim 64 (got {cfg.head_dim})")
        self.workspace = torch.empty(nb, dtype=torch.uint8, device=self.device)
        self.length = 0

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (*self.k, *self.v))

    def reset(self) -> None:
        self.pos.zero_()
        self.length = 0


def rope_kv_append(qkv: torch.Tensor, bq, bk, bv, cfg: AttnConfig, inv_freq: torch.Tensor, amp: float,
                   kv: DeviceKV, layer: int) -> None:
    """Bias, rotary on the q and k rows (q in place), k and v into the cache at kv.pos."""
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    N.check(N.load().nsx_rope_kv_append(qkv.data_ptr(), ptr(bq), ptr(bk), ptr(bv), cfg.n_head, cfg.n_head_kv,
                                        cfg.head_dim, inv_freq.data_ptr(), float(amp), kv.pos.data_ptr(),
                                        kv.k[layer].data_ptr(), kv.v[layer].data_ptr(), kv.ctx_max,
                                        N.stream_ptr(qkv.device)), "rope_kv_append")


def attn_decode(q: torch.Tensor, kv: DeviceKV, layer: int, sinks: torch.Tensor | None, window: int,
                cfg: AttnConfig, out: torch.Tensor | None = None) -> torch.Tensor:
    """Sink attention of the token at kv.pos over the layer's cache -> (n_head, head_dim)."""
    y = torch.empty((cfg.n_head, cfg.head_dim), dtype=torch.float32, device=q.device) if out is None else out
    N.check(N.load().nsx_attn_decode(q.data_ptr(), kv.k[layer].data_ptr(), kv.v[layer].data_ptr(),
                                     None if sinks is None else sinks.data_ptr(), cfg.n_head, cfg.n_head_kv,
                                     cfg.head_dim, kv.pos.data_ptr(), kv.ctx_max, int(window),
                                     1.0 / math.sqrt(cfg.head_dim), kv.workspace.data_ptr(), y.data_ptr(),
                                     N.stream_ptr(q.device)), "attn_decode")
    return y


def attn_decode_qkv(qkv: torch.Tensor, bq, bk, bv, cfg: AttnConfig, inv_freq: torch.Tensor, amp: float,
                    kv: DeviceKV, layer: int, sinks: torch.Tensor | None, window: int,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """rope_kv_append + attn_decode as one launch (two with the chunk combine); qkv (the raw
    projection, no bias) is left unchanged. Bit-identical to the two calls."""
    y = torch.empty((cfg.n_head, cfg.head_dim), dtype=torch.float32, device=qkv.device) if out is None else out
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    N.check(N.load().nsx_attn_decode_qkv(qkv.data_ptr(), ptr(bq), ptr(bk), ptr(bv), inv_freq.data_ptr(), float(amp),
                                         ptr(sinks), cfg.n_head, cfg.n_head_kv, cfg.head_dim, kv.pos.data_ptr(),
                                         kv.k[layer].data_ptr(), kv.v[layer].data_ptr(), kv.ctx_max, int(window),
                                         1.0 / math.sqrt(cfg.head_dim), kv.workspace.data_ptr(), y.data_ptr(),
                                         N.stream_ptr(qkv.device)), "attn_decode_qkv")
    return y


def advance(kv: DeviceKV, n: int = 1) -> None:
    N.check(N.load().nsx_pos_advance(kv.pos.data_ptr(), int(n), N.stream_ptr(kv.pos.device)), "pos_advance")
    kv.length += n


def dequantize_rows(raw: torch.Tensor, dtype, n_rows: int, K: int, ids: torch.Tensor,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 rows ids (device int32) of an (n_rows, K) GGUF matrix (gather_embeddings, blockffn.py:470-487)."""
    N.require_device(raw, ids)
    if ids.dtype != torch.int32:
        raise TypeError("ids must be int32")
    y = torch.empty((ids.numel(), K), dtype=torch.float32, device=raw.device) if out is None else out
    N.check(N.load().nsx_dequantize_rows(int(GGMLType(dtype)), raw.data_ptr(), n_rows, K, ids.data_ptr(),
                                         ids.numel(), y.data_ptr(), N.stream_ptr(raw.device)), "dequantize_rows")
    return y


__all__ = ["AttnConfig", "DeviceKV", "yarn_inv_freq", "rope_kv_append", "attn_decode", "attn_decode_qkv", "advance",
           "dequantize_rows", "FLOAT_TYPES"]
