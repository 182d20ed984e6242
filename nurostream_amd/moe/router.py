"""Qwen3-style sparse MoE FFN over a weight cache (moe/router.py:1-219 of the reference).

The reference's seams, same names and contracts:
  * `RouterStats` (moe/router.py:26-56): tokens routed, expert reads, per
    (layer, expert) hits, `top_experts`, `skew`, `summary`; `record(layer,
    ids)` is the one addition (hit counting from a device id tensor, used by
    the fused layer whose routing never leaves the device).
  * `route(model, h, layer)` (:59-69): softmax over all experts in fp32,
    top-k, renormalise -- here one HIP kernel (nsx_router_topk, mode qwen3).
  * `submit_expert_reads` (:81-109): queue every non-resident slab of the
    chosen experts at once; stop quietly when the arena is full.
  * `_expert_matmul` (:112-170): x @ W_e.T through a pending read, a cache
    hit (raw bytes or a t64 slab) or the cache's dequantizing fetch; quantized
    products run on the fused HIP GEMV (T <= 16) or dequantize on the device.
  * `moe_ffn` (:173-219): route, read only the chosen experts, silu(gate)*up,
    down, out[rows] += w_e * y_e in ascending expert id.

`model` is duck-typed as in the reference: cfg (n_expert_used, n_ffn_expert,
n_embd), w(name), cache, gguf, device, dtype, has(name), _linear(name, x).
"""
from __future__ import annotations

import heapq
from collections import Counter
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from ..compute import kernels as tk
from ..compute.quant import dequantize
from ..io.arena import BudgetExceeded


@dataclass
class RouterStats:
    """Routing counters (the fields of moe/router.py:26-56): tokens routed,
    expert reads (one per distinct expert a forward touched), and per
    (layer, expert) hit counts -- what pin_hot_experts ranks experts by."""
    tokens_routed: int = 0
    expert_reads: int = 0
    hits: Counter = field(default_factory=Counter)

    def top_experts(self, layer: int, k: int = 8) -> list[tuple[int, int]]:
        """Up to k (expert, hits) of `layer`, most hits first (ties: lower expert id)."""
        mine = [(c, e) for (lay, e), c in self.hits.items() if lay == layer]
        return [(e, c) for c, e in heapq.nsmallest(k, mine, key=lambda ce: (-ce[0], ce[1]))]

    def skew(self) -> float:
        """How concentrated routing is: the share of all hits that land on the
        most-hit fifth of the (layer, expert) entries seen (at least one)."""
        n = len(self.hits)
        if n == 0:
            return 0.0
        busiest = heapq.nlargest(max(1, n // 5), self.hits.values())
        return sum(busiest) / sum(self.hits.values())

    def summary(self) -> str:
        return (f"router: {self.tokens_routed} tokens, {self.expert_reads} expert reads, "
                f"{len(self.hits)} (layer, expert) pairs used, busiest fifth takes {100 * self.skew():.1f}%")

    def record(self, layer: int, ids: torch.Tensor) -> None:
        """Count one forward's routing: ids (T, k) of `layer` (device or host)."""
        flat = ids.reshape(ids.shape[0], -1).cpu()
        self.tokens_routed += flat.shape[0]
        # hits per expert = tokens routing to it (an expert appears once per token)
        uniq, counts = torch.unique(flat, return_counts=True)
        for e, c in zip(uniq.tolist(), counts.tolist()):
            self.hits[(layer, e)] += c
        self.expert_reads += len(uniq)


def route(model, h: torch.Tensor, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(expert ids int64 (T, k), weights (T, k) in h.dtype): moe/router.py:59-69."""
    from .fused import router_topk
    W = model.w(f"blk.{layer}.ffn_gate_inp.weight")
    ids, wts, _ = router_topk(h, W, None, model.cfg.n_expert_used, "qwen3")
    return ids.long(), wts.to(h.dtype)


def _expert_slabs(cfg):
    """(tensor suffix, rows per expert) of the three expert matrices."""
    return (("ffn_gate_exps.weight", cfg.n_ffn_expert), ("ffn_up_exps.weight", cfg.n_ffn_expert),
            ("ffn_down_exps.weight", cfg.n_embd))


def submit_expert_reads(model, layer: int, experts) -> dict:
    """Queue a read of every chosen expert matrix the cache does not hold,
    all at once, without waiting for the arena (moe/router.py:81-109):
    {(name, lo): (future, nbytes)}. The first read the arena cannot take now
    ends the queueing; _expert_matmul reads the rest when it gets to them."""
    cache = model.cache
    src = getattr(cache, "source", None)
    if src is None or not hasattr(src, "submit_rows"):
        return {}

    def wanted():
        for e in experts:
            for suffix, per in _expert_slabs(model.cfg):
                name = f"blk.{layer}.{suffix}"
                lo, hi = e * per, (e + 1) * per
                if name in model.gguf.tensors and not (cache.is_resident(name) or cache.has_slab(name, lo, hi)):
                    yield name, lo, hi

    pending: dict = {}
    for name, lo, hi in wanted():
        try:
            pending[(name, lo)] = src.submit_rows(name, lo, hi, timeout=0)
        except (BudgetExceeded, TimeoutError):
            break
    return pending


def _product(raw, dt, x: torch.Tensor, rows: int, row_elems: int, out_dtype) -> torch.Tensor:
    """x @ dequant(raw).T: fused GEMV for t64 windows (any T) and for T <= 16,
    else a device dequantize and a matmul (batched prefill, cache.py reuse)."""
    if isinstance(raw, tk.T64Rows) or tk.can_fuse(dt, x):
        return tk.fused_gemv(raw, dt, x, rows, row_elems, out_dtype=out_dtype)
    w = dequantize(raw, dt, rows * row_elems, out_dtype=out_dtype).reshape(rows, row_elems)
    return x.to(out_dtype) @ w.T


def _expert_matmul(model, name: str, expert: int, rows_per_expert: int, x: torch.Tensor,
                   pending: dict | None = None) -> torch.Tensor:
    """x @ W_expert.T (moe/router.py:112-170)."""
    lo, hi = expert * rows_per_expert, (expert + 1) * rows_per_expert
    info = model.gguf.tensors[name]
    row_elems = info.torch_shape[-1]
    entry = pending.pop((name, lo), None) if pending else None
    if entry is not None:
        fut, nbytes = entry
        src = model.cache.source
        reader = src._reader_for(name) if hasattr(src, "_reader_for") else src.reader
        try:
            raw = reader.wait(fut).to(model.device, non_blocking=True)
            return _product(raw, info.dtype, x, rows_per_expert, row_elems, model.dtype)
        finally:
            src.arena.release(nbytes)
    hit = model.cache.raw_rows(name, lo, hi)
    if hit is not None:
        return _product(hit[0], hit[1], x, rows_per_expert, row_elems, model.dtype)
    w = model.cache.fetch_rows(name, lo, hi, device=model.device, dtype=model.dtype)
    return x @ w.T


def moe_ffn(model, h: torch.Tensor, layer: int) -> torch.Tensor:
    """Sparse SwiGLU FFN reading only the chosen experts (moe/router.py:173-219)."""
    cfg = model.cfg
    p = f"blk.{layer}."
    stats: RouterStats = getattr(model, "router_stats", None) or RouterStats()
    model.router_stats = stats
    ids, weights = route(model, h, layer)
    stats.tokens_routed += h.shape[0]
    chosen = torch.unique(ids).tolist()
    pending = submit_expert_reads(model, layer, chosen)
    out = torch.zeros_like(h)
    try:
        for e in chosen:
            mask = ids == e
            rows = mask.any(dim=-1).nonzero(as_tuple=True)[0]
            if rows.numel() == 0:
                continue
            w = (weights * mask).sum(dim=-1)[rows].unsqueeze(-1)
            stats.hits[(layer, e)] += int(rows.numel())
            stats.expert_reads += 1
            x = h[rows]
            gate = _expert_matmul(model, p + "ffn_gate_exps.weight", e, cfg.n_ffn_expert, x, pending)
            up = _expert_matmul(model, p + "ffn_up_exps.weight", e, cfg.n_ffn_expert, x, pending)
            act = F.silu(gate) * up
            out[rows] += w * _expert_matmul(model, p + "ffn_down_exps.weight", e, cfg.n_embd, act, pending)
    finally:  # a failed forward must not strand arena leases
        for fut, nbytes in pending.values():
            fut.cancel()
            model.cache.source.arena.release(nbytes)
    if model.has(p + "ffn_gate_shexp.weight"):  # shared expert (other Qwen MoE generations)
        sg = model._linear(p + "ffn_gate_shexp.weight", h)
        su = model._linear(p + "ffn_up_shexp.weight", h)
        out = out + model._linear(p + "ffn_down_shexp.weight", F.silu(sg) * su)
    return out
