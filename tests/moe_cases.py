"""Shared MoE layer builders for the GPU tests: synthetic layers as MoELayer
objects and their oracle results (not a test module)."""
from __future__ import annotations

import torch

from oracle import moe as OM


def _expert_set(cfg, t):
    """oracle.ExpertSet over raw tensors of a synthetic layer (CPU copies)."""
    raw = {k: t[k].cpu().numpy() for k in ("gate", "up", "down")}
    bias = {k: t[k + "_b"].cpu().numpy() for k in ("gate", "up", "down")} if cfg.bias else {}
    return OM.ExpertSet(int(cfg.ggml_type), cfg.n_embd, cfg.n_ff, raw, bias)


def _layer(cfg, t, layout, slabs=False, dispatch="auto"):
    """MoELayer over stacked tensors, or (slabs=True) one tensor per expert."""
    from nurostream_amd.compute.kernels import t64_pack, t64_pack_stacked
    from nurostream_amd.moe.fused import MoELayer
    mats = {}
    for kind in ("gate", "up", "down"):
        rows, K = cfg.rows_K(kind)
        per = cfg.expert_bytes(kind)
        if layout == "t64" and slabs:
            mats[kind] = [t64_pack(t[kind][e * per:(e + 1) * per], cfg.ggml_type, rows, K)
                          for e in range(cfg.n_expert)]
        elif layout == "t64":
            mats[kind] = t64_pack_stacked(t[kind], cfg.ggml_type, cfg.n_expert, rows, K)
        elif slabs:
            mats[kind] = [t[kind][e * per:(e + 1) * per].clone() for e in range(cfg.n_expert)]
        else:
            mats[kind] = t[kind]
    return MoELayer(ggml_type=cfg.ggml_type, n_expert=cfg.n_expert, top_k=cfg.top_k, n_embd=cfg.n_embd,
                    n_ff=cfg.n_ff, router_w=t["router_w"], router_b=t["router_b"], gate=mats["gate"],
                    up=mats["up"], down=mats["down"], gate_b=t["gate_b"], up_b=t["up_b"], down_b=t["down_b"],
                    layout=layout, router_mode=cfg.router_mode, act=cfg.act, dispatch=dispatch)


def _oracle_layer(cfg, t, h, ex=None):
    """(out, ids, weights, logits) of the reference path for a synthetic layer."""
    ex = _expert_set(cfg, t) if ex is None else ex
    Wr = t["router_w"].float().cpu().numpy()
    if cfg.router_mode == "gptoss":
        ids, w, logits = OM.route_gptoss(h, Wr, t["router_b"].cpu().numpy(), cfg.top_k)
    else:
        ids, w, logits = OM.route_qwen3(h, Wr, cfg.top_k)
    act = OM.clamped_swiglu if cfg.act == "clamped_swiglu" else OM.silu_mul
    return OM.combine(h, ids, w, ex, act), ids, w, logits


def _small(name):
    from nurostream_amd import synth
    if name == "gptoss-small":
        return synth.MoEConfig("gptoss-small", synth.GGMLType.MXFP4, 16, 4, 256, 192, "gptoss", "clamped_swiglu",
                               True, torch.bfloat16)
    if name == "qwen3-small":
        return synth.MoEConfig("qwen3-small", synth.GGMLType.Q4_K, 12, 8, 512, 256, "qwen3", "silu_mul", False,
                               torch.float32)
    if name == "qwen3b-small":  # Q4_K with expert biases (a GGUF of a biased model, as GPT-OSS in Q4_K)
        return synth.MoEConfig("qwen3b-small", synth.GGMLType.Q4_K, 12, 8, 512, 256, "qwen3", "silu_mul", True,
                               torch.float32)
    if name == "q4_0-small":
        return synth.MoEConfig("q40-small", synth.GGMLType.Q4_0, 8, 2, 128, 96, "gptoss", "silu_mul", True,
                               torch.float32)
    if name == "q8_0-small":  # 170- and 102-byte rows: rows and 34-byte units at 2-byte offsets
        return synth.MoEConfig("q80-small", synth.GGMLType.Q8_0, 8, 3, 160, 96, "qwen3", "silu_mul", False,
                               torch.float32)
    raise KeyError(name)
