"""A tiny GPT-OSS GGUF written with this build's GGUFWriter (not a test module)."""
from __future__ import annotations

import numpy as np
import torch


def write_gptoss_gguf(path, cfg, n_layers: int, seed: int):
    """Write n_layers MoE FFN blocks of `cfg` (synth.make_layer tensors) plus a
    post-attention norm weight per layer; returns {layer: tensors} (CPU)."""
    from nurostream_amd import synth
    from nurostream_amd.format.gguf import GGMLType, GGUFWriter
    wr = GGUFWriter(path, "gpt-oss")
    wr.add("gpt-oss.block_count", n_layers)
    wr.add("gpt-oss.embedding_length", cfg.n_embd)
    wr.add("gpt-oss.expert_count", cfg.n_expert)
    wr.add("gpt-oss.expert_used_count", cfg.top_k)
    wr.add("gpt-oss.expert_feed_forward_length", cfg.n_ff)
    wr.add("gpt-oss.attention.layer_norm_rms_epsilon", 1e-5)
    layers = {}
    for li in range(n_layers):
        t = synth.make_layer(cfg, seed=seed, device="cpu", layer=li)
        g = torch.Generator().manual_seed(seed * 31 + li)
        t["norm"] = torch.rand(cfg.n_embd, generator=g) + 0.5
        p = f"blk.{li}."
        wr.add_tensor(p + "ffn_gate_inp.weight", (cfg.n_expert, cfg.n_embd), GGMLType.BF16,
                      t["router_w"].contiguous().view(torch.uint8).numpy().tobytes())
        wr.add_tensor(p + "ffn_gate_inp.bias", (cfg.n_expert,), GGMLType.F32, t["router_b"].numpy().tobytes())
        for kind in ("gate", "up", "down"):
            rows, K = cfg.rows_K(kind)
            wr.add_tensor(p + f"ffn_{kind}_exps.weight", (cfg.n_expert, rows, K), cfg.ggml_type,
                          t[kind].numpy().tobytes())
            wr.add_tensor(p + f"ffn_{kind}_exps.bias", (cfg.n_expert, rows), GGMLType.F32,
                          t[kind + "_b"].numpy().astype(np.float32).tobytes())
        wr.add_tensor(p + "post_attention_norm.weight", (cfg.n_embd,), GGMLType.F32, t["norm"].numpy().tobytes())
        layers[li] = t
    wr.write()
    return layers


def oracle_stack(cfg, layers, x, eps=1e-5):
    """x after each layer's FFN block (oracle.moe restatement)."""
    from oracle import moe as OM
    x = np.asarray(x, np.float32)
    for li in sorted(layers):
        t = layers[li]
        ex = OM.ExpertSet(int(cfg.ggml_type), cfg.n_embd, cfg.n_ff, {k: t[k].numpy() for k in ("gate", "up", "down")},
                          {k: t[k + "_b"].numpy() for k in ("gate", "up", "down")})
        h = OM.rms_norm(x, t["norm"].numpy(), eps)
        out = OM.moe_gptoss(h, t["router_w"].float().numpy(), t["router_b"].numpy(), cfg.top_k, ex)[0]
        x = (x + out).astype(np.float32)
    return x
