"""A tiny GPT-OSS GGUF written with this build's GGUFWriter (not a test module)."""
from __future__ import annotations

import numpy as np
import torch


# attention geometry of the tiny model: 8 query heads, 2 kv heads of 64, vocab 300
ATTN = dict(n_head=8, n_head_kv=2, head_dim=64, vocab=300, rope_base=150000.0, context=4096, window=4,
            rope_factor=32.0, original_context=4096, beta_fast=32.0, beta_slow=1.0)


def _q8(rows, K, g):
    from nurostream_amd import synth
    from nurostream_amd.format.gguf import GGMLType
    return synth.matrix_bytes(GGMLType.Q8_0, rows, K, g, "cpu", d_std=0.02)


def write_gptoss_gguf(path, cfg, n_layers: int, seed: int, attention: bool = False):
    """Write n_layers MoE FFN blocks of `cfg` (synth.make_layer tensors) plus a
    post-attention norm weight per layer; returns {layer: tensors} (CPU).

    attention=True adds what a decode token needs around the FFN (the
    reference's GPT-OSS tensor names): token_embd / output (Q8_0),
    output_norm, and per layer attn_norm, attn_q/k/v/output (Q8_0) with
    biases, attn_sinks, plus the attention and rope metadata (ATTN); those
    tensors come back under layers["model"]."""
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
    if attention:
        a = ATTN
        wr.add("gpt-oss.attention.head_count", a["n_head"])
        wr.add("gpt-oss.attention.head_count_kv", a["n_head_kv"])
        wr.add("gpt-oss.attention.key_length", a["head_dim"])
        wr.add("gpt-oss.rope.freq_base", a["rope_base"])
        wr.add("gpt-oss.context_length", a["context"])
        wr.add("gpt-oss.attention.sliding_window", a["window"])
        wr.add("gpt-oss.rope.scaling.factor", a["rope_factor"])
        wr.add("gpt-oss.rope.scaling.original_context_length", a["original_context"])
        wr.add("gpt-oss.rope.scaling.yarn_beta_fast", a["beta_fast"])
        wr.add("gpt-oss.rope.scaling.yarn_beta_slow", a["beta_slow"])
        g = torch.Generator().manual_seed(seed * 7 + 3)
        nq, nkv = a["n_head"] * a["head_dim"], a["n_head_kv"] * a["head_dim"]
        m = {"token_embd.weight": _q8(a["vocab"], cfg.n_embd, g), "output.weight": _q8(a["vocab"], cfg.n_embd, g),
             "output_norm.weight": torch.rand(cfg.n_embd, generator=g) + 0.5}
        for li in range(n_layers):
            p = f"blk.{li}."
            m[p + "attn_norm.weight"] = torch.rand(cfg.n_embd, generator=g) + 0.5
            for nm, rows, K in (("attn_q", nq, cfg.n_embd), ("attn_k", nkv, cfg.n_embd), ("attn_v", nkv, cfg.n_embd),
                                ("attn_output", cfg.n_embd, nq)):
                m[p + nm + ".weight"] = _q8(rows, K, g)
                m[p + nm + ".bias"] = torch.randn(rows, generator=g) * 0.1
            m[p + "attn_sinks.weight"] = torch.randn(a["n_head"], generator=g)
        for name, tnsr in m.items():
            if tnsr.dtype == torch.uint8:
                rows = a["vocab"] if name in ("token_embd.weight", "output.weight") else None
                if rows is None:
                    nm = name.split(".")[2]
                    rows = {"attn_q": nq, "attn_k": nkv, "attn_v": nkv, "attn_output": cfg.n_embd}[nm]
                K = len(tnsr) // rows // 34 * 32
                wr.add_tensor(name, (rows, K), GGMLType.Q8_0, tnsr.numpy().tobytes())
            else:
                wr.add_tensor(name, tuple(tnsr.shape), GGMLType.F32, tnsr.float().numpy().tobytes())
        layers["model"] = m
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
