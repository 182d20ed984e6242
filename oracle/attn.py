"""CPU restatement (numpy) of the step either side of the MoE FFN in the
reference's GPT-OSS model: YaRN rotary tables, rotary application, sink
attention with the alternating sliding window, the attention block and the
decode forward (embedding -> layers -> output norm -> LM head).

TEST INFRASTRUCTURE ONLY: tests/, the graft smoke check and bench.py's
cpu_baseline leg import it as the checker. No product code imports it.

Each function restates one reference function (neurostream/...):
  yarn_inv_freq, yarn_tables  model/gpt_oss.py:42-58
  apply_rope                  compute/ops.py:95-104 (rotate_half convention)
  repeat_kv                   compute/ops.py:107-113
  sink_attention              model/gpt_oss.py:73-85
  attention_block             model/gpt_oss.py:101-114
  rms_norm                    compute/ops.py:14-20
  forward_tokens              model/gpt_oss.py:207-228 with the FFN of
                              oracle.moe (model/gpt_oss.py:123-177)

Pinning (tests/test_oracle_attn.py):
  * yarn_inv_freq / yarn_tables: against transformers' GPT-OSS rotary
    embedding (modeling_gpt_oss.GptOssRotaryEmbedding with yarn,
    truncate=False), and factor 1 reducing to plain RoPE (base^(-2i/d));
  * apply_rope: against transformers' _apply_rotary_emb, norm preservation,
    and position 0 as the identity;
  * sink_attention: against transformers' eager_attention_forward (sinks,
    causal and sliding masks), a sink of -inf reducing to torch's
    scaled_dot_product_attention, and the one-key closed form
    out = v / (1 + exp(sink - s));
  * attention_block / forward_tokens: compositions of the above with the
    pinned rms_norm (oracle.moe) and expert FFN.
"""
from __future__ import annotations

import math

import numpy as np

from . import moe as OM
from . import quant as OQ


def yarn_inv_freq(head_dim: int, base: float, factor: float, original_context: int, beta_fast: float,
                  beta_slow: float) -> tuple[np.ndarray, float]:
    """(inverse frequencies (head_dim/2,) float32, cos/sin amplitude) (gpt_oss.py:42-58)."""
    half = head_dim // 2
    dims = np.arange(half, dtype=np.float32)
    inv = (1.0 / np.power(np.float32(base), dims / np.float32(half))).astype(np.float32)
    if factor != 1:
        def correction(rotations):
            return head_dim * math.log(original_context / (rotations * 2 * math.pi)) / (2 * math.log(base))
        low = max(correction(beta_fast), 0)  # untruncated (non-integer) range
        high = min(correction(beta_slow), head_dim - 1)
        ramp = np.clip((dims - np.float32(low)) / np.float32(high - low if high != low else 0.001), 0, 1)
        inv = (inv * (1 - ramp) + inv / np.float32(factor) * ramp).astype(np.float32)
    amplitude = 1 + 0.1 * math.log(factor) if factor > 1 else 1.0
    return inv, amplitude


def yarn_tables(head_dim, base, factor, original_context, beta_fast, beta_slow, positions):
    """cos, sin of shape (T, head_dim), the half table repeated (gpt_oss.py:42-58)."""
    inv, amp = yarn_inv_freq(head_dim, base, factor, original_context, beta_fast, beta_slow)
    freqs = np.asarray(positions, dtype=np.float32)[:, None] * inv[None, :]
    freqs = np.concatenate([freqs, freqs], axis=-1)
    return (np.cos(freqs) * np.float32(amp)).astype(np.float32), (np.sin(freqs) * np.float32(amp)).astype(np.float32)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x (H, T, D) * cos + rotate_half(x) * sin, rotate_half = cat(-x2, x1) (ops.py:95-104)."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * cos[None] + rot * sin[None]


def repeat_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    """(H_kv, T, D) -> (H_kv * n_rep, T, D), each kv head repeated n_rep times in a row (ops.py:107-113)."""
    return x if n_rep == 1 else np.repeat(x, n_rep, axis=0)


def sink_attention(q, k, v, sinks, sliding_window: int = 0, f64: bool = True):
    """Causal attention with one learned softmax sink per query head (gpt_oss.py:73-85).

    q (H, Tq, D) are the last Tq positions of the Tk keys; sinks (H,).
    """
    dt = np.float64 if f64 else np.float32
    q, k, v = (np.asarray(a, dtype=dt) for a in (q, k, v))
    tq, tk = q.shape[1], k.shape[1]
    qp = np.arange(tk - tq, tk)[:, None]
    kp = np.arange(tk)[None, :]
    visible = kp <= qp
    if sliding_window:
        visible &= kp > qp - sliding_window
    scores = q @ np.swapaxes(k, -1, -2) / math.sqrt(q.shape[-1])
    scores = np.where(visible[None], scores, -np.inf)
    sink = np.broadcast_to(np.asarray(sinks, dtype=dt)[:, None, None], (q.shape[0], tq, 1))
    logits = np.concatenate([scores, sink], axis=-1)
    m = logits.max(axis=-1, keepdims=True)
    p = np.exp(logits - m)
    p = p / p.sum(axis=-1, keepdims=True)
    return p[..., :-1] @ v


class AttnWeights:
    """One layer's attention tensors as float arrays (dequantized)."""

    def __init__(self, norm, wq, bq, wk, bk, wv, bv, wo, bo, sinks):
        self.norm, self.wq, self.bq, self.wk, self.bk = norm, wq, bq, wk, bk
        self.wv, self.bv, self.wo, self.bo, self.sinks = wv, bv, wo, bo, sinks


def attention_block(x, A: AttnWeights, cos, sin, kv: dict, layer: int, n_head: int, n_kv: int, head_dim: int,
                    window: int, eps: float):
    """x + o_proj(sink_attention(rope(q), rope(k) ++ cache, v ++ cache)) (gpt_oss.py:101-114).

    `kv` maps layer -> (K (H_kv, T, D), V) and grows like KVCache.append.
    """
    t = x.shape[0]
    h = OM.rms_norm(x, A.norm, eps)
    q = (h @ A.wq.T + A.bq).reshape(t, n_head, head_dim).transpose(1, 0, 2)
    k = (h @ A.wk.T + A.bk).reshape(t, n_kv, head_dim).transpose(1, 0, 2)
    v = (h @ A.wv.T + A.bv).reshape(t, n_kv, head_dim).transpose(1, 0, 2)
    q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
    if layer in kv:
        k = np.concatenate([kv[layer][0], k], axis=1)
        v = np.concatenate([kv[layer][1], v], axis=1)
    kv[layer] = (k, v)
    n_rep = n_head // n_kv
    out = sink_attention(q, repeat_kv(k, n_rep), repeat_kv(v, n_rep), A.sinks,
                         window if layer % 2 == 0 else 0)
    out = out.transpose(1, 0, 2).reshape(t, n_head * head_dim)
    return x + (out @ A.wo.T + A.bo)


def dequant(raw: np.ndarray, dtype: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    return OQ.dequantize(np.asarray(raw).reshape(-1), dtype, n).reshape(shape).astype(np.float64)


def forward_tokens(tokens, emb, attn: list, experts: list, routers: list, out_norm, lm_head, cfg: dict, kv: dict,
                   start_pos: int):
    """Logits (T, vocab) of tokens at positions start_pos.. (gpt_oss.py:207-228, all positions).

    emb / lm_head (vocab, n_embd) float; attn: AttnWeights per layer;
    experts: oracle.moe.ExpertSet per layer; routers: (W, b) per layer.
    """
    c = cfg
    x = emb[np.asarray(tokens)].astype(np.float64)
    pos = np.arange(start_pos, start_pos + x.shape[0])
    cos, sin = yarn_tables(c["head_dim"], c["rope_base"], c["rope_factor"], c["original_context"], c["beta_fast"],
                           c["beta_slow"], pos)
    for layer in range(len(attn)):
        x = attention_block(x, attn[layer], cos.astype(np.float64), sin.astype(np.float64), kv, layer,
                            c["n_head"], c["n_head_kv"], c["head_dim"], c["sliding_window"], c["rms_eps"])
        Wr, br = routers[layer]
        h = OM.rms_norm(x, c["ffn_norm"][layer], c["rms_eps"])  # post_attention_norm (gpt_oss.py:123-130)
        x = x + OM.moe_gptoss(h, Wr, br, c["top_k"], experts[layer])[0]
    x = OM.rms_norm(x, out_norm, c["rms_eps"])
    return x @ lm_head.T
