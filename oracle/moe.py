"""CPU restatement (numpy) of the reference's MoE routing, activations and combine.

TEST INFRASTRUCTURE ONLY (the checker for the HIP path; never shipped).

Reference functions restated (paths relative to neurostream/):
  route_gptoss    model/gpt_oss.py:97-99,116-121  logits = h W^T + b; top-k on
                  logits; softmax over the k selected, in float32
  route_qwen3     moe/router.py:59-69             softmax over all experts in
                  float32; top-k; renormalise
  clamped_swiglu  model/gpt_oss.py:61-70
  silu_mul        moe/router.py:208 (F.silu(gate) * up)
  expert_ffn      compute/blockffn.py:396-449 (stream_expert_ffn: gate/up
                  windows, + bias row, activation, down window, + bias row)
  stream_linear   compute/blockffn.py:57-241 row-block walk, non-fused branch:
                  out[:, s-r0:e-r0] = x @ dequant(W[s:e]).T
  moe_gptoss      model/gpt_oss.py:123-177: per chosen expert in ascending id
                  order, out[rows] += w_e * y_e
  moe_qwen3       moe/router.py:173-219 (same combine, SiLU*up, no biases)
  rms_norm        compute/ops.py:14-20 (float32: x * rsqrt(mean(x^2) + eps) * w)
  ffn_stack       model/gpt_oss.py:123-177 per layer, attention left out:
                  x <- x + moe_l(rms_norm(x)) (composition of the above)

Top-k tie rule: torch.topk leaves the order of equal values unspecified; this
restatement (and the HIP kernel) takes the lower expert index first.

Pinning (tests/test_oracle_moe.py): brute force over all k-subsets on tiny
inputs, closed forms (softmax over the top-k sums to 1 and is monotone in the
logits, renormalised Qwen3 weights sum to 1), the activation's clamp and
sigmoid special values, block-decomposition invariance of stream_linear for
block_rows in {1, 7, 8, 64, 4096} (tests/test_gpt_oss.py:176-192), the
reference's known answer 528 (tests/test_tuning.py:135-153), and for rms_norm
unit output RMS at eps 0, invariance under power-of-two scaling, and the
closed form c / sqrt(c^2 + eps) of a constant row.
"""
from __future__ import annotations

import numpy as np

from . import quant


def topk_lower_index(v: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """(values, ids) of the k largest per row, descending; ties -> lower index."""
    v = np.asarray(v, dtype=np.float32)
    T, E = v.shape
    idx = np.empty((T, k), dtype=np.int64)
    for t in range(T):
        order = np.lexsort((np.arange(E), -v[t].astype(np.float64)))
        idx[t] = order[:k]
    return np.take_along_axis(v, idx, axis=1), idx


def softmax_f32(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, dtype=np.float32)
    m = v.max(axis=-1, keepdims=True)
    e = np.exp(v - m, dtype=np.float32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


def router_logits(h: np.ndarray, W: np.ndarray, b: np.ndarray | None) -> np.ndarray:
    logits = (np.asarray(h, np.float32) @ np.asarray(W, np.float32).T).astype(np.float32)
    if b is not None:
        logits = (logits + np.asarray(b, np.float32)).astype(np.float32)
    return logits


def route_gptoss(h, W, b, k):
    """(ids, weights, logits) -- gpt_oss.py:116-121."""
    logits = router_logits(h, W, b)
    top, ids = topk_lower_index(logits, k)
    return ids, softmax_f32(top), logits


def route_qwen3(h, W, k):
    """(ids, weights, logits) -- router.py:59-69."""
    logits = router_logits(h, W, None)
    probs = softmax_f32(logits)
    w, ids = topk_lower_index(probs, k)
    w = (w / w.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return ids, w, logits


def topk_margin(logits: np.ndarray, k: int) -> np.ndarray:
    """Gap between the k-th and (k+1)-th largest logit per token (near-tie check)."""
    s = -np.sort(-np.asarray(logits, np.float64), axis=-1)
    if s.shape[-1] <= k:
        return np.full(s.shape[0], np.inf)
    return s[:, k - 1] - s[:, k]


def clamped_swiglu(gate, up, alpha: float = 1.702, limit: float = 7.0):
    """GPT-OSS activation (gpt_oss.py:61-70), float32."""
    gate = np.minimum(np.asarray(gate, np.float32), np.float32(limit))
    up = np.clip(np.asarray(up, np.float32), np.float32(-limit), np.float32(limit))
    sig = (np.float32(1) / (np.float32(1) + np.exp(-gate * np.float32(alpha), dtype=np.float32)))
    return ((up + np.float32(1)) * (gate * sig)).astype(np.float32)


def silu_mul(gate, up):
    gate = np.asarray(gate, np.float32)
    sig = np.float32(1) / (np.float32(1) + np.exp(-gate, dtype=np.float32))
    return (gate * sig * np.asarray(up, np.float32)).astype(np.float32)


def stream_linear(raw_window: np.ndarray, dtype: int, x: np.ndarray, n_rows: int, K: int,
                  block_rows: int) -> np.ndarray:
    """x @ W.T over a row window, one block of rows at a time (blockffn.py:146-231)."""
    if block_rows <= 0:
        raise ValueError("block_rows must be positive")
    x = np.asarray(x, np.float32).reshape(-1, K)
    rb = quant.row_bytes(dtype, K)
    out = np.empty((x.shape[0], n_rows), dtype=np.float32)
    for lo in range(0, n_rows, block_rows):
        hi = min(lo + block_rows, n_rows)
        out[:, lo:hi] = quant.gemv(raw_window[lo * rb:hi * rb], dtype, x, hi - lo, K)
    return out


class ExpertSet:
    """Stacked expert tensors as raw GGUF bytes, expert e = rows [e*out, (e+1)*out).

    `raw[kind]` is a flat uint8 array or a callable e -> raw bytes of expert e,
    so large layers can be produced one expert at a time.
    """

    def __init__(self, dtype, n_embd, n_ff, raw, bias=None):
        self.dtype = dtype
        self.n_embd = n_embd
        self.n_ff = n_ff
        self.raw = raw
        self.bias = bias or {}

    def rows(self, kind):
        return self.n_ff if kind in ("gate", "up") else self.n_embd

    def K(self, kind):
        return self.n_embd if kind in ("gate", "up") else self.n_ff

    def expert_raw(self, kind, e):
        src = self.raw[kind]
        if callable(src):
            return src(e)
        n = self.rows(kind) * quant.row_bytes(self.dtype, self.K(kind))
        return src[e * n:(e + 1) * n]


def expert_ffn(ex: ExpertSet, e: int, x: np.ndarray, act, block_rows: int = 0) -> np.ndarray:
    """stream_expert_ffn (blockffn.py:396-449) for one expert."""
    def project(kind, value):
        n, K = ex.rows(kind), ex.K(kind)
        raw = ex.expert_raw(kind, e)
        if block_rows:
            y = stream_linear(raw, ex.dtype, value, n, K, block_rows)
        else:
            y = quant.gemv(raw, ex.dtype, value, n, K)
        if kind in ex.bias:
            y = (y + np.asarray(ex.bias[kind][e], np.float32)).astype(np.float32)
        return y

    gate = project("gate", x)
    up = project("up", x)
    return project("down", act(gate, up))


def combine(h, ids, weights, ex: ExpertSet, act, block_rows: int = 0) -> np.ndarray:
    """Ascending-expert combine: out[rows] += w_e * y_e (gpt_oss.py:139-177, router.py:186-211)."""
    h = np.asarray(h, np.float32)
    out = np.zeros_like(h)
    for e in np.unique(ids):
        mask = ids == e
        rows = np.nonzero(mask.any(-1))[0]
        if rows.size == 0:
            continue
        w = (weights * mask).sum(-1, dtype=np.float32)[rows, None]
        y = expert_ffn(ex, int(e), h[rows], act, block_rows)
        out[rows] += (w * y).astype(np.float32)
    return out


def moe_gptoss(h, W_r, b_r, k, ex: ExpertSet, alpha=1.702, limit=7.0, block_rows=0):
    """GPT-OSS MoE FFN output (without the residual) -- gpt_oss.py:123-177."""
    ids, w, logits = route_gptoss(h, W_r, b_r, k)
    act = lambda g, u: clamped_swiglu(g, u, alpha, limit)  # noqa: E731
    return combine(h, ids, w, ex, act, block_rows), ids, w, logits


def moe_qwen3(h, W_r, k, ex: ExpertSet, block_rows=0):
    """Qwen3-MoE FFN output -- router.py:173-219."""
    ids, w, logits = route_qwen3(h, W_r, k)
    return combine(h, ids, w, ex, silu_mul, block_rows), ids, w, logits


def rms_norm(x, weight=None, eps=1e-5):
    """compute/ops.py:14-20 in float32."""
    x = np.asarray(x, np.float32)
    var = (x * x).mean(-1, keepdims=True, dtype=np.float32)
    y = x * (np.float32(1) / np.sqrt(var + np.float32(eps), dtype=np.float32))
    if weight is not None:
        y = y * np.asarray(weight, np.float32)
    return y.astype(np.float32)


def ffn_stack(x, layers, k, eps=1e-5, block_rows=0):
    """x after each layer's FFN block, x <- x + moe_gptoss(rms_norm(x)).
    layers: [(W_r, b_r, ExpertSet)] (gpt_oss.py:123-177, one per layer)."""
    x = np.asarray(x, np.float32)
    for W_r, b_r, ex in layers:
        out = moe_gptoss(rms_norm(x, eps=eps), W_r, b_r, k, ex, block_rows=block_rows)[0]
        x = (x + out).astype(np.float32)
    return x
