"""The reference's CPU torch path, restated in torch, for bench.py's CPU baseline.

TEST INFRASTRUCTURE ONLY (the checker side, like the rest of oracle/): bench.py
times it on the GPU box's host cores as `cpu_baseline`, and tests compare it
with the numpy oracle. No product code imports it.

The reference computes its CPU path with torch ATen ops on CPU tensors; this
module does the same steps on the same dtypes so that its timing stands for
the reference's (paths relative to neurostream/):
  dequantize      compute/quant.py:118-184 -- block-vectorised ATen
                  elementwise passes over int32 / float32 temporaries
  stream_linear   compute/blockffn.py:57-241, the non-fused branch taken on a
                  CPU tensor (can_fuse is False off the GPU,
                  triton_kernels.py:189-196): per block of block_rows rows,
                  fetch the rows' bytes, dequantize, then x @ w.T in float32
                  (blockffn.py:218-223, via residency/cache.py fetch_rows)
  route_gptoss    model/gpt_oss.py:116-121 (biased router, topk, softmax of
                  the selected logits)
  route_qwen3     moe/router.py:59-69 (softmax, topk, renormalise)
  moe_layer       model/gpt_oss.py:123-177 (neuron path) and
                  moe/router.py:173-219: per chosen expert in ascending id,
                  gate / up windows (+ bias), activation, down window
                  (+ bias), out[rows] += w * y

Pinned in tests/test_oracle_torch_path.py: dequantize bit for bit against
oracle.quant for every block type, stream_linear and moe_layer against the
numpy oracle within fp32 summation-order tolerance.
"""
from __future__ import annotations

import torch

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16, MXFP4 = 0, 1, 2, 8, 12, 14, 30, 39
LAYOUT = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), MXFP4: (32, 17)}

# quant.py:137-139: ggml's doubled e2m1 values; with the halved scale below they are the OCP values
_E2M1X2 = torch.tensor([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], dtype=torch.float32)


def _half(b: torch.Tensor, at: int) -> torch.Tensor:
    """fp16 little-endian field at byte `at` of each block row, as a float32 column."""
    return b[:, at:at + 2].contiguous().view(torch.float16).float()


def _q4_0(b: torch.Tensor) -> torch.Tensor:
    q = b[:, 2:18].int()
    codes = torch.cat((q & 15, q >> 4), 1) - 8  # elements 0..15 low nibbles, 16..31 high
    return _half(b, 0) * codes.float()


def _q8_0(b: torch.Tensor) -> torch.Tensor:
    return _half(b, 0) * b[:, 2:34].contiguous().view(torch.int8).float()


def _mxfp4(b: torch.Tensor) -> torch.Tensor:
    e = b[:, :1].int()
    # 2^(e - 128) as float bits: subnormal patterns for e < 2, exponent field e - 1 otherwise
    bits = torch.where(e < 2, torch.bitwise_left_shift(torch.full_like(e, 1 << 21), e), (e - 1) << 23)
    scale = bits.view(torch.float32)
    q = b[:, 1:17]
    codes = torch.cat((q & 15, q >> 4), 1).long()
    return scale * _E2M1X2[codes]


def _q4_k(b: torch.Tensor) -> torch.Tensor:
    n = b.shape[0]
    s = b[:, 4:16].int()
    lo, mid, hi = s[:, 0:4], s[:, 4:8], s[:, 8:12]
    # get_scale_min_k4 (quant.py:24-38): sub-blocks 0..3 plain 6-bit fields, 4..7 split fields
    sc = torch.cat((lo & 63, (hi & 15) | ((lo >> 6) << 4)), 1).float()
    mn = torch.cat((mid & 63, (hi >> 4) | ((mid >> 6) << 4)), 1).float()
    qs = b[:, 16:144].int().view(n, 4, 32)
    codes = torch.stack((qs & 15, qs >> 4), 2).reshape(n, 8, 32).float()  # sub-block 2g low, 2g + 1 high
    d, dmin = _half(b, 0), _half(b, 2)
    return ((d * sc).unsqueeze(-1) * codes - (dmin * mn).unsqueeze(-1)).reshape(n, 256)


def _q6_k(b: torch.Tensor) -> torch.Tensor:
    n = b.shape[0]
    ql = b[:, 0:128].int().view(n, 2, 64)
    qh = b[:, 128:192].int().view(n, 2, 32)
    sc = b[:, 192:208].contiguous().view(torch.int8).float().view(n, 2, 8)
    d = _half(b, 208).view(n, 1, 1)
    parts = []
    for j, (src, shift) in enumerate(((ql[:, :, :32] & 15, 0), (ql[:, :, 32:] & 15, 2),
                                      (ql[:, :, :32] >> 4, 4), (ql[:, :, 32:] >> 4, 6))):
        q = (src | (((qh >> shift) & 3) << 4)) - 32
        # element l of the 32-wide quarter j uses scale 2 j + l // 16 of its half
        s = torch.repeat_interleave(sc[:, :, 2 * j:2 * j + 2], 16, dim=2)
        parts.append(d * s * q.float())
    return torch.cat(parts, 2).reshape(n, 256)


_DEQ = {Q4_0: _q4_0, Q8_0: _q8_0, MXFP4: _mxfp4, Q4_K: _q4_k, Q6_K: _q6_k}


def row_bytes(dtype: int, K: int) -> int:
    be, bb = LAYOUT[dtype]
    return K // be * bb


def dequantize(raw: torch.Tensor, dtype: int, n_elements: int) -> torch.Tensor:
    """compute/quant.py:153-184 on a CPU uint8 tensor -> float32 (n_elements,)."""
    if raw.dtype != torch.uint8:
        raise TypeError(f"expected a uint8 byte buffer, got {raw.dtype}")
    if dtype == F32:
        return raw.contiguous().view(torch.float32)[:n_elements].clone()
    if dtype in (F16, BF16):
        return raw.contiguous().view(torch.float16 if dtype == F16 else torch.bfloat16)[:n_elements].float()
    if dtype not in _DEQ:
        raise NotImplementedError(f"no dequantizer for ggml type {dtype}")
    bb = LAYOUT[dtype][1]
    nb = raw.numel() // bb
    return _DEQ[dtype](raw[:nb * bb].view(nb, bb)).reshape(-1)[:n_elements]


def stream_linear(raw: torch.Tensor, dtype: int, x: torch.Tensor, n_rows: int, K: int, block_rows: int = 512,
                  row_start: int = 0, row_end: int | None = None) -> torch.Tensor:
    """x @ W[row_start:row_end].T by blocks of rows, the CPU branch of
    compute/blockffn.py:57-241: each block's bytes are dequantized and
    multiplied on their own (the reference's peak memory is one block)."""
    if block_rows <= 0:
        raise ValueError("block_rows must be positive")
    if x.shape[-1] != K:
        raise ValueError(f"x has {x.shape[-1]} features, W rows span {K}")
    rb = row_bytes(dtype, K)
    row_end = n_rows if row_end is None else min(n_rows, row_end)
    row_start = max(0, row_start)
    out = torch.empty((x.shape[0], max(0, row_end - row_start)), dtype=torch.float32)
    for lo in range(row_start, row_end, block_rows):
        hi = min(lo + block_rows, row_end)
        w = dequantize(raw[lo * rb:hi * rb], dtype, (hi - lo) * K).view(hi - lo, K)
        out[:, lo - row_start:hi - row_start] = x @ w.T
    return out


def route_gptoss(h: torch.Tensor, W: torch.Tensor, b: torch.Tensor | None, k: int):
    logits = h @ W.T
    if b is not None:
        logits = logits + b
    top, ids = torch.topk(logits, k, dim=-1)
    return ids, torch.softmax(top.float(), dim=-1)


def route_qwen3(h: torch.Tensor, W: torch.Tensor, k: int):
    probs = torch.softmax((h @ W.T).float(), dim=-1)
    w, ids = torch.topk(probs, k, dim=-1)
    return ids, w / w.sum(-1, keepdim=True)


def clamped_swiglu(gate: torch.Tensor, up: torch.Tensor, alpha: float = 1.702, limit: float = 7.0):
    g = gate.clamp(max=limit)
    return (up.clamp(-limit, limit) + 1) * (g * torch.sigmoid(g * alpha))


def silu_mul(gate: torch.Tensor, up: torch.Tensor):
    return torch.nn.functional.silu(gate) * up


class Experts:
    """Stacked CPU expert tensors (uint8 GGUF rows; expert e = rows [e*out,
    (e+1)*out)) with optional float32 biases (n_expert, out) per projection."""

    def __init__(self, dtype: int, n_embd: int, n_ff: int, raw: dict, bias: dict | None = None):
        self.dtype, self.n_embd, self.n_ff = dtype, n_embd, n_ff
        self.raw = raw
        self.bias = bias or {}

    def project(self, kind: str, e: int, x: torch.Tensor, block_rows: int) -> torch.Tensor:
        """stream_expert_ffn's projection (blockffn.py:396-449): expert e's row
        window of the stacked tensor, plus the expert's bias row."""
        rows, K = (self.n_ff, self.n_embd) if kind in ("gate", "up") else (self.n_embd, self.n_ff)
        total = self.raw[kind].numel() // row_bytes(self.dtype, K)
        y = stream_linear(self.raw[kind], self.dtype, x, total, K, block_rows, e * rows, (e + 1) * rows)
        if kind in self.bias:
            y = y + self.bias[kind][e]
        return y


def moe_layer(h: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, ex: Experts, act, block_rows: int = 512,
              experts: list[int] | None = None) -> torch.Tensor:
    """The routed experts and the ascending-expert combine for routed tokens
    (gpt_oss.py:139-177, router.py:186-211). `experts` limits the walk to a
    subset of the chosen experts (a bounded timing sample)."""
    out = torch.zeros_like(h)
    chosen = torch.unique(ids).tolist() if experts is None else experts
    for e in chosen:
        mask = ids == e
        rows = mask.any(-1).nonzero(as_tuple=True)[0]
        if rows.numel() == 0:
            continue
        w = (weights * mask).sum(-1)[rows, None]
        x = h[rows]
        a = act(ex.project("gate", e, x, block_rows), ex.project("up", e, x, block_rows))
        out[rows] += w * ex.project("down", e, a, block_rows)
    return out
