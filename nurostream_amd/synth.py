"""Seeded synthetic weights and activations for the BASELINE configurations.

Raw GGUF bytes are generated directly (uniform code bytes; scale fields drawn
as the configurations specify), on whatever device the generator lives on, so
a 61 GB resident stack is produced on the GPU in seconds. Everything is a
function of (config, seed, layer); tests and bench.py share these builders.

Distribution choices not fixed by the configuration text:
  * MXFP4 exponent bytes e ~ U{117..123}: the scale 2^(e-127) spans
    2^-10..2^-4 in OCP terms (ggml stores 2^(e-128) times a doubled table).
  * Q4_K d, dmin = fp16(|N(0, 2^-8)|); Q4_0 d = fp16(|N(0, 0.02)|).
  * expert biases and router bias ~ N(0, 0.02) fp32; GPT-OSS router weight
    bf16 N(0, 0.02); Qwen3 router weight fp32 N(0, 0.02).
"""
from __future__ import annotations

import math

from dataclasses import dataclass

import torch

from .format.gguf import GGMLType, TYPE_LAYOUT


@dataclass(frozen=True)
class MoEConfig:
    name: str
    ggml_type: GGMLType
    n_expert: int
    top_k: int
    n_embd: int
    n_ff: int
    router_mode: str  # "gptoss" | "qwen3"
    act: str          # "clamped_swiglu" | "silu_mul"
    bias: bool
    router_dtype: torch.dtype

    def expert_bytes(self, kind: str) -> int:
        be, bb = TYPE_LAYOUT[self.ggml_type]
        rows, K = (self.n_ff, self.n_embd) if kind in ("gate", "up") else (self.n_embd, self.n_ff)
        return rows * (K // be) * bb

    def rows_K(self, kind: str):
        return (self.n_ff, self.n_embd) if kind in ("gate", "up") else (self.n_embd, self.n_ff)

    def layer_bytes_per_token(self) -> int:
        """Algorithmic bytes of one decode token through one layer (k experts)."""
        w = self.top_k * sum(self.expert_bytes(k) for k in ("gate", "up", "down"))
        router = self.n_expert * self.n_embd * torch.tensor([], dtype=self.router_dtype).element_size()
        bias = (self.n_expert * 4 + self.top_k * (2 * self.n_ff + self.n_embd) * 4) if self.bias else 0
        return w + router + bias + 2 * self.n_embd * 4


GPTOSS_120B = MoEConfig("gpt-oss-120b", GGMLType.MXFP4, 128, 4, 2880, 2880, "gptoss", "clamped_swiglu",
                        True, torch.bfloat16)
QWEN3_235B = MoEConfig("qwen3-235b-a22b", GGMLType.Q4_K, 128, 8, 4096, 1536, "qwen3", "silu_mul",
                       False, torch.float32)


def generator(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=torch.device(device))
    g.manual_seed(int(seed))
    return g


def _f16_abs_normal(n, std, gen, device) -> torch.Tensor:
    v = (torch.randn(n, generator=gen, device=device) * std).abs().to(torch.float16)
    return v.view(torch.uint8).reshape(n, 2)


def block_bytes(dtype: GGMLType, n_blocks: int, gen: torch.Generator, device, *, e_lo: int = 117,
                e_hi: int = 123, d_std: float | None = None) -> torch.Tensor:
    """n_blocks random ggml blocks of `dtype` as a flat uint8 tensor."""
    dtype = GGMLType(dtype)
    _, bb = TYPE_LAYOUT[dtype]
    b = torch.randint(0, 256, (n_blocks, bb), generator=gen, device=device, dtype=torch.uint8)
    if dtype == GGMLType.MXFP4:
        b[:, 0] = torch.randint(e_lo, e_hi + 1, (n_blocks,), generator=gen, device=device,
                                dtype=torch.int32).to(torch.uint8)
    elif dtype == GGMLType.Q4_0:
        b[:, 0:2] = _f16_abs_normal(n_blocks, 0.02 if d_std is None else d_std, gen, device)
    elif dtype == GGMLType.Q8_0:
        b[:, 0:2] = _f16_abs_normal(n_blocks, 0.02 if d_std is None else d_std, gen, device)
    elif dtype == GGMLType.Q4_K:
        s = 2.0 ** -8 if d_std is None else d_std
        b[:, 0:2] = _f16_abs_normal(n_blocks, s, gen, device)
        b[:, 2:4] = _f16_abs_normal(n_blocks, s, gen, device)
    elif dtype == GGMLType.Q6_K:
        # random int8 sub-block scales (bytes 192:208) and 6-bit codes; d small
        b[:, 208:210] = _f16_abs_normal(n_blocks, 2.0 ** -10 if d_std is None else d_std, gen, device)
    else:
        raise NotImplementedError(dtype)
    return b.reshape(-1)


def matrix_bytes(dtype: GGMLType, rows: int, K: int, gen, device, **kw) -> torch.Tensor:
    be, _ = TYPE_LAYOUT[GGMLType(dtype)]
    return block_bytes(dtype, rows * (K // be), gen, device, **kw)


def layer_seed(seed: int, layer: int) -> int:
    return int(seed) * 1000003 + int(layer) * 7919 + 17


def make_layer(cfg: MoEConfig, seed: int, device, layer: int = 0):
    """Raw tensors of one MoE layer: dict with router_w, router_b, gate/up/down
    (stacked raw GGUF bytes, expert-major), gate_b/up_b/down_b (or None)."""
    g = generator(layer_seed(seed, layer), device)
    out = {}
    out["router_w"] = (torch.randn(cfg.n_expert, cfg.n_embd, generator=g, device=device) * 0.02).to(cfg.router_dtype)
    # a router bias where the router uses one (GPT-OSS's; Qwen3's router has none, moe/router.py:59-69)
    rb = cfg.bias and cfg.router_mode == "gptoss"
    out["router_b"] = (torch.randn(cfg.n_expert, generator=g, device=device) * 0.02) if rb else None
    for kind in ("gate", "up", "down"):
        rows, K = cfg.rows_K(kind)
        out[kind] = matrix_bytes(cfg.ggml_type, cfg.n_expert * rows, K, g, device)
    for kind in ("gate", "up", "down"):
        rows, _ = cfg.rows_K(kind)
        out[kind + "_b"] = (torch.randn(cfg.n_expert, rows, generator=g, device=device) * 0.02) if cfg.bias else None
    return out


def activations(T: int, K: int, seed: int, device) -> torch.Tensor:
    g = generator(seed, device)
    return torch.randn(T, K, generator=g, device=device)


def zipf_router_bias(n_expert: int, s: float = 1.1, c: float = 1.0, seed: int = 0) -> torch.Tensor:
    """Per-expert router bias c*log(p_e), p_e ~ rank^-s over a seeded expert permutation."""
    g = torch.Generator().manual_seed(int(seed))
    ranks = torch.randperm(n_expert, generator=g).double() + 1.0
    p = ranks ** (-s)
    p = p / p.sum()
    return (c * torch.log(p)).float()


def _mean_distinct(logit_fn, n_expert: int, top_k: int, tokens: int, trials: int, seed: int) -> float:
    import numpy as np
    rng = np.random.default_rng(seed)
    tot = 0
    for _ in range(trials):
        v = logit_fn(rng)
        top = np.argpartition(-v, top_k - 1, axis=1)[:, :top_k]
        tot += len(np.unique(top))
    return tot / trials


def zipf_scale(router_w: torch.Tensor, s: float = 1.1, top_k: int = 4, tokens: int = 128,
               seed: int = 0) -> float:
    """c for zipf_router_bias such that top-k routing of `tokens` tokens with
    x ~ N(0, I) touches as many distinct experts as Gumbel-top-k sampling of
    Zipf(s) popularity does (Plackett-Luce: the reading of "expert popularity
    is Zipf(s)"). Logit e of a token is N(0, |w_e|^2); the bias c log p_e is
    found by bisection on the mean distinct count (seeded simulation)."""
    import numpy as np
    E = router_w.shape[0]
    sig = router_w.float().norm(dim=1).cpu().numpy().astype(np.float64)
    ranks = np.arange(1, E + 1, dtype=np.float64)
    logp = np.log(ranks ** (-s) / (ranks ** (-s)).sum())
    target = _mean_distinct(lambda r: logp + r.gumbel(size=(tokens, E)), E, top_k, tokens, 64, seed)
    lo, hi = 0.0, 20.0 * float(sig.mean())
    for _ in range(30):  # more bias -> fewer distinct experts
        c = 0.5 * (lo + hi)
        got = _mean_distinct(lambda r: c * logp + r.standard_normal((tokens, E)) * sig, E, top_k, tokens, 64, seed + 1)
        lo, hi = (c, hi) if got > target else (lo, c)
    return 0.5 * (lo + hi)


def make_zipf_layer(cfg: MoEConfig, seed: int, device, s: float = 1.1, layer: int = 0):
    """make_layer with the router bias replaced by zipf_router_bias (BASELINE
    config 3: expert popularity ~ Zipf(s)); returns (tensors, c)."""
    t = make_layer(cfg, seed, device, layer)
    c = zipf_scale(t["router_w"], s=s, top_k=cfg.top_k)
    t["router_b"] = zipf_router_bias(cfg.n_expert, s=s, c=c, seed=layer_seed(seed, layer)).to(device)
    return t, c
