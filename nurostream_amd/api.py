"""Public surface of the reference (api.py:30-237, 336-441) over this build's MoE path.

    ns = NeuroStream.load("model.gguf", mem_budget="2GB", slab_budget="60GB")
    y = ns.model.ffn_stack(x)          # every layer's routed-expert FFN block
    for piece in ns.generate([1, 2, 3], max_tokens=16): ...
    ns.pin_hot_experts()
    print(ns.report())
    ns.close()                         # or: with NeuroStream.load(...) as ns:

`NeuroStream.load` keeps the reference's keyword arguments and their meaning
for the parts this build covers: the arena budget (`mem_budget`), VRAM/RAM
tiers, expert slabs in HBM (`slab_budget`, admitted in layer order as t64
tiles), `block_rows` and `expert_lookahead` for the streamed neuron path.
`generate` runs a GPT-OSS GGUF token by token on the device (embedding,
attention with YaRN rotary and sinks, the MoE FFN, the LM head) and takes
the prompt as token ids: the GGUF tokenizer is outside this build, so a str
prompt raises NotImplementedError. `report()` gathers the arena, reader,
cache, router and generation counters.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import torch

from .compute.blockffn import DEFAULT_BLOCK_ROWS, DEFAULT_LOOKAHEAD
from .format.gguf import FLOAT_TYPES, row_geometry
from .io.arena import Arena
from .io.stream import DiskSource
from .residency.cache import TieredCache

_UNIT_SHIFT = {"": 0, "K": 10, "M": 20, "G": 30, "T": 40}


def parse_size(v: int | str) -> int:
    """A byte count from an int (returned as is) or a string such as "2GB",
    "1.5G", "512MiB", "64K" or "4096": K / M / G / T are powers of 1024, the
    trailing "B" / "iB" optional (api.py:30-37 accepts the same forms)."""
    if isinstance(v, bool):
        raise ValueError(f"cannot parse size: {v!r}")
    if isinstance(v, int):
        return v
    text = str(v).strip().upper()
    for tail in ("IB", "B"):
        if text.endswith(tail) and len(text) > len(tail):
            text = text[:-len(tail)]
            break
    unit = text[-1] if text and text[-1] in _UNIT_SHIFT else ""
    number = text[:len(text) - len(unit)].strip()
    try:
        value = float(number)
    except ValueError:
        raise ValueError(f"cannot parse size: {v!r}") from None
    if not value >= 0 or value == float("inf"):
        raise ValueError(f"cannot parse size: {v!r}")
    return int(value * (1 << _UNIT_SHIFT[unit]))


@dataclass
class GenerationStats:
    prompt_tokens: int = 0
    generated_tokens: int = 0
    prefill_seconds: float = 0.0
    decode_seconds: float = 0.0

    @property
    def tokens_per_second(self) -> float:
        return 0.0 if self.decode_seconds <= 0 else self.generated_tokens / self.decode_seconds

    def summary(self) -> str:
        return (f"generate: {self.prompt_tokens} prompt tokens in {self.prefill_seconds:.3f} s, "
                f"{self.generated_tokens} generated in {self.decode_seconds:.3f} s "
                f"({self.tokens_per_second:.2f} tok/s)")


_EXPERT_TENSORS = ("ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight")


class NeuroStream:
    def __init__(self, path: str | Path, mem_budget: int | str = "2GB", vram_budget: int | str = 0,
                 ram_budget: int | str = 0, device: str | None = None, compute_dtype: torch.dtype | None = None,
                 block_rows: int = DEFAULT_BLOCK_ROWS, n_workers: int = 16, prefetch_depth: int = 1,
                 reserve_vram: int | str = "1.5GB", slab_budget: int | str = 0, strict_neuron: bool = False,
                 expert_lookahead: int = DEFAULT_LOOKAHEAD, verbose: bool = False) -> None:
        from .model.gpt_oss import GptOssModel, MoEModelConfig
        if device is None:
            device = "cuda" if torch.cuda.is_available() else "cpu"
        self.device = device
        self.dtype = compute_dtype or torch.float32
        self.verbose = verbose
        self.arena = Arena(parse_size(mem_budget))
        # weights stream from the file through n_workers reader threads (api.py:96-101)
        self.source = DiskSource(path, self.arena, n_workers=n_workers, device=device)
        self.gguf = self.source.gguf
        arch = self.gguf.arch()
        if arch != "gpt-oss":
            self.source.close()
            raise ValueError(f"unsupported architecture: {arch} (this build runs GPT-OSS MoE FFN stacks; "
                             "Qwen3 MoE layers run through nurostream_amd.model.qwen3 / moe.router.moe_ffn)")
        self.cfg = MoEModelConfig.from_gguf(self.gguf)
        self.cache = TieredCache(self.source, device=device, compute_dtype=self.dtype,
                                 vram_budget=parse_size(vram_budget), ram_budget=parse_size(ram_budget))
        self.cache.slab_budget = parse_size(slab_budget)
        if self.cache.vram_budget:
            self._admit_dense()
        if self.cache.slab_budget:
            self._admit_experts()
        self.model = GptOssModel(self.cache, self.cfg, device, self.dtype, block_rows=block_rows,
                                 expert_lookahead=expert_lookahead)
        self.stats = GenerationStats()

    @classmethod
    def load(cls, path: str | Path, **kw) -> "NeuroStream":
        return cls(path, **kw)

    def _expert_slabs(self, layer: int, e: int):
        """[(name, lo, hi, bytes)] of expert e's three matrices in `layer` not yet in HBM."""
        c, out = self.cfg, []
        for nm, rpe in zip(_EXPERT_TENSORS, (c.n_ffn_expert, c.n_ffn_expert, c.n_embd)):
            name = f"blk.{layer}.{nm}"
            if name not in self.gguf.tensors:
                continue
            lo, hi = e * rpe, (e + 1) * rpe
            if self.cache.is_resident(name) or self.cache.has_slab(name, lo, hi):
                continue
            info = self.gguf.tensors[name]
            if info.dtype in FLOAT_TYPES:
                continue
            out.append((name, lo, hi, rpe * row_geometry(info)[2]))
        return out

    def _admit_dense(self) -> int:
        """The non-expert tensors into HBM (TieredCache VRAM-Q: quantized ones
        stay raw for the fused GEMV), in file order while the VRAM budget lasts."""
        n = 0
        for name in self.gguf.tensors:
            if "_exps." in name:
                continue
            n += bool(self.cache.admit_vram(name))
        if self.verbose:
            print(f"  {n} dense tensors resident ({self.cache.stats.vram_bytes / 1e9:.2f}GB)", flush=True)
        return n

    def _admit(self, slabs) -> bool:
        """All of an expert's slabs or none (api.py:364-386: a partial expert
        must not consume the budget)."""
        need = sum(s[3] for s in slabs)
        if not slabs or need > self.cache.slab_budget - self.cache.slab_bytes:
            return False
        for name, lo, hi, _ in slabs:
            self.cache.admit_slab(name, lo, hi)
        return True

    def _admit_experts(self) -> int:
        """Expert slabs into HBM in layer order until the slab budget is spent."""
        n = 0
        for layer in range(self.cfg.n_layer):
            for e in range(self.cfg.n_expert):
                n += self._admit(self._expert_slabs(layer, e))
        if self.verbose:
            print(f"  {n} expert slabs resident ({self.cache.slab_bytes / 1e9:.2f}GB)", flush=True)
        return n

    def pin_hot_experts(self, verbose: bool = False) -> int:
        """api.py:342-388: promote the most-routed experts' three slabs into HBM,
        busiest first, skipping experts that do not fit whole."""
        rs = getattr(self.model, "router_stats", None)
        if rs is None or not self.cache.slab_budget:
            return 0
        pinned = 0
        for (layer, e), _count in rs.hits.most_common():
            pinned += self._admit(self._expert_slabs(layer, e))
        if verbose:
            print(f"  pinned {pinned} expert slabs ({self.cache.slab_bytes / 1e9:.2f}GB)", flush=True)
        return pinned

    # -- generation (api.py:179-237) -----------------------------------------

    @staticmethod
    def _sample(logits: torch.Tensor, temperature: float, top_p: float) -> int:
        """The next token (api.py:179-191): argmax at temperature <= 0; else a
        draw from softmax(logits / temperature) restricted, when 0 < top_p <
        1, to the smallest set of most likely tokens whose mass reaches top_p."""
        if temperature <= 0:
            return int(logits.argmax())
        probs = torch.softmax(logits.float() / temperature, dim=-1)
        if not 0 < top_p < 1:
            return int(torch.multinomial(probs, 1))
        p_desc, order = torch.sort(probs, descending=True)
        mass = torch.cumsum(p_desc, 0)
        n_keep = min(int(torch.searchsorted(mass, torch.tensor([top_p], dtype=mass.dtype))) + 1, p_desc.numel())
        return int(order[torch.multinomial(p_desc[:n_keep], 1)])

    def _piece(self, token: int) -> str:
        """The token's entry in the GGUF vocabulary (tokenizer.ggml.tokens), or <id> without one."""
        vocab = self.gguf.metadata.get("tokenizer.ggml.tokens")
        if vocab is not None and 0 <= token < len(vocab):
            return str(vocab[token])
        return f"<{token}>"

    def generate(self, prompt, max_tokens: int = 128, temperature: float = 0.0, top_p: float = 0.95,
                 stop_on_eos: bool = True):
        """Yield one text piece per generated token (api.py:193-237).

        The prompt is a list of token ids: the GGUF tokenizer (text to ids) is
        outside this build, so a str prompt raises NotImplementedError. The
        prompt runs through the model token by token, then each sampled token
        is decoded the same way (embedding, every layer's attention and MoE
        FFN, LM head, on the GPU). A piece is the token's vocabulary entry when
        the GGUF has one, else "<id>"."""
        import time
        from .model.decode import DeviceKV
        if isinstance(prompt, str):
            raise NotImplementedError("text prompts need the GGUF tokenizer, which is outside this build; "
                                      "pass a list of token ids")
        ids = [int(t) for t in prompt]
        if not ids:
            raise ValueError("empty prompt")
        c = self.model.attn_config()
        kv = DeviceKV(self.cfg.n_layer, c, min(c.context_length, len(ids) + max_tokens), self.device)
        self.stats = GenerationStats(prompt_tokens=len(ids))
        t0 = time.perf_counter()
        with torch.no_grad():
            logits = self.model.forward(ids, kv, start_pos=0)
        self.stats.prefill_seconds = time.perf_counter() - t0
        eos_id = self.gguf.metadata.get("tokenizer.ggml.eos_token_id")
        eos = set() if eos_id is None else {int(eos_id)}
        pos = len(ids)
        t0 = time.perf_counter()
        for _ in range(max_tokens):
            nxt = self._sample(logits[-1], temperature, top_p)
            if stop_on_eos and nxt in eos:
                break
            self.stats.generated_tokens += 1
            yield self._piece(nxt)
            if self.stats.generated_tokens >= max_tokens or pos >= kv.ctx_max:
                break
            with torch.no_grad():
                logits = self.model.forward([nxt], kv, start_pos=pos)
            pos += 1
        self.stats.decode_seconds = time.perf_counter() - t0

    # -- warm-up and introspection (api.py:336-341, 399-441) -------------------

    def warmup(self, prompt=None, tokens: int = 24) -> None:
        """Generate a few tokens greedily only to observe which experts fire,
        so that pin_hot_experts has measured routing to rank. The prompt is
        token ids (default: the GGUF's BOS id, else token 0, and the next
        seven ids)."""
        if prompt is None:
            bos = self.gguf.metadata.get("tokenizer.ggml.bos_token_id")
            start = 0 if bos is None else int(bos)
            vocab = self.gguf.tensors.get("token_embd.weight")
            n_vocab = vocab.torch_shape[0] if vocab is not None else 8
            prompt = [(start + i) % n_vocab for i in range(8)]
        for _ in self.generate(prompt, max_tokens=tokens, temperature=0.0, stop_on_eos=False):
            pass

    def report(self) -> str:
        """One line per subsystem: model file, device, arena budget, disk
        reader, cache tiers and slabs, router statistics, last generation."""
        info = [("model", f"{self.gguf.path.name}, {self.gguf.arch()}, "
                          f"{self.gguf.total_tensor_bytes() / 2**30:.2f} GiB of tensors"),
                ("device", f"{self.device}, compute {str(self.dtype).replace('torch.', '')}"),
                ("arena", self.arena.summary()),
                ("io", self.source.stats.summary()),
                ("cache", self.cache.stats.summary())]
        if self.cache.slab_bytes:
            info.append(("slabs", f"{self.cache.slab_bytes / 2**30:.2f} GiB of expert slabs in HBM, "
                                  f"{self.cache.stats.slab_hits} block reads served from them"))
        rs = getattr(self.model, "router_stats", None)
        if rs is not None:
            info.append(("router", rs.summary()))
        info.append(("generate", self.stats.summary()))
        width = max(len(k) for k, _ in info)
        return "\n".join(f"{k:<{width}} : {v}" for k, v in info)

    def close(self) -> None:
        """Drop every cached tensor and slab and close the disk reader."""
        cache = getattr(self, "cache", None)
        if cache is not None:
            cache.clear()
        src = getattr(self, "source", None)
        if src is not None:
            src.close()

    def __enter__(self) -> "NeuroStream":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
