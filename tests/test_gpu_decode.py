"""GPU parity of a GPT-OSS decode token around the MoE FFN: the rotary +
cache-append and sink-attention kernels step by step against the oracle, the
embedding row gather, and a whole tiny GPT-OSS model (GGUF on disk) through
NeuroStream -- eager forward, generate() and the one-graph decode token."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import MFMA_TOL, bit_mismatches, rel_max, to_np
from oracle import attn as OA
from oracle import moe as OM
from oracle import quant as OQ

pytestmark = pytest.mark.gpu


def _cfg(n_head=16, n_kv=2, window=128, ctx=4096):
    from nurostream_amd.model.decode import AttnConfig
    return AttnConfig(n_head=n_head, n_head_kv=n_kv, head_dim=64, vocab_size=10, rope_base=150000.0,
                      context_length=ctx, sliding_window=window)


@pytest.mark.parametrize("window", [0, 128])
@pytest.mark.parametrize("heads", [(16, 2), (4, 4), (6, 2), (32, 2)], ids=["rep8", "rep1", "rep3", "rep16"])
def test_attention_kernels_match_oracle(dev, window, heads):
    """300 decode steps (past two 128-key chunks, each two 64-key rounds): bias + YaRN rotary +
    append, then sink attention against the oracle with the caches built the reference's way;
    1, 3, 8 and 16 query heads per kv head (one to four heads per wave)."""
    from nurostream_amd.model.decode import DeviceKV, advance, attn_decode, rope_kv_append, yarn_inv_freq
    c = _cfg(n_head=heads[0], n_kv=heads[1])
    L = 300
    rng = np.random.default_rng(5)
    kv = DeviceKV(1, c, L, dev)
    inv_p, amp = yarn_inv_freq(c, dev)
    inv_o, amp_o = OA.yarn_inv_freq(64, c.rope_base, c.rope_factor, c.original_context, c.beta_fast, c.beta_slow)
    # the product's frequencies (torch fp32) are the oracle's up to a last-place pow rounding; the
    # kernel gets the oracle's, so the comparison below isolates the kernel's own arithmetic
    np.testing.assert_allclose(to_np(inv_p), inv_o, rtol=1e-6)
    assert amp == pytest.approx(amp_o, rel=1e-12)
    inv = torch.from_numpy(inv_o).to(dev)
    bq, bk, bv = (torch.from_numpy(rng.standard_normal(n * 64).astype(np.float32)).to(dev)
                  for n in (c.n_head, c.n_head_kv, c.n_head_kv))
    sinks = torch.from_numpy(rng.standard_normal(c.n_head).astype(np.float32)).to(dev)
    Kref = np.zeros((c.n_head_kv, 0, 64))
    Vref = np.zeros((c.n_head_kv, 0, 64))
    checks = {0, 1, 2, 63, 64, 65, 127, 128, 129, 191, 192, 255, 256, 257, L - 1}
    worst = 0.0
    for p in range(L):
        rows = rng.standard_normal((c.n_head + 2 * c.n_head_kv, 64)).astype(np.float32)
        qkv = torch.from_numpy(rows.reshape(-1)).to(dev)
        rope_kv_append(qkv, bq, bk, bv, c, inv, amp, kv, 0)
        att = attn_decode(qkv[:c.n_head * 64], kv, 0, sinks, window, c)
        advance(kv)
        cos, sin = OA.yarn_tables(64, c.rope_base, c.rope_factor, c.original_context, c.beta_fast, c.beta_slow, [p])
        x = rows.astype(np.float64)
        q = OA.apply_rope((x[:c.n_head] + bq.cpu().numpy().reshape(c.n_head, 64))[:, None], cos, sin)
        nkv = c.n_head_kv
        k = OA.apply_rope((x[c.n_head:c.n_head + nkv] + bk.cpu().numpy().reshape(nkv, 64))[:, None], cos, sin)
        v = (x[c.n_head + nkv:] + bv.cpu().numpy().reshape(nkv, 64))[:, None]
        Kref = np.concatenate([Kref, k], axis=1)
        Vref = np.concatenate([Vref, v], axis=1)
        if p in checks:
            ref = OA.sink_attention(q, OA.repeat_kv(Kref, c.n_rep), OA.repeat_kv(Vref, c.n_rep),
                                    sinks.cpu().numpy(), window)[:, 0]
            err = rel_max(to_np(att), ref)
            worst = max(worst, err)
            assert err < 2e-5, (p, err)
            np.testing.assert_allclose(to_np(qkv[:c.n_head * 64]).reshape(c.n_head, 64), q[:, 0], rtol=0, atol=2e-5)
    assert kv.length == L and int(kv.pos.item()) == L
    np.testing.assert_allclose(to_np(kv.k[0]), Kref, rtol=0, atol=2e-5)
    np.testing.assert_allclose(to_np(kv.v[0]), Vref, rtol=0, atol=1e-6)


@pytest.mark.parametrize("window", [0, 128])
@pytest.mark.parametrize("heads", [(16, 2), (6, 2)], ids=["rep8", "rep3"])
def test_fused_attention_equals_two_calls(dev, window, heads):
    """attn_decode_qkv (bias + rotary + append inside the attention launch) against rope_kv_append
    followed by attn_decode: outputs and both caches bit-identical over 300 positions, the raw
    q | k | v block left unchanged."""
    from nurostream_amd.model.decode import (DeviceKV, advance, attn_decode, attn_decode_qkv, rope_kv_append,
                                             yarn_inv_freq)
    c = _cfg(n_head=heads[0], n_kv=heads[1])
    L = 300
    g = torch.Generator(device="cpu").manual_seed(11)
    kv1, kv2 = DeviceKV(1, c, L, dev), DeviceKV(1, c, L, dev)
    inv, amp = yarn_inv_freq(c, dev)
    bq, bk, bv = (torch.randn(n * 64, generator=g).to(dev) for n in (c.n_head, c.n_head_kv, c.n_head_kv))
    sinks = torch.randn(c.n_head, generator=g).to(dev)
    rows = c.n_head + 2 * c.n_head_kv
    for p in range(L):
        raw = torch.randn(rows * 64, generator=g).to(dev)
        qkv = raw.clone()
        rope_kv_append(qkv, bq, bk, bv, c, inv, amp, kv1, 0)
        a1 = attn_decode(qkv[:c.n_head * 64], kv1, 0, sinks, window, c)
        keep = raw.clone()
        a2 = attn_decode_qkv(raw, bq, bk, bv, c, inv, amp, kv2, 0, sinks, window)
        advance(kv1)
        advance(kv2)
        if p in (0, 1, 63, 64, 127, 128, 129, 255, 256, L - 1):
            assert torch.equal(a1, a2), p
            assert torch.equal(raw, keep), p
    torch.cuda.synchronize()
    assert torch.equal(kv1.k[0], kv2.k[0]) and torch.equal(kv1.v[0], kv2.v[0])
    # no bias: the same identity
    q0 = torch.randn(rows * 64, generator=g).to(dev)
    kv1.reset(), kv2.reset()
    q1 = q0.clone()
    rope_kv_append(q1, None, None, None, c, inv, amp, kv1, 0)
    assert torch.equal(attn_decode(q1[:c.n_head * 64], kv1, 0, None, window, c),
                       attn_decode_qkv(q0, None, None, None, c, inv, amp, kv2, 0, None, window))


def test_attention_position_outside_cache_writes_nothing(dev):
    """A position at or past the cache capacity leaves the caches and the output untouched."""
    from nurostream_amd.model.decode import DeviceKV, attn_decode, attn_decode_qkv, rope_kv_append, yarn_inv_freq
    c = _cfg(n_head=8, n_kv=8, window=0)
    kv = DeviceKV(1, c, 4, dev)
    kv.pos.fill_(4)
    inv, amp = yarn_inv_freq(c, dev)
    qkv = torch.ones((c.n_head + 2 * c.n_head_kv) * 64, device=dev)
    rope_kv_append(qkv, None, None, None, c, inv, amp, kv, 0)
    out = torch.full((c.n_head, 64), 7.0, device=dev)
    attn_decode(qkv[:c.n_head * 64], kv, 0, None, 0, c, out=out)
    attn_decode_qkv(qkv, None, None, None, c, inv, amp, kv, 0, None, 0, out=out)
    torch.cuda.synchronize()
    assert float(kv.k[0].abs().sum()) == 0.0 and float(kv.v[0].abs().sum()) == 0.0
    assert bool((out == 7.0).all())


@pytest.mark.parametrize("fmt", ["Q8_0", "Q6_K", "MXFP4", "Q4_K", "Q4_0", "F32", "BF16"])
def test_dequantize_rows_bit_exact(dev, fmt):
    """Embedding rows by device ids (gather_embeddings) equal the oracle's dequantized rows; an id
    outside the table gives zeros."""
    from nurostream_amd import synth
    from nurostream_amd.model.decode import dequantize_rows
    rows, K = 50, 512
    t = getattr(OQ, fmt)
    if fmt in ("F32", "BF16"):
        w = np.random.default_rng(1).standard_normal((rows, K)).astype(np.float32)
        raw = (torch.from_numpy(w).to(torch.bfloat16) if fmt == "BF16" else torch.from_numpy(w)).view(torch.uint8)
        raw = raw.reshape(-1).clone()
    else:
        raw = synth.matrix_bytes(t, rows, K, synth.generator(3, "cpu"), "cpu")
    ids = torch.tensor([0, 7, 49, 7, -1, 50, 23], dtype=torch.int32)
    got = to_np(dequantize_rows(raw.to(dev), t, rows, K, ids.to(dev)))
    full = OQ.dequantize(raw.numpy(), t, rows * K).reshape(rows, K)
    want = np.stack([full[i] if 0 <= i < rows else np.zeros(K, np.float32) for i in ids.tolist()])
    assert bit_mismatches(got, want).size == 0


def _tiny_model(tmp_path, dev, n_layers=2):
    """A two-layer GPT-OSS GGUF (MXFP4 experts, Q8_0 attention / embedding / head) loaded with
    every tensor in HBM, and the float weights the oracle needs."""
    from api_cases import ATTN, write_gptoss_gguf
    from nurostream_amd import synth
    from nurostream_amd.api import NeuroStream
    from nurostream_amd.format.gguf import GGMLType
    cfg = synth.MoEConfig("s", GGMLType.MXFP4, 8, 4, 256, 192, "gptoss", "clamped_swiglu", True, torch.bfloat16)
    path = tmp_path / "tiny.gguf"
    layers = write_gptoss_gguf(path, cfg, n_layers=n_layers, seed=4, attention=True)
    ns = NeuroStream.load(path, device="cuda", vram_budget="1GB", slab_budget="1GB", block_rows=64)
    m = layers["model"]
    a = ATTN
    dq = lambda name, shape: OA.dequant(m[name].numpy(), OQ.Q8_0, shape)  # noqa: E731
    nq, nkv = a["n_head"] * 64, a["n_head_kv"] * 64
    attn, experts, routers, norms = [], [], [], []
    for li in range(n_layers):
        p = f"blk.{li}."
        attn.append(OA.AttnWeights(m[p + "attn_norm.weight"].numpy(), dq(p + "attn_q.weight", (nq, cfg.n_embd)),
                                   m[p + "attn_q.bias"].numpy(), dq(p + "attn_k.weight", (nkv, cfg.n_embd)),
                                   m[p + "attn_k.bias"].numpy(), dq(p + "attn_v.weight", (nkv, cfg.n_embd)),
                                   m[p + "attn_v.bias"].numpy(), dq(p + "attn_output.weight", (cfg.n_embd, nq)),
                                   m[p + "attn_output.bias"].numpy(), m[p + "attn_sinks.weight"].numpy()))
        t = layers[li]
        experts.append(OM.ExpertSet(OQ.MXFP4, cfg.n_embd, cfg.n_ff, {k: t[k].numpy() for k in ("gate", "up", "down")},
                                    {k: t[k + "_b"].numpy() for k in ("gate", "up", "down")}))
        routers.append((t["router_w"].float().numpy(), t["router_b"].numpy()))
        norms.append(t["norm"].numpy())
    ocfg = dict(head_dim=64, rope_base=a["rope_base"], rope_factor=a["rope_factor"],
                original_context=a["original_context"], beta_fast=a["beta_fast"], beta_slow=a["beta_slow"],
                n_head=a["n_head"], n_head_kv=a["n_head_kv"], sliding_window=a["window"], rms_eps=1e-5,
                top_k=cfg.top_k, ffn_norm=norms)
    emb = dq("token_embd.weight", (a["vocab"], cfg.n_embd))
    head = dq("output.weight", (a["vocab"], cfg.n_embd))
    oracle = dict(emb=emb, attn=attn, experts=experts, routers=routers, out_norm=m["output_norm.weight"].numpy(),
                  lm_head=head, cfg=ocfg)
    return ns, oracle


def test_tiny_gptoss_decode_matches_oracle(dev, tmp_path):
    """Prompt of 6 tokens (past the sliding window of 4) then 3 more, logits at every position
    against the oracle's forward (the experts run as fused t64 layers: MFMA tolerance)."""
    from nurostream_amd.model.decode import DeviceKV
    ns, o = _tiny_model(tmp_path, dev)
    model = ns.model
    assert all(model._fused_layer(li) is not None for li in range(ns.cfg.n_layer))
    toks = [5, 17, 42, 7, 250, 3, 99, 1, 288]
    kv = DeviceKV(ns.cfg.n_layer, model.attn_config(), 16, dev)
    got = to_np(model.forward(toks[:6], kv, start_pos=0, last_only=False))
    for i, t in enumerate(toks[6:]):
        got = np.concatenate([got, to_np(model.forward([t], kv, start_pos=6 + i))])
    ref = OA.forward_tokens(toks, o["emb"], o["attn"], o["experts"], o["routers"], o["out_norm"], o["lm_head"],
                            o["cfg"], {}, 0)
    for i in range(len(toks)):
        assert rel_max(got[i], ref[i]) < 2 * MFMA_TOL, i
    with pytest.raises(ValueError):
        model.forward([1], kv, start_pos=3)  # positions must follow the cache


def test_tiny_gptoss_generate_greedy(dev, tmp_path):
    """generate(list of ids) at temperature 0 yields the oracle's greedy continuation."""
    ns, o = _tiny_model(tmp_path, dev)
    prompt = [11, 200, 37]
    pieces = list(ns.generate(prompt, max_tokens=5))
    assert len(pieces) == 5 and ns.stats.generated_tokens == 5 and ns.stats.prompt_tokens == 3
    toks = list(prompt)
    for _ in range(5):
        ref = OA.forward_tokens(toks, o["emb"], o["attn"], o["experts"], o["routers"], o["out_norm"], o["lm_head"],
                                o["cfg"], {}, 0)[-1]
        s = np.sort(ref)
        assert s[-1] - s[-2] > 1e-3 * np.abs(ref).max(), "near-tie in the oracle's argmax"
        toks.append(int(np.argmax(ref)))
    assert pieces == [f"<{t}>" for t in toks[3:]]


def test_tiny_gptoss_decode_graph_replays(dev, tmp_path):
    """The whole decode token as one HIP graph: each replay (with eager work in between) equals
    the eager path on its own cache, bit for bit, and the position advances on the device."""
    from nurostream_amd.model.decode import DeviceKV
    from nurostream_amd.model.gpt_oss import GptOssDecodeGraph
    ns, _ = _tiny_model(tmp_path, dev)
    model = ns.model
    c = model.attn_config()
    kv_g, kv_e = DeviceKV(ns.cfg.n_layer, c, 12, dev), DeviceKV(ns.cfg.n_layer, c, 12, dev)
    g = GptOssDecodeGraph(model, kv_g)
    assert kv_g.length == 0 and int(kv_g.pos.item()) == 0
    for i, t in enumerate([5, 17, 42, 7, 250, 3, 99]):
        lg = g.step(t).clone()
        le = model.forward([t], kv_e, start_pos=i)
        torch.cuda.synchronize()
        assert torch.equal(lg, le), i
        _ = torch.randn(1000, device=dev).sum().item()  # eager work between replays
    assert kv_g.length == 7 and int(kv_g.pos.item()) == 7
    assert torch.equal(kv_g.k[1], kv_e.k[1]) and torch.equal(kv_g.v[0], kv_e.v[0])
