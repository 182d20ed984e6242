"""Pins the attention oracle (CPU only) by routes independent of its own formulas:
transformers' GPT-OSS rotary embedding and eager sink attention, torch's
scaled_dot_product_attention, and closed forms."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attn as OA

# GPT-OSS-120B attention geometry and rope parameters (GGUF keys of the model; BASELINE config 2's layer)
GPTOSS = dict(head_dim=64, base=150000.0, factor=32.0, original_context=4096, beta_fast=32.0, beta_slow=1.0)


def _hf_rotary():
    M = pytest.importorskip("transformers.models.gpt_oss.modeling_gpt_oss")
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig
    cfg = GptOssConfig(hidden_size=2880, num_attention_heads=64, num_key_value_heads=8, head_dim=64,
                       rope_theta=GPTOSS["base"], max_position_embeddings=131072,
                       rope_scaling={"rope_type": "yarn", "factor": GPTOSS["factor"], "beta_fast": GPTOSS["beta_fast"],
                                     "beta_slow": GPTOSS["beta_slow"], "truncate": False,
                                     "original_max_position_embeddings": GPTOSS["original_context"]})
    return M, M.GptOssRotaryEmbedding(cfg)


def test_yarn_matches_transformers():
    """Inverse frequencies, amplitude and cos/sin tables against transformers' GPT-OSS yarn rotary
    (untruncated correction range)."""
    M, rot = _hf_rotary()
    inv, amp = OA.yarn_inv_freq(**GPTOSS)
    np.testing.assert_allclose(inv, rot.inv_freq.numpy(), rtol=1e-6)
    assert amp == pytest.approx(rot.attention_scaling, rel=1e-12)
    pos = np.array([0, 1, 7, 127, 4095, 100_000])
    cos, sin = OA.yarn_tables(positions=pos, **GPTOSS)
    hc, hs = rot(torch.zeros(1, dtype=torch.float32), torch.from_numpy(pos)[None])
    # transformers keeps the half table; the reference repeats it
    hc, hs = np.concatenate([hc[0].numpy()] * 2, -1), np.concatenate([hs[0].numpy()] * 2, -1)
    np.testing.assert_allclose(cos[:-1], hc[:-1], rtol=0, atol=2e-4)
    np.testing.assert_allclose(sin[:-1], hs[:-1], rtol=0, atol=2e-4)
    # at position 1e5 a one-ulp difference of an fp32 inverse frequency (numpy's vs torch's pow)
    # moves the fp32 angle by up to 1e5 * 1.2e-7 rad: the tables agree to that
    np.testing.assert_allclose(cos[-1], hc[-1], rtol=0, atol=1e5 * 1.2e-7 * 1.35 * 2)
    np.testing.assert_allclose(sin[-1], hs[-1], rtol=0, atol=1e5 * 1.2e-7 * 1.35 * 2)


def test_yarn_factor_one_is_plain_rope():
    inv, amp = OA.yarn_inv_freq(64, 10000.0, 1.0, 4096, 32.0, 1.0)
    np.testing.assert_allclose(inv, 10000.0 ** (-np.arange(32) / 32.0), rtol=1e-6)
    assert amp == 1.0


def test_yarn_ramp_direction():
    """High-frequency dims (small i) keep the base frequency, low-frequency dims are divided by the factor."""
    inv, _ = OA.yarn_inv_freq(**GPTOSS)
    base = GPTOSS["base"] ** (-np.arange(32) / 32.0)
    assert inv[0] == pytest.approx(base[0], rel=1e-6)
    assert inv[-1] == pytest.approx(base[-1] / GPTOSS["factor"], rel=1e-5)


def test_apply_rope_matches_transformers():
    M, _ = _hf_rotary()
    rng = np.random.default_rng(0)
    x = rng.standard_normal((8, 5, 64)).astype(np.float32)
    pos = np.array([0, 3, 64, 1000, 77_777])
    cos, sin = OA.yarn_tables(positions=pos, **GPTOSS)
    got = OA.apply_rope(x, cos, sin)
    want = M._apply_rotary_emb(torch.from_numpy(x), torch.from_numpy(cos[:, :32])[None], torch.from_numpy(sin[:, :32])[None])
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-5, atol=1e-5)
    # position 0 with amplitude 1 is the identity; rotation keeps each pair's norm
    c1, s1 = OA.yarn_tables(64, 10000.0, 1.0, 4096, 32.0, 1.0, np.array([0, 9]))
    y = OA.apply_rope(x[:, :2], c1, s1)
    np.testing.assert_allclose(y[:, 0], x[:, 0], atol=1e-6)
    np.testing.assert_allclose(np.linalg.norm(y[:, 1], axis=-1), np.linalg.norm(x[:, 1], axis=-1), rtol=1e-5)


class _Mod:
    training = False

    def __init__(self, sinks, groups):
        self.sinks = sinks
        self.num_key_value_groups = groups


@pytest.mark.parametrize("window", [0, 4])
def test_sink_attention_matches_transformers_eager(window):
    """q/k/v with 8 query and 2 kv heads, a causal (and sliding) mask, learned sinks: the oracle
    equals transformers' eager GPT-OSS attention."""
    M, _ = _hf_rotary()
    rng = np.random.default_rng(1)
    tq, tk, H, Hkv, D = 3, 11, 8, 2, 16
    q = rng.standard_normal((H, tq, D)).astype(np.float32)
    k = rng.standard_normal((Hkv, tk, D)).astype(np.float32)
    v = rng.standard_normal((Hkv, tk, D)).astype(np.float32)
    sinks = rng.standard_normal(H).astype(np.float32)
    got = OA.sink_attention(q, OA.repeat_kv(k, H // Hkv), OA.repeat_kv(v, H // Hkv), sinks, window)
    qp = np.arange(tk - tq, tk)[:, None]
    kp = np.arange(tk)[None, :]
    vis = (kp <= qp) & ((kp > qp - window) if window else True)
    mask = torch.from_numpy(np.where(vis, 0.0, -np.inf).astype(np.float64))[None, None]
    want, _ = M.eager_attention_forward(_Mod(torch.from_numpy(sinks).double(), H // Hkv), torch.from_numpy(q).double()[None],
                                        torch.from_numpy(k).double()[None], torch.from_numpy(v).double()[None], mask,
                                        scaling=1 / math.sqrt(D))
    np.testing.assert_allclose(got, want[0].transpose(0, 1).numpy(), rtol=1e-10, atol=1e-12)


def test_sink_attention_limits():
    rng = np.random.default_rng(2)
    H, T, D = 4, 6, 8
    q, k, v = (rng.standard_normal((H, T, D)) for _ in range(3))
    # a sink of -inf leaves plain causal softmax attention
    got = OA.sink_attention(q, k, v, np.full(H, -np.inf))
    want = torch.nn.functional.scaled_dot_product_attention(*(torch.from_numpy(a) for a in (q, k, v)), is_causal=True)
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-10, atol=1e-12)
    # one key: out = v / (1 + exp(sink - s)), s = q.k / sqrt(D)
    q1, k1, v1 = q[:, :1], k[:, :1], v[:, :1]
    sinks = rng.standard_normal(H)
    s = (q1 * k1).sum(-1) / math.sqrt(D)
    np.testing.assert_allclose(OA.sink_attention(q1, k1, v1, sinks), v1 / (1 + np.exp(sinks[:, None, None] - s[..., None])),
                               rtol=1e-12)
    # a window of 1 sees only the query's own key
    w1 = OA.sink_attention(q, k, v, sinks, sliding_window=1)
    sd = (q * k).sum(-1) / math.sqrt(D)
    np.testing.assert_allclose(w1, v / (1 + np.exp(sinks[:, None, None] - sd[..., None])), rtol=1e-12)
