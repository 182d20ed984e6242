"""oracle/torch_path.py (the torch restatement bench.py times as the CPU
baseline) against the numpy oracle: dequantize bit for bit for every block
type, stream_linear and the MoE layer within fp32 summation-order tolerance."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bit_mismatches, rel_max
from oracle import moe as OM
from oracle import quant as OQ
from oracle import torch_path as TP


def _random_blocks(dtype, n_blocks, seed, all_exponents=False):
    """Random block bytes with finite fp16 scale fields; MXFP4 exponents in
    117..123 (BASELINE's range), or cycling through every byte value."""
    rng = np.random.default_rng(seed)
    be, bb = OQ.LAYOUT[dtype]
    raw = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)
    fields = {OQ.Q4_0: (0,), OQ.Q8_0: (0,), OQ.Q4_K: (0, 2), OQ.Q6_K: (208,)}.get(dtype, ())
    for at in fields:
        raw[:, at:at + 2] = (rng.standard_normal(n_blocks) * 0.02).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if dtype == OQ.MXFP4:
        raw[:, 0] = np.arange(n_blocks) % 256 if all_exponents else rng.integers(117, 124, size=n_blocks)
    return raw.reshape(-1)


@pytest.mark.parametrize("dtype", [OQ.Q4_0, OQ.Q8_0, OQ.Q4_K, OQ.Q6_K, OQ.MXFP4])
def test_dequantize_bit_exact(dtype):
    be, _ = OQ.LAYOUT[dtype]
    raw = _random_blocks(dtype, 512, seed=dtype, all_exponents=True)
    n = 512 * be - 7  # truncated to n_elements as quant.py:184
    ref = OQ.dequantize(raw, dtype, n)
    got = TP.dequantize(torch.from_numpy(raw), dtype, n).numpy()
    assert got.dtype == np.float32 and got.shape == ref.shape
    assert bit_mismatches(got, ref).size == 0


def test_dequantize_errors():
    with pytest.raises(TypeError):
        TP.dequantize(torch.zeros(34, dtype=torch.int8), OQ.Q8_0, 32)
    with pytest.raises(NotImplementedError):
        TP.dequantize(torch.zeros(176, dtype=torch.uint8), 13, 256)  # Q5_K


@pytest.mark.parametrize("dtype,K", [(OQ.Q4_0, 4096), (OQ.MXFP4, 2880), (OQ.Q4_K, 1536)])
@pytest.mark.parametrize("block_rows", [1, 7, 512])
def test_stream_linear_matches_oracle(dtype, K, block_rows):
    rows = 40
    raw = _random_blocks(dtype, rows * K // OQ.LAYOUT[dtype][0], seed=K + block_rows)
    x = np.random.default_rng(1).standard_normal((2, K)).astype(np.float32)
    ref = OQ.gemv(raw, dtype, x, rows, K, f64=True)
    got = TP.stream_linear(torch.from_numpy(raw), dtype, torch.from_numpy(x), rows, K, block_rows).numpy()
    assert rel_max(got, ref) < 1e-5
    # a row window equals the same columns of the whole product
    win = TP.stream_linear(torch.from_numpy(raw), dtype, torch.from_numpy(x), rows, K, block_rows, 9, 33).numpy()
    assert rel_max(win, ref[:, 9:33]) < 1e-5
    with pytest.raises(ValueError):
        TP.stream_linear(torch.from_numpy(raw), dtype, torch.from_numpy(x), rows, K, 0)
    with pytest.raises(ValueError):
        TP.stream_linear(torch.from_numpy(raw), dtype, torch.from_numpy(x[:, :-32]), rows, K, 8)


@pytest.mark.parametrize("mode", ["gptoss", "qwen3"])
def test_moe_layer_matches_oracle(mode):
    rng = np.random.default_rng(3)
    E, k, n_embd, n_ff, T = 8, 2, 64, 96, 5
    dtype = OQ.MXFP4 if mode == "gptoss" else OQ.Q4_K
    if dtype == OQ.Q4_K:
        n_embd, n_ff = 256, 512
    raw = {kind: _random_blocks(dtype, E * rows * K // OQ.LAYOUT[dtype][0], seed=i)
           for i, (kind, rows, K) in enumerate((("gate", n_ff, n_embd), ("up", n_ff, n_embd),
                                                ("down", n_embd, n_ff)))}
    bias = ({kind: (rng.standard_normal((E, rows)) * 0.02).astype(np.float32)
             for kind, rows in (("gate", n_ff), ("up", n_ff), ("down", n_embd))} if mode == "gptoss" else {})
    h = rng.standard_normal((T, n_embd)).astype(np.float32)
    W = (rng.standard_normal((E, n_embd)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(E) * 0.1).astype(np.float32)
    ex = OM.ExpertSet(dtype, n_embd, n_ff, raw, bias)
    tex = TP.Experts(dtype, n_embd, n_ff, {kk: torch.from_numpy(v) for kk, v in raw.items()},
                     {kk: torch.from_numpy(v) for kk, v in bias.items()})
    ht = torch.from_numpy(h)
    if mode == "gptoss":
        ref, rid, rw, _ = OM.moe_gptoss(h, W, b, k, ex)
        ids, w = TP.route_gptoss(ht, torch.from_numpy(W), torch.from_numpy(b), k)
        act = TP.clamped_swiglu
    else:
        ref, rid, rw, _ = OM.moe_qwen3(h, W, k, ex)
        ids, w = TP.route_qwen3(ht, torch.from_numpy(W), k)
        act = TP.silu_mul
    np.testing.assert_array_equal(np.sort(ids.numpy(), 1), np.sort(rid, 1))
    got = TP.moe_layer(ht, ids, w, tex, act, block_rows=32).numpy()
    assert rel_max(got, ref) < 1e-5
