"""nsx_moe_forward_static (the allocation-free variant of nsx_moe_forward,
whose workspace is the library's per-GPU static array) against
nsx_moe_forward on the same layer and inputs: two calls in a row, the second
with fewer tokens, each bit-identical to the caller-workspace entry point
(the same kernels run) and within the parity bar of the CPU oracle."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from helpers import FFN_BAR, rel_max, to_np
from moe_cases import _layer, _oracle_layer, _small

pytestmark = pytest.mark.gpu


def _static(layer, h):
    """Through the C ABI directly: nsx_moe_forward_static(L, h, T, out, ids, weights, stream)."""
    from nurostream_amd import _native as N
    T = h.shape[0]
    out = torch.full((T, layer.n_embd), float("nan"), device=h.device)
    ids = torch.full((T, layer.top_k), -1, dtype=torch.int32, device=h.device)
    wts = torch.full((T, layer.top_k), float("nan"), device=h.device)
    rc = N.load().nsx_moe_forward_static(C.byref(layer._c), h.data_ptr(), T, out.data_ptr(), ids.data_ptr(),
                                         wts.data_ptr(), N.stream_ptr(h.device))
    N.check(rc, "moe_forward_static")
    return out, ids, wts


@pytest.mark.parametrize("name,layout,seq", [("gptoss-small", "t64", (20, 3)), ("qwen3-small", "gguf", (17, 2)),
                                             ("q4_0-small", "gguf", (9, 1)), ("gptoss-120b", "t64", (8, 1))])
def test_static_workspace_matches_forward(dev, name, layout, seq):
    from nurostream_amd import synth
    cfg = _small(name) if name != "gptoss-120b" else synth.GPTOSS_120B
    print(f"[no_alloc] {name} layout={layout} T={seq}", flush=True)
    t = synth.make_layer(cfg, seed=77, device=dev)
    layer = _layer(cfg, t, layout)
    for i, T in enumerate(seq):
        h = synth.activations(T, cfg.n_embd, seed=100 + i, device=dev)
        ref_out, ref_ids, ref_w = layer.forward(h)
        out, ids, w = _static(layer, h)
        torch.cuda.synchronize()
        assert torch.equal(ids, ref_ids)
        assert torch.equal(w, ref_w)
        assert torch.equal(out, ref_out), float((out - ref_out).abs().max())
        if T <= 3 or name != "gptoss-120b":
            ref, rid, _, _ = _oracle_layer(cfg, t, h.cpu().numpy())
            assert rel_max(to_np(out), ref) < FFN_BAR
            np.testing.assert_array_equal(np.sort(to_np(ids), 1), np.sort(rid, 1))


def test_static_workspace_python_method(dev):
    """MoELayer.forward_static is the same call, with the output checks of forward()."""
    from nurostream_amd import synth
    cfg = _small("gptoss-small")
    t = synth.make_layer(cfg, seed=5, device=dev)
    layer = _layer(cfg, t, "t64")
    h = synth.activations(4, cfg.n_embd, seed=6, device=dev)
    a = layer.forward(h)
    b = layer.forward_static(h)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    with pytest.raises(ValueError):
        layer.forward_static(h, out=torch.empty(4, cfg.n_embd + 1, device=dev))
