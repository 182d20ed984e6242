"""GGML blocks -> float tensors, on the GPU (compute/quant.py seam).

`dequantize` keeps the reference's signature and error behaviour
(neurostream/compute/quant.py:153-184): uint8 input or TypeError, F32/F16/BF16
are views plus a cast, unknown types raise NotImplementedError, the output is
truncated to `n_elements` and cast to `out_dtype`. Block formats (Q4_0, Q8_0,
Q4_K, Q6_K, MXFP4) expand in one HIP kernel, bit-exact with the reference; they need
the tensor on the GPU.
"""
from __future__ import annotations

import torch

from .. import _native as N
from ..format.gguf import GGMLType, TYPE_LAYOUT

_OUT = {torch.float32: N.DT_F32, torch.float16: N.DT_F16, torch.bfloat16: N.DT_BF16}


def dequantize(raw: torch.Tensor, dtype, n_elements: int,
               out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Expand `raw` bytes (uint8, 1-D) into a flat tensor of `n_elements`."""
    if raw.dtype != torch.uint8:
        raise TypeError(f"expected uint8 byte buffer, got {raw.dtype}")
    dtype = GGMLType(dtype)
    if dtype == GGMLType.F32:
        return raw.contiguous().view(torch.float32)[:n_elements].to(out_dtype)
    if dtype == GGMLType.F16:
        return raw.contiguous().view(torch.float16)[:n_elements].to(out_dtype)
    if dtype == GGMLType.BF16:
        return raw.contiguous().view(torch.bfloat16)[:n_elements].to(out_dtype)
    if dtype not in N.BLOCK_TYPES:
        raise NotImplementedError(
            f"no dequant kernel for {dtype.name}; supported: F32 F16 BF16 "
            + " ".join(t.name for t in sorted(N.BLOCK_TYPES)))
    N.require_device(raw)
    raw = raw.reshape(-1)
    if not raw.is_contiguous():
        raw = raw.contiguous()
    be, bb = TYPE_LAYOUT[dtype]
    nb = raw.numel() // bb
    n_elements = min(int(n_elements), nb * be)
    code = _OUT.get(out_dtype)
    out = torch.empty(n_elements, dtype=out_dtype if code is not None else torch.float32,
                      device=raw.device)
    if n_elements:
        with torch.cuda.device(raw.device):
            N.check(N.load().nsx_dequantize(int(dtype), raw.data_ptr(), raw.numel(), n_elements,
                                            out.data_ptr(), N.DT_F32 if code is None else code,
                                            N.stream_ptr(raw.device)), "dequantize")
    return out if code is not None else out.to(out_dtype)
