"""Row normalisation between stacked MoE layers, on the device.

compute/ops.py:14-20 (rms_norm, fp32) of the reference; `add_rms_norm`
folds the residual add of model/gpt_oss.py:177 into the same kernel
(nsx_add_rmsnorm). Quantized-weight math never runs here.
"""
from __future__ import annotations

import torch

from .. import _native as N


def add_rms_norm(x: torch.Tensor, r: torch.Tensor | None, weight: torch.Tensor | None, eps: float,
                 out: torch.Tensor | None = None, sum_out: torch.Tensor | None = None) -> torch.Tensor:
    """rms_norm(x + r) * weight over the last dimension, fp32 (r, weight
    optional); with sum_out, x + r is written there too (it may be x)."""
    N.require_device(x)
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise TypeError("add_rms_norm takes a contiguous fp32 x")
    n = x.shape[-1]
    T = x.numel() // n if n else 0
    for t in (r, out, sum_out):
        if t is not None and (t.shape != x.shape or t.dtype != torch.float32 or not t.is_contiguous()):
            raise ValueError("r, out and sum_out must be contiguous fp32 tensors shaped like x")
    w = None if weight is None else weight.float().contiguous()
    if w is not None and w.numel() != n:
        raise ValueError(f"weight of {w.numel()} elements for rows of {n}")
    y = torch.empty_like(x) if out is None else out
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    with torch.cuda.device(x.device):
        N.check(N.load().nsx_add_rmsnorm(x.data_ptr(), ptr(r), T, n, float(eps), ptr(w), ptr(sum_out), y.data_ptr(),
                                         N.stream_ptr(x.device)), "add_rmsnorm")
    return y


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """compute/ops.py:14-20: x * rsqrt(mean(x^2) + eps) * weight, in fp32."""
    return add_rms_norm(x.float().contiguous(), None, weight, eps)
