"""Fused dequant-GEMV seam (compute/triton_kernels.py replacement).

`can_fuse(dtype, x)` / `fused_gemv(raw, dtype, x, n_rows, K, out_dtype)` keep
the reference's signatures (neurostream/compute/triton_kernels.py:189-228).
Differences, all widenings: Q4_0 has a fused kernel here (the reference has
none), T up to 16 tokens is fused (the reference fuses T == 1 only), and `raw`
may also be a `T64Rows` window of a slab admitted in the t64 layout.
`block_n` / `num_warps` are accepted for call compatibility and ignored: the
HIP kernels choose their own launch shapes.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _native as N
from ..format.gguf import GGMLType, TYPE_LAYOUT

MAX_FUSED_T = 16
MAX_T64_T = 4


@dataclass
class T64Rows:
    """Rows [lo, hi) of an (n_rows, K) MXFP4 matrix stored in the t64 layout.

    Produced by `TieredCache.raw_rows` for slabs admitted with layout="t64";
    `buf` is the whole slab (the tile layout has no cheap byte sub-range).
    """

    buf: torch.Tensor
    dtype: GGMLType
    n_rows: int
    K: int
    lo: int
    hi: int

    @property
    def device(self):
        return self.buf.device

    @property
    def is_cuda(self) -> bool:
        return self.buf.is_cuda

    def rows(self, lo: int, hi: int) -> "T64Rows":
        """Sub-window [lo, hi) relative to this window."""
        return T64Rows(self.buf, self.dtype, self.n_rows, self.K, self.lo + lo, self.lo + hi)

    def to_gguf(self) -> torch.Tensor:
        """The window's raw GGUF bytes (untiled on the device)."""
        K, n = self.K, self.n_rows
        raw = torch.empty(n * (K // 32) * 17, dtype=torch.uint8, device=self.buf.device)
        with torch.cuda.device(self.buf.device):
            N.check(N.load().nsx_t64_unpack(int(self.dtype), self.buf.data_ptr(), n, K, raw.data_ptr(),
                                             N.stream_ptr(self.buf.device)), "t64_unpack")
        rb = (K // 32) * 17
        return raw[self.lo * rb:self.hi * rb]


def t64_pack(raw: torch.Tensor, dtype, n_rows: int, K: int) -> torch.Tensor:
    """Re-lay raw MXFP4 rows (device uint8) into a new t64 slab tensor."""
    N.require_device(raw)
    dtype = GGMLType(dtype)
    nbytes = N.load().nsx_t64_bytes(int(dtype), n_rows, K)
    if nbytes < 0:
        raise NotImplementedError(f"t64 layout for {dtype.name} K={K}")
    raw = raw.reshape(-1).contiguous()
    out = torch.empty(nbytes, dtype=torch.uint8, device=raw.device)
    with torch.cuda.device(raw.device):
        N.check(N.load().nsx_t64_pack(int(dtype), raw.data_ptr(), n_rows, K, out.data_ptr(),
                                      N.stream_ptr(raw.device)), "t64_pack")
    return out


def t64_pack_stacked(raw: torch.Tensor, dtype, n_expert: int, rows: int, K: int) -> torch.Tensor:
    """Re-lay a stacked (n_expert, rows, K) raw MXFP4 tensor as n_expert
    contiguous t64 slabs (expert e at e * nsx_t64_bytes(rows, K))."""
    N.require_device(raw)
    dtype = GGMLType(dtype)
    per = N.load().nsx_t64_bytes(int(dtype), rows, K)
    if per < 0:
        raise NotImplementedError(f"t64 layout for {dtype.name} K={K}")
    be, bb = TYPE_LAYOUT[dtype]
    rb = rows * (K // be) * bb
    raw = raw.reshape(-1).contiguous()
    if raw.numel() < rb * n_expert:
        raise ValueError(f"{raw.numel()} bytes for {n_expert} x {rows} x {K}")
    out = torch.empty(per * n_expert, dtype=torch.uint8, device=raw.device)
    lib = N.load()
    with torch.cuda.device(raw.device):
        s = N.stream_ptr(raw.device)
        for e in range(n_expert):
            N.check(lib.nsx_t64_pack(int(dtype), raw[e * rb:].data_ptr(), rows, K, out[e * per:].data_ptr(), s),
                    "t64_pack")
    return out


def can_fuse(dtype, x: torch.Tensor) -> bool:
    """Fused path: block-quantized weights, activations on the GPU, T <= 16."""
    try:
        dtype = GGMLType(dtype)
    except ValueError:
        return False
    if dtype not in N.BLOCK_TYPES or not x.is_cuda:
        return False
    T = x.shape[0] if x.dim() > 1 else 1
    if not 1 <= T <= MAX_FUSED_T:
        return False
    try:
        N.load()
    except N.NativeError:
        return False
    return True


def fused_gemv_norm(raw, dtype, x: torch.Tensor, r: torch.Tensor | None, weight: torch.Tensor | None, eps: float,
                    n_rows: int, K: int, sum_out: torch.Tensor | None = None, bias: torch.Tensor | None = None,
                    resid: torch.Tensor | None = None) -> torch.Tensor:
    """One token's y = W . rms_norm(x + r) * weight (+ bias, + resid) -> (1, n_rows) fp32, the norm in the
    GEMV's prologue with the bits add_rms_norm gives it (one launch instead of two); with sum_out, x + r is
    written there too (sum_out must not overlap x, r, resid or y). Raw GGUF rows; x, r, weight: K fp32 values."""
    dtype = GGMLType(dtype)
    if dtype not in N.BLOCK_TYPES:
        raise KeyError(dtype)
    if raw.dtype != torch.uint8:
        raise TypeError(f"expected uint8 byte buffer, got {raw.dtype}")
    N.require_device(raw)
    be, bb = TYPE_LAYOUT[dtype]
    flat = raw.reshape(-1)
    if flat.numel() < n_rows * (K // be) * bb:
        raise ValueError(f"raw has {flat.numel()} bytes, {n_rows} x {K} {dtype.name} needs {n_rows * (K // be) * bb}")
    if not flat.is_contiguous():
        flat = flat.contiguous()
    vec = {"x": (x, K), "r": (r, K), "weight": (weight, K), "sum_out": (sum_out, K), "bias": (bias, n_rows),
           "resid": (resid, n_rows)}
    for name, (t, n) in vec.items():
        if t is not None and (not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != n):
            raise ValueError(f"{name} must be a contiguous fp32 device tensor of {n} elements")
    if x.data_ptr() % 16:
        raise ValueError("x must be 16-byte aligned")
    if sum_out is not None and (sum_out.data_ptr() == x.data_ptr() or (r is not None and sum_out.data_ptr() == r.data_ptr())):
        raise ValueError("sum_out must not be x or r")
    y = torch.empty((1, n_rows), dtype=torch.float32, device=x.device)
    if n_rows == 0:
        return y
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    with torch.cuda.device(x.device):
        N.check(N.load().nsx_fused_gemv_norm(int(dtype), flat.data_ptr(), n_rows, K, x.data_ptr(), ptr(r),
                                             ptr(weight), float(eps), ptr(sum_out), y.data_ptr(), ptr(bias),
                                             ptr(resid), N.stream_ptr(x.device)), "fused_gemv_norm")
    return y


def fused_gemv(raw, dtype, x: torch.Tensor, n_rows: int, K: int,
               out_dtype: torch.dtype = torch.float16, block_n: int = 16,
               num_warps: int = 2, bias: torch.Tensor | None = None,
               resid: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ dequant(raw).T without materialising the weights -> (T, n_rows).

    bias (n_rows) and resid (T, n_rows) fp32, both optional and raw rows only,
    are added in the kernel's epilogue as resid + (y + bias)."""
    dtype = GGMLType(dtype)
    x2 = x.reshape(-1, K)
    T = x2.shape[0]
    N.require_device(x2)
    y = torch.empty((T, n_rows), dtype=torch.float32, device=x2.device)
    if n_rows == 0:
        return y.to(out_dtype)
    lib = N.load()
    with torch.cuda.device(x2.device):
        s = N.stream_ptr(x2.device)
        if isinstance(raw, T64Rows):
            if bias is not None or resid is not None:
                raise NotImplementedError("bias / resid epilogue on t64 windows")
            if raw.hi - raw.lo != n_rows or raw.K != K:
                raise ValueError(f"t64 window [{raw.lo}, {raw.hi}) x {raw.K} does not match {n_rows} x {K}")
            xf = x2.float().contiguous()
            for t0 in range(0, T, MAX_T64_T):
                t1 = min(T, t0 + MAX_T64_T)
                N.check(lib.nsx_t64_gemv(int(dtype), raw.buf.data_ptr(), raw.n_rows, K, raw.lo, raw.hi,
                                         xf[t0:t1].data_ptr(), N.DT_F32, t1 - t0, y[t0:t1].data_ptr(), s),
                        "t64_gemv")
        else:
            if raw.dtype != torch.uint8:
                raise TypeError(f"expected uint8 byte buffer, got {raw.dtype}")
            N.require_device(raw)
            be, bb = TYPE_LAYOUT[dtype] if dtype in TYPE_LAYOUT else (0, 0)
            if dtype not in N.BLOCK_TYPES:
                raise KeyError(dtype)
            need = n_rows * (K // be) * bb
            flat = raw.reshape(-1)
            if flat.numel() < need:
                raise ValueError(f"raw has {flat.numel()} bytes, {n_rows} x {K} {dtype.name} needs {need}")
            if not flat.is_contiguous():
                flat = flat.contiguous()
            xc = x2 if x2.is_contiguous() else x2.contiguous()
            for name, t, n in (("bias", bias, n_rows), ("resid", resid, T * n_rows)):
                if t is not None and (not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous()
                                      or t.numel() != n):
                    raise ValueError(f"{name} must be a contiguous fp32 device tensor of {n} elements")
            N.check(lib.nsx_fused_gemv_ex(int(dtype), flat.data_ptr(), n_rows, K, xc.data_ptr(),
                                          N.act_dtype_code(xc.dtype), T, y.data_ptr(),
                                          None if bias is None else bias.data_ptr(),
                                          None if resid is None else resid.data_ptr(), s), "fused_gemv")
    return y if out_dtype == torch.float32 else y.to(out_dtype)
