"""CPU restatement (numpy) of the reference's GGML dequantizers and fused GEMV.

TEST INFRASTRUCTURE ONLY. This module is the checker the parity tests, the
graft smoke check and bench.py's cpu_baseline leg compare the HIP kernels
against. No product code imports it.

Each function restates one reference function (paths relative to the
reference root, neurostream/compute/):
  dequant_q4_0   quant.py:118-126
  dequant_q4_k   quant.py:24-56  (+ get_scale_min_k4 index maths, triton_kernels.py:52-88)
  dequant_mxfp4  quant.py:129-140
  dequant_q8_0   quant.py:110-115
  dequant_q6_k   quant.py:84-107 (layout as in the Triton kernel, triton_kernels.py:97-143)
  dequantize     quant.py:153-184
  gemv           triton_kernels.py:199-228 semantics, computed the way the
                 reference's non-fused branch does it: dequantize, then x @ w.T
                 in float32 (blockffn.py:172-176, 203-207)

Pinning (see tests/test_oracle_quant.py):
  * MXFP4: all 256 exponents x 16 codes against an independent decoder
    (OCP e2m1 table x 2^(e-127), the convention of transformers'
    integrations/mxfp4.py:29-45,271-275) and against the reference's own
    known-answer input (tests/test_gpt_oss.py:103-109);
  * Q4_0 / Q4_K / Q8_0 / Q6_K: round trips through independent encoders that
    pack chosen (d, dmin, sub-scale, min, code) values into bytes, exhaustive
    over every 6-bit scale/min pattern of the Q4_K 12-byte field and over
    every 6-bit Q6_K code and int8 Q6_K scale, plus the reference's Q8_0 known
    answer arange(1, 33) (tests/test_tuning.py:104-133). The reference's tests
    hold no Q6_K vector; the Q6_K encoder follows ggml's published
    quantize_row_q6_K packing (ggml-quants.c, MIT), with scale index
    element // 16;
  * gemv: against float64 x @ dequant.T and brute force on tiny inputs.
"""
from __future__ import annotations

import numpy as np

# ggml type ids (format/gguf.py:19-35)
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, BF16, MXFP4 = 0, 1, 2, 8, 12, 14, 30, 39

LAYOUT = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34),
          Q4_K: (256, 144), Q6_K: (256, 210), MXFP4: (32, 17)}

# quant.py:137-139 -- ggml's doubled e2m1 table; code 8 is +0.0
MXFP4_LUT2 = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12],
                      dtype=np.float32)


def _f16_field(blocks: np.ndarray, lo: int) -> np.ndarray:
    """2-byte little-endian fp16 field -> float32 column (quant.py:19-21)."""
    return np.ascontiguousarray(blocks[:, lo:lo + 2]).view(np.float16).astype(np.float32)


def k_scales_mins(scales: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """get_scale_min_k4 for all 8 sub-blocks (quant.py:24-38)."""
    q = scales.astype(np.int32)
    d_lo = q[:, 0:4] & 63
    m_lo = q[:, 4:8] & 63
    d_hi = (q[:, 8:12] & 0x0F) | ((q[:, 0:4] >> 6) << 4)
    m_hi = (q[:, 8:12] >> 4) | ((q[:, 4:8] >> 6) << 4)
    sc = np.concatenate([d_lo, d_hi], axis=1).astype(np.float32)
    mn = np.concatenate([m_lo, m_hi], axis=1).astype(np.float32)
    return sc, mn


def dequant_q4_k(blocks: np.ndarray) -> np.ndarray:
    """Q4_K: d | dmin | scales[12] | qs[128]; value = (d*sc)*q - dmin*m (quant.py:41-56)."""
    nb = blocks.shape[0]
    d = _f16_field(blocks, 0)
    dmin = _f16_field(blocks, 2)
    sc, mn = k_scales_mins(blocks[:, 4:16])
    qs = blocks[:, 16:144].reshape(nb, 4, 32).astype(np.int32)
    q = np.stack([qs & 0x0F, qs >> 4], axis=2).reshape(nb, 8, 32).astype(np.float32)
    scale = (d * sc)[:, :, None]
    offset = (dmin * mn)[:, :, None]
    return (scale * q - offset).reshape(nb, 256).astype(np.float32)


def dequant_q4_0(blocks: np.ndarray) -> np.ndarray:
    """Q4_0: d | qs[16]; element j<16 = lo nibble - 8, j>=16 = hi nibble - 8 (quant.py:118-126)."""
    d = _f16_field(blocks, 0)
    qs = blocks[:, 2:18].astype(np.int32)
    q = np.concatenate([(qs & 0x0F) - 8, (qs >> 4) - 8], axis=1).astype(np.float32)
    return (d * q).astype(np.float32)


def dequant_q8_0(blocks: np.ndarray) -> np.ndarray:
    """Q8_0: d | qs[32] int8 (quant.py:110-115)."""
    d = _f16_field(blocks, 0)
    q = np.ascontiguousarray(blocks[:, 2:34]).view(np.int8).astype(np.float32)
    return (d * q).astype(np.float32)


def dequant_q6_k(blocks: np.ndarray) -> np.ndarray:
    """Q6_K: ql[128] | qh[64] | int8 scales[16] | d (quant.py:84-107).

    Each 128-element half h has four 32-wide lanes L; element l of lane L takes
    its low 4 bits from ql[64h + 32(L % 2) + l] (low nibble for L < 2, high
    for L >= 2), its high 2 bits from qh[32h + l] >> 2L, and is scaled by
    d * scales[8h + l // 16 + 2L]; value = d * sc * (q - 32).
    """
    nb = blocks.shape[0]
    ql = blocks[:, 0:128].reshape(nb, 2, 64).astype(np.int32)
    qh = blocks[:, 128:192].reshape(nb, 2, 32).astype(np.int32)
    sc = np.ascontiguousarray(blocks[:, 192:208]).view(np.int8).reshape(nb, 2, 8).astype(np.float32)
    d = _f16_field(blocks, 208)[:, :, None]  # (nb, 1, 1)
    half_of_lane = np.arange(32) // 16
    out = np.empty((nb, 2, 128), np.float32)
    for L in range(4):
        src = ql[:, :, 32 * (L % 2):32 * (L % 2) + 32]
        low = (src & 0x0F) if L < 2 else (src >> 4)
        q = low | (((qh >> (2 * L)) & 3) << 4)
        s = sc[:, :, half_of_lane + 2 * L]
        out[:, :, 32 * L:32 * L + 32] = (d * s) * (q - 32).astype(np.float32)
    return out.reshape(nb, 256)


def mxfp4_scale(e: np.ndarray) -> np.ndarray:
    """2^(e-128) built from raw float bits; e=0,1 are denormals, e=255 -> 2^127 (quant.py:131-134)."""
    e = e.astype(np.int64)
    bits = np.where(e < 2, np.int64(0x00200000) << e, (e - 1) << 23).astype(np.uint32)
    return bits.view(np.float32)


def dequant_mxfp4(blocks: np.ndarray) -> np.ndarray:
    """MXFP4: e8m0 | qs[16]; code j<16 = lo nibble, j>=16 = hi nibble (quant.py:129-140)."""
    scale = mxfp4_scale(blocks[:, :1])
    packed = blocks[:, 1:17]
    codes = np.concatenate([packed & 15, packed >> 4], axis=1)
    return (scale * MXFP4_LUT2[codes]).astype(np.float32)


_KERNELS = {MXFP4: dequant_mxfp4, Q4_K: dequant_q4_k, Q6_K: dequant_q6_k, Q8_0: dequant_q8_0,
            Q4_0: dequant_q4_0}


def dequantize(raw: np.ndarray, dtype: int, n_elements: int) -> np.ndarray:
    """Flat float32 expansion of `raw` uint8 bytes (quant.py:153-184)."""
    raw = np.asarray(raw)
    if raw.dtype != np.uint8:
        raise TypeError(f"expected uint8 byte buffer, got {raw.dtype}")
    raw = raw.reshape(-1)
    if dtype == F32:
        return raw.view(np.float32)[:n_elements].copy()
    if dtype == F16:
        return raw.view(np.float16)[:n_elements].astype(np.float32)
    if dtype == BF16:
        u = raw.view(np.uint16)[:n_elements].astype(np.uint32) << 16
        return u.view(np.float32).copy()
    kern = _KERNELS.get(dtype)
    if kern is None:
        raise NotImplementedError(f"no dequant kernel for ggml type {dtype}")
    be, bb = LAYOUT[dtype]
    nb = raw.size // bb
    flat = kern(raw[: nb * bb].reshape(nb, bb)).reshape(-1)
    return flat[:n_elements]


def dequant_rows(raw: np.ndarray, dtype: int, n_rows: int, K: int) -> np.ndarray:
    return dequantize(raw, dtype, n_rows * K).reshape(n_rows, K)


def gemv(raw: np.ndarray, dtype: int, x: np.ndarray, n_rows: int, K: int,
         f64: bool = False) -> np.ndarray:
    """y = x @ dequant(raw).T; x is (T, K). float32 like the reference's torch path."""
    w = dequant_rows(raw, dtype, n_rows, K)
    x = np.asarray(x).reshape(-1, K)
    if f64:
        return x.astype(np.float64) @ w.astype(np.float64).T
    return (x.astype(np.float32) @ w.T).astype(np.float32)


def row_bytes(dtype: int, K: int) -> int:
    be, bb = LAYOUT[dtype]
    if K % be:
        raise ValueError(f"K={K} is not a multiple of the block size {be}")
    return (K // be) * bb
