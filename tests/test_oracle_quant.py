"""Pins the numpy oracle's dequantizers and GEMV (CPU only).

Every check here reaches the oracle's result by a second route: an
independent decoder or encoder written from the format's bit layout, a
third-party decoder present in this container (torch's float8_e8m0fnu,
transformers' FP4_VALUES table), a float64 closed form, or one of the
reference's own known answers.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import moe as OM
from oracle import quant as OQ


def _e2m1(code: int) -> float:
    """OCP FP4 E2M1 from its bits: sign | 2-bit exponent (bias 1) | 1-bit mantissa."""
    s = -1.0 if code & 8 else 1.0
    e = (code >> 1) & 3
    m = code & 1
    mag = (m * 0.5) if e == 0 else (1.0 + 0.5 * m) * 2.0 ** (e - 1)
    return s * mag


def _mx_block(e: int, codes: np.ndarray) -> np.ndarray:
    """Pack 32 4-bit codes (element j<16 -> low nibble of byte j, j>=16 -> high nibble of byte j-16)."""
    qs = (codes[:16] & 15) | ((codes[16:] & 15) << 4)
    return np.concatenate([[e], qs]).astype(np.uint8)


# element j and element j + 16 share a byte: distinct halves catch a nibble swap
_CODES32 = np.concatenate([np.arange(16), np.arange(15, -1, -1)])


@np.errstate(over="ignore")  # e >= 254 overflows float32 for the larger codes, as in the reference
def test_mxfp4_every_exponent_and_code():
    """All 256 exponent bytes x 16 codes against value = e2m1(code) * 2^(e-127)."""
    codes = _CODES32
    blocks = np.stack([_mx_block(e, codes) for e in range(256)])
    got = OQ.dequantize(blocks.reshape(-1), OQ.MXFP4, 256 * 32).reshape(256, 32)
    for e in range(255):
        want = np.array([_e2m1(int(c)) * 2.0 ** (e - 127) for c in codes]).astype(np.float32)
        np.testing.assert_array_equal(np.abs(got[e]), np.abs(want), err_msg=f"e={e}")
        assert np.array_equal(np.signbit(got[e]), np.signbit(want) & (want != 0)), e  # code 8 is +0.0
    # e = 255: the reference keeps 2^127 * doubled table (no NaN): 2^127 * 2 * e2m1 in float32
    want255 = np.array([np.float32(2.0 ** 127) * np.float32(2 * _e2m1(int(c))) for c in codes], dtype=np.float32)
    np.testing.assert_array_equal(np.abs(got[255]), np.abs(want255))


def test_mxfp4_scale_matches_torch_e8m0():
    """The scale factor against torch's own float8_e8m0fnu decoding (2^(e-127); NaN at 255)."""
    torch = pytest.importorskip("torch")
    e = np.arange(255, dtype=np.uint8)
    t = torch.from_numpy(e).view(torch.float8_e8m0fnu).float().numpy()
    # oracle scale is 2^(e-128) (ggml stores half the OCP scale and doubles the table)
    np.testing.assert_array_equal(OQ.mxfp4_scale(e.reshape(-1, 1)).reshape(-1) * np.float32(2), t)


def test_mxfp4_table_matches_transformers():
    """transformers' FP4_VALUES (true e2m1) times two is the oracle's doubled table (up to the sign of zero)."""
    M = pytest.importorskip("transformers.integrations.mxfp4")
    np.testing.assert_array_equal(np.abs(np.array(M.FP4_VALUES, np.float32) * 2), np.abs(OQ.MXFP4_LUT2))


@np.errstate(over="ignore")
def test_mxfp4_reference_known_answer_input():
    """The reference's KAT input (tests/test_gpt_oss.py:103-109: seed 42, exponents 0..253)
    against the independent decoder (the reference compares with gguf, absent here)."""
    rng = np.random.default_rng(42)
    raw = rng.integers(0, 256, (254, 17), dtype=np.uint8)
    raw[:, 0] = np.arange(254, dtype=np.uint8)
    got = OQ.dequantize(raw.reshape(-1), OQ.MXFP4, 254 * 32).reshape(254, 32)
    lo, hi = raw[:, 1:] & 15, raw[:, 1:] >> 4
    codes = np.concatenate([lo, hi], axis=1)
    table = np.array([_e2m1(c) for c in range(16)])
    want = (table[codes] * np.exp2(raw[:, :1].astype(np.float64) - 127)).astype(np.float32)
    np.testing.assert_array_equal(np.abs(got), np.abs(want))


_F16_SPECIAL = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF, 0x3555],
                        dtype=np.uint16)


def test_q4_0_every_code_and_special_scales():
    """d * (q - 8) for every code and fp16 d incl. +-0, subnormals and +-max (float64 product is exact)."""
    codes = _CODES32
    blocks = []
    for dbits in _F16_SPECIAL:
        qs = (codes[:16] | (codes[16:] << 4)).astype(np.uint8)
        blocks.append(np.concatenate([np.array([dbits], np.uint16).view(np.uint8), qs]))
    blocks = np.stack(blocks)
    got = OQ.dequantize(blocks.reshape(-1), OQ.Q4_0, len(blocks) * 32).reshape(-1, 32)
    d = _F16_SPECIAL.view(np.float16).astype(np.float64)
    want = (d[:, None] * (codes[None, :] - 8)).astype(np.float32)
    np.testing.assert_array_equal(got, want)


def test_q8_0_reference_known_answer():
    """Q8_0 row with d = 1.0 and bytes 1..32 (tests/test_tuning.py:104-133): values 1..32; a
    dot with ones is 528 (tests/test_tuning.py:135-153)."""
    row = np.concatenate([np.array([1.0], np.float16).view(np.uint8), np.arange(1, 33, dtype=np.uint8)])
    raw = np.tile(row, 4)
    np.testing.assert_array_equal(OQ.dequant_rows(raw, OQ.Q8_0, 4, 32), np.tile(np.arange(1, 33, dtype=np.float32), (4, 1)))
    y = OQ.gemv(raw, OQ.Q8_0, np.ones((2, 32), np.float32), 4, 32)
    np.testing.assert_array_equal(y, np.full((2, 4), 528.0, np.float32))
    # signed bytes: 0x80..0xff are -128..-1
    b = np.arange(112, 144)
    row2 = np.concatenate([np.array([0.5], np.float16).view(np.uint8), b.astype(np.uint8)])
    np.testing.assert_array_equal(OQ.dequantize(row2, OQ.Q8_0, 32), (0.5 * np.where(b >= 128, b - 256, b)).astype(np.float32))


def _q4k_pack_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Pack eight 6-bit (scale, min) pairs into the 12-byte Q4_K field, written from ggml's
    layout description as an encoder: bytes 0-3 hold sc[0..3] (bits 0-5) and the top two bits
    of sc[4..7] (bits 6-7); bytes 4-7 hold mn[0..3] and the top bits of mn[4..7]; bytes 8-11 hold
    the low nibbles of sc[4..7] (low) and mn[4..7] (high)."""
    b = np.zeros(12, np.uint8)
    for i in range(4):
        b[i] = (sc[i] & 63) | ((sc[i + 4] >> 4) << 6)
        b[i + 4] = (mn[i] & 63) | ((mn[i + 4] >> 4) << 6)
        b[i + 8] = (sc[i + 4] & 15) | ((mn[i + 4] & 15) << 4)
    return b


def _q4k_block(d: float, dmin: float, sc, mn, codes) -> np.ndarray:
    """Encode element j (sub-block s = j // 32, l = j % 32) into nibble s % 2 of qs[(s // 2) * 32 + l]."""
    qs = np.zeros(128, np.uint8)
    for j in range(256):
        s, l = divmod(j, 32)
        qs[(s // 2) * 32 + l] |= (int(codes[j]) & 15) << (4 * (s % 2))
    head = np.array([d, dmin], np.float16).view(np.uint8)
    return np.concatenate([head, _q4k_pack_scales(np.asarray(sc), np.asarray(mn)), qs])


def test_q4_k_scale_field_exhaustive():
    """Every 6-bit value at every one of the 8 scale slots and 8 min slots decodes back."""
    for v in range(64):
        for slot in range(8):
            sc = np.full(8, 17, np.int64)
            mn = np.full(8, 42, np.int64)
            sc[slot] = v
            mn[(slot + 3) % 8] = 63 - v
            got_sc, got_mn = OQ.k_scales_mins(_q4k_pack_scales(sc, mn)[None, :])
            np.testing.assert_array_equal(np.asarray(got_sc).reshape(-1), sc, err_msg=f"v={v} slot={slot}")
            np.testing.assert_array_equal(np.asarray(got_mn).reshape(-1), mn, err_msg=f"v={v} slot={slot}")


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q4_k_values_from_encoder(seed):
    """(d*sc)*q - dmin*m with one float32 rounding, blocks built by the encoder above."""
    rng = np.random.default_rng(seed)
    blocks, want = [], []
    for b in range(8):
        d = np.float16(rng.choice([0.0, 2.0 ** -24, 0.0078125, 1.5, 65504.0, -0.25]))
        dmin = np.float16(rng.choice([0.0, 2.0 ** -20, 0.001, 3.0]))
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        codes = rng.integers(0, 16, 256)
        blocks.append(_q4k_block(float(d), float(dmin), sc, mn, codes))
        s = np.arange(256) // 32
        exact = (float(d) * sc[s]) * codes - float(dmin) * mn[s]
        want.append(exact.astype(np.float32))
    got = OQ.dequantize(np.concatenate(blocks), OQ.Q4_K, 8 * 256).reshape(8, 256)
    np.testing.assert_array_equal(got, np.stack(want))


def _q6k_block(dbits: int, scales: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """Pack 256 6-bit codes and 16 int8 scales the way ggml's quantize_row_q6_K
    writes them: per 128-element half, element l, l+32, l+64, l+96 (l < 32)
    share qh[l] (2 bits each, in that order from bit 0) and element l / l+64
    (l+32 / l+96) share ql[l] (ql[l+32]) as low / high nibble. Scale s covers
    elements 16s .. 16s+15."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for half in range(2):
        c = codes[128 * half:128 * half + 128].astype(np.int64)
        for l in range(32):
            ql[64 * half + l] = (c[l] & 15) | ((c[l + 64] & 15) << 4)
            ql[64 * half + l + 32] = (c[l + 32] & 15) | ((c[l + 96] & 15) << 4)
            qh[32 * half + l] = ((c[l] >> 4) | ((c[l + 32] >> 4) << 2) | ((c[l + 64] >> 4) << 4)
                                 | ((c[l + 96] >> 4) << 6))
    return np.concatenate([ql, qh, scales.astype(np.int8).view(np.uint8),
                           np.array([dbits], np.uint16).view(np.uint8)])


def _q6k_expected(dbits: int, scales: np.ndarray, codes: np.ndarray) -> np.ndarray:
    d = float(np.array([dbits], np.uint16).view(np.float16)[0])
    s = scales.astype(np.float64)[np.arange(256) // 16]
    return (d * s * (codes.astype(np.float64) - 32)).astype(np.float32)  # exact: <= 23 significant bits


def test_q6_k_every_code_and_scale():
    """Every 6-bit code at every position class and every int8 scale value, against the
    independent packer and value = d * scales[e // 16] * (code - 32)."""
    rng = np.random.default_rng(11)
    all_scales = np.arange(-128, 128)
    blocks, want = [], []
    for i in range(16):  # 16 blocks x 16 scales = all 256 int8 values
        sc = all_scales[16 * i:16 * i + 16][rng.permutation(16)]
        # lane offsets 13 (e // 32): elements 32 or 64 apart (which share ql / qh bytes) get
        # different nibbles; over the 16 blocks every code lands in every (half, lane) class
        e = np.arange(256)
        codes = (e + 13 * (e // 32) + 17 * i) % 64
        dbits = int(_F16_SPECIAL[i % len(_F16_SPECIAL)])
        blocks.append(_q6k_block(dbits, sc, codes))
        want.append(_q6k_expected(dbits, sc, codes))
    got = OQ.dequantize(np.concatenate(blocks), OQ.Q6_K, 16 * 256).reshape(16, 256)
    np.testing.assert_array_equal(got, np.stack(want))
    # the sign of zero follows the float32 product order d * sc * 0 (as in the reference)
    assert np.array_equal(np.signbit(got), np.signbit(np.stack(want)))


def test_q6_k_random_blocks_round_trip():
    """Random codes, scales and d: decode(pack(c, s, d)) == d * s[e // 16] * (c - 32)."""
    rng = np.random.default_rng(12)
    blocks, want = [], []
    for _ in range(40):
        codes = rng.integers(0, 64, 256)
        sc = rng.integers(-128, 128, 16)
        dbits = int(np.array([abs(rng.normal(0, 2 ** -10))], np.float16).view(np.uint16)[0])
        blocks.append(_q6k_block(dbits, sc, codes))
        want.append(_q6k_expected(dbits, sc, codes))
    got = OQ.dequantize(np.concatenate(blocks), OQ.Q6_K, 40 * 256 - 3)
    np.testing.assert_array_equal(got, np.concatenate(want)[:40 * 256 - 3])


def test_dequantize_dispatch_errors():
    """The reference dispatcher's error contract (quant.py:153-184)."""
    with pytest.raises(TypeError):
        OQ.dequantize(np.zeros(34, np.int8), OQ.Q8_0, 32)
    with pytest.raises(NotImplementedError):
        OQ.dequantize(np.zeros(176, np.uint8), 13, 256)  # Q5_K: no kernel on this path
    # truncation to n_elements
    assert OQ.dequantize(np.zeros(34 * 2, np.uint8), OQ.Q8_0, 40).shape == (40,)


@pytest.mark.parametrize("fmt", ["MXFP4", "Q4_0", "Q8_0", "Q4_K", "Q6_K"])
def test_gemv_matches_float64_closed_form(fmt):
    """oracle.gemv (float32, the reference's non-fused torch path) within fp32 accumulation of
    float64 x @ W^T over independently decoded W."""
    t = getattr(OQ, fmt)
    be, bb = OQ.LAYOUT[t]
    rows, K = 19, 512 if fmt not in ("Q4_K", "Q6_K") else 1024
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 256, rows * (K // be) * bb, dtype=np.uint8).reshape(-1, bb)
    if fmt == "MXFP4":
        raw[:, 0] = rng.integers(117, 124, raw.shape[0])
    elif fmt in ("Q4_0", "Q8_0"):
        raw[:, 0:2] = np.abs(rng.normal(0, 0.02, raw.shape[0])).astype(np.float16).view(np.uint8).reshape(-1, 2)
    elif fmt == "Q6_K":
        raw[:, 208:210] = np.abs(rng.normal(0, 2 ** -10, raw.shape[0])).astype(np.float16).view(np.uint8).reshape(-1, 2)
    else:
        raw[:, 0:4] = np.abs(rng.normal(0, 2 ** -8, (raw.shape[0], 2))).astype(np.float16).view(np.uint8).reshape(-1, 4)
    x = np.linspace(-1, 1, K, dtype=np.float32)[None, :]  # the reference's test input
    y = OQ.gemv(raw.reshape(-1), t, x, rows, K)
    w64 = OQ.dequant_rows(raw.reshape(-1), t, rows, K).astype(np.float64)
    ref = x.astype(np.float64) @ w64.T
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-4 * np.abs(ref).max())


@pytest.mark.parametrize("block_rows", [1, 7, 8, 64, 4096])
def test_stream_linear_block_invariance(block_rows):
    """Row-block decomposition leaves the result unchanged (tests/test_gpt_oss.py:176-192)."""
    rng = np.random.default_rng(5)
    rows, K = 67, 256
    raw = rng.integers(0, 256, rows * (K // 32) * 17, dtype=np.uint8).reshape(-1, 17)
    raw[:, 0] = rng.integers(117, 124, raw.shape[0])
    x = rng.standard_normal((3, K)).astype(np.float32)
    whole = OQ.gemv(raw.reshape(-1), OQ.MXFP4, x, rows, K, f64=True)
    got = OM.stream_linear(raw.reshape(-1), OQ.MXFP4, x, rows, K, block_rows)
    np.testing.assert_allclose(got, whole, rtol=1e-5, atol=1e-5 * np.abs(whole).max())
    with pytest.raises(ValueError):
        OM.stream_linear(raw.reshape(-1), OQ.MXFP4, x, rows, K, 0)
