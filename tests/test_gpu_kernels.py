"""Parity of the HIP kernels with the CPU oracle (dequant bit-exact, GEMV 1e-3)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bit_mismatches, rel_max, to_np
from oracle import moe as OM
from oracle import quant as OQ

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3  # north-star bar (fp32 accumulate); the observed error is far smaller
GEMV_TIGHT = 2e-5


def _lib():
    from nurostream_amd import _native as N
    return N


def _mxfp4_all_exponents(rng):
    raw = rng.integers(0, 256, (256 * 4, 17), dtype=np.uint8)
    raw[:, 0] = np.repeat(np.arange(256, dtype=np.uint8), 4)
    return raw


def _q_special_d(rng, nb, bb):
    raw = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    specials = np.array([0x0000, 0x8000, 0x0001, 0x03ff, 0x0400, 0x3c00, 0xbc00, 0x7bff, 0xfbff, 0x0200],
                        dtype=np.uint16)
    d = rng.choice(specials, nb).astype(np.uint16)
    raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    return raw


@pytest.mark.parametrize("fmt", ["MXFP4", "Q4_0", "Q8_0", "Q4_K", "Q6_K"])
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_dequant_bit_exact(dev, fmt, offset):
    from nurostream_amd.compute.quant import dequantize
    rng = np.random.default_rng(7 + offset)
    t = getattr(OQ, fmt)
    be, bb = OQ.LAYOUT[t]
    if fmt == "MXFP4":
        raw = _mxfp4_all_exponents(rng)
    elif fmt == "Q4_K":
        raw = rng.integers(0, 256, (300, bb), dtype=np.uint8)
        raw[:150, 0:4] = _q_special_d(rng, 150, 4)[:, 0:4]
    elif fmt == "Q6_K":  # d sits at bytes 208:210
        raw = rng.integers(0, 256, (300, bb), dtype=np.uint8)
        raw[:150, 208:210] = _q_special_d(rng, 150, 2)
    else:
        raw = _q_special_d(rng, 777, bb)
    flat = raw.reshape(-1)
    buf = np.zeros(flat.size + 8, dtype=np.uint8)
    buf[offset:offset + flat.size] = flat
    gpu = torch.from_numpy(buf).to(dev)[offset:offset + flat.size]
    n = raw.shape[0] * be - 5  # truncated like the reference's n_elements
    expect = OQ.dequantize(flat, t, n)
    got = to_np(dequantize(gpu, t, n))
    assert got.shape == expect.shape
    bad = bit_mismatches(got, expect)
    if bad.size:
        i = bad[:8]
        blocks = raw[i // be]
        pytest.fail(f"{bad.size} mismatches at {i.tolist()}: got {got[i].tolist()} "
                    f"({[hex(v) for v in got.view(np.uint32)[i]]}) expected {expect[i].tolist()} "
                    f"({[hex(v) for v in expect.view(np.uint32)[i]]}); block head bytes "
                    f"{[b[:4].tolist() for b in blocks]}")
    for odt in (torch.float16, torch.bfloat16):
        g2 = dequantize(gpu, t, n, out_dtype=odt).cpu()
        ref = torch.from_numpy(expect).to(odt)  # torch's own float32 -> half rounding
        bad = bit_mismatches(g2.view(torch.int16).numpy().view(np.float16) if odt == torch.float16
                             else g2.float().numpy(),
                             ref.view(torch.int16).numpy().view(np.float16) if odt == torch.float16
                             else ref.float().numpy())
        assert bad.size == 0, (odt, bad[:8].tolist())


def test_mxfp4_reference_known_answer_input(dev):
    """The reference's MXFP4 KAT input (tests/test_gpt_oss.py:103-109): every exponent 0..253."""
    from nurostream_amd.compute.quant import dequantize
    rng = np.random.default_rng(42)
    raw = rng.integers(0, 256, (254, 17), dtype=np.uint8)
    raw[:, 0] = np.arange(254, dtype=np.uint8)
    expect = OQ.dequantize(raw.reshape(-1), OQ.MXFP4, 254 * 32)
    got = to_np(dequantize(torch.from_numpy(raw.reshape(-1)).to(dev), OQ.MXFP4, 254 * 32))
    assert bit_mismatches(got, expect).size == 0


def _gemv_case(fmt, rows, K, seed, e_lo=117, e_hi=123):
    from nurostream_amd import synth
    g = synth.generator(seed, "cpu")
    raw = synth.matrix_bytes(getattr(OQ, fmt), rows, K, g, "cpu", e_lo=e_lo, e_hi=e_hi)
    return raw.numpy()


@pytest.mark.parametrize("fmt,rows,K", [("MXFP4", 19, 2880), ("Q8_0", 19, 2880), ("MXFP4", 2880, 2880),
                                        ("Q4_0", 512, 4096), ("Q4_K", 1536, 4096), ("Q4_K", 96, 1536),
                                        ("Q4_0", 7, 64), ("MXFP4", 1, 32), ("Q6_K", 300, 4096),
                                        ("Q6_K", 33, 2816), ("Q6_K", 5, 256)])
@pytest.mark.parametrize("T", [1, 3, 16])
def test_fused_gemv_matches_oracle(dev, fmt, rows, K, T):
    from nurostream_amd.compute.kernels import can_fuse, fused_gemv
    t = getattr(OQ, fmt)
    raw = _gemv_case(fmt, rows, K, seed=rows + K + T)
    if T == 1:
        x = np.linspace(-1, 1, K, dtype=np.float32)[None, :]  # the reference's test input
    else:
        x = np.random.default_rng(T).standard_normal((T, K)).astype(np.float32)
    xt = torch.from_numpy(x).to(dev)
    assert can_fuse(t, xt)
    y = to_np(fused_gemv(torch.from_numpy(raw).to(dev), t, xt, rows, K, out_dtype=torch.float32))
    ref = OQ.gemv(raw, t, x, rows, K, f64=True)
    err = rel_max(y, ref)
    assert err < GEMV_TIGHT, err
    np.testing.assert_allclose(y, ref, atol=1e-4 * np.abs(ref).max() + 1e-6, rtol=1e-4)


@pytest.mark.parametrize("fmt,rows,K", [("Q4_0", 4096, 4096), ("Q4_0", 4097, 4096), ("MXFP4", 5000, 2880),
                                        ("Q4_0", 4095, 1024), ("Q8_0", 4096, 4096)])
def test_fused_gemv_one_token_paths_agree(dev, fmt, rows, K):
    """T = 1 runs on one of three kernel paths by shape and x: one row per wave
    in 16-wave workgroups (small Q4_0 / MXFP4 matrices, fp32 x 16-byte
    aligned), the 4-wave persistent grid with x in registers, or x staged per
    row from LDS (f16 or misaligned x). BASELINE config 1's shape, partial last
    workgroups and the fallbacks, against the float64 oracle; fp32 and f16
    views of one x must agree with the oracle alike."""
    from nurostream_amd.compute.kernels import fused_gemv
    t = getattr(OQ, fmt)
    raw = _gemv_case(fmt, rows, K, seed=rows * 7 + K)
    x = np.random.default_rng(rows).standard_normal((1, K)).astype(np.float16).astype(np.float32)
    ref = OQ.gemv(raw, t, x, rows, K, f64=True)
    w = torch.from_numpy(raw).to(dev)
    y = to_np(fused_gemv(w, t, torch.from_numpy(x).to(dev), rows, K, out_dtype=torch.float32))
    assert rel_max(y, ref) < GEMV_TIGHT
    y16 = to_np(fused_gemv(w, t, torch.from_numpy(x).to(dev).half(), rows, K, out_dtype=torch.float32))
    assert rel_max(y16, ref) < GEMV_TIGHT
    buf = torch.zeros(K + 1, dtype=torch.float32, device=dev)  # x at a 4-byte but not 16-byte aligned address
    buf[1:] = torch.from_numpy(x[0]).to(dev)
    ym = to_np(fused_gemv(w, t, buf[1:].reshape(1, K), rows, K, out_dtype=torch.float32))
    assert rel_max(ym, ref) < GEMV_TIGHT


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_fused_gemv_q6k_any_alignment(dev, offset):
    """Q6_K rows are 210 B per block, so rows start at any byte: the kernel's
    arithmetic does not depend on where the bytes sit (bitwise equal)."""
    from nurostream_amd.compute.kernels import fused_gemv
    rows, K = 77, 2816
    raw = _gemv_case("Q6_K", rows, K, seed=5)
    x = torch.from_numpy(np.random.default_rng(2).standard_normal((3, K)).astype(np.float32)).to(dev)
    base = torch.from_numpy(raw).to(dev)
    buf = torch.zeros(raw.size + 8, dtype=torch.uint8, device=dev)
    buf[offset:offset + raw.size] = base
    y0 = fused_gemv(base, OQ.Q6_K, x, rows, K, out_dtype=torch.float32)
    y1 = fused_gemv(buf[offset:offset + raw.size], OQ.Q6_K, x, rows, K, out_dtype=torch.float32)
    assert torch.equal(y0, y1)


@pytest.mark.parametrize("fmt,T,rows,K", [("Q8_0", 1, 300, 1024), ("Q6_K", 1, 300, 1024), ("MXFP4", 3, 300, 1024),
                                         ("Q4_K", 2, 300, 1024), ("Q8_0", 1, 40000, 256), ("Q6_K", 1, 20000, 256)])
def test_fused_gemv_bias_residual_epilogue(dev, fmt, T, rows, K):
    """nsx_fused_gemv_ex: resid + (x @ W.T + bias). The 20000 / 40000-row cases give every wave
    of the persistent grid several rows, so each row's bias and residual (loaded with its weights)
    must reach that row's epilogue."""
    from nurostream_amd.compute.kernels import fused_gemv
    t = getattr(OQ, fmt)
    raw = _gemv_case(fmt, rows, K, seed=9)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((T, K)).astype(np.float32)
    b = rng.standard_normal(rows).astype(np.float32)
    r = rng.standard_normal((T, rows)).astype(np.float32)
    raw_t, xt = torch.from_numpy(raw).to(dev), torch.from_numpy(x).to(dev)
    bt, rt = torch.from_numpy(b).to(dev), torch.from_numpy(r).to(dev)
    ref = r + (OQ.gemv(raw, t, x, rows, K, f64=True) + b)
    y = fused_gemv(raw_t, t, xt, rows, K, out_dtype=torch.float32, bias=bt, resid=rt)
    assert rel_max(to_np(y), ref) < GEMV_TIGHT
    plain = fused_gemv(raw_t, t, xt, rows, K, out_dtype=torch.float32)
    torch.testing.assert_close(y, rt + (plain + bt), rtol=0, atol=0)  # the same fp32 operations
    with pytest.raises(ValueError):
        fused_gemv(raw_t, t, xt, rows, K, out_dtype=torch.float32, bias=bt[:-1])


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_fused_gemv_half_activations(dev, xdt):
    from nurostream_amd.compute.kernels import fused_gemv
    rows, K = 64, 2880
    raw = _gemv_case("MXFP4", rows, K, seed=3)
    x = torch.randn(2, K).to(xdt)
    y = to_np(fused_gemv(torch.from_numpy(raw).to(dev), OQ.MXFP4, x.to(dev), rows, K, out_dtype=torch.float32))
    ref = OQ.gemv(raw, OQ.MXFP4, x.float().numpy(), rows, K, f64=True)
    assert rel_max(y, ref) < GEMV_TIGHT


@pytest.mark.parametrize("rows,K", [(2880, 2880), (100, 64), (64, 4096), (1, 32)])
def test_t64_roundtrip_and_gemv(dev, rows, K):
    from nurostream_amd.compute.kernels import T64Rows, fused_gemv, t64_pack
    raw = _gemv_case("MXFP4", rows, K, seed=rows * 3 + K, e_lo=0, e_hi=255)
    raw_t = torch.from_numpy(raw).to(dev)
    tiles = t64_pack(raw_t, OQ.MXFP4, rows, K)
    win = T64Rows(tiles, OQ.MXFP4, rows, K, 0, rows)
    back = win.to_gguf()
    assert torch.equal(back.cpu(), raw_t.cpu())
    # GEMV over sub-windows, including ones that do not start on a tile
    x = np.random.default_rng(1).standard_normal((2, K)).astype(np.float32)
    raw_n = _gemv_case("MXFP4", rows, K, seed=rows + 11)
    tiles = t64_pack(torch.from_numpy(raw_n).to(dev), OQ.MXFP4, rows, K)
    ref = OQ.gemv(raw_n, OQ.MXFP4, x, rows, K, f64=True)
    for lo, hi in [(0, rows), (rows // 3, rows), (min(5, rows - 1), max(min(70, rows), min(5, rows - 1) + 1))]:
        w = T64Rows(tiles, OQ.MXFP4, rows, K, lo, hi)
        y = to_np(fused_gemv(w, OQ.MXFP4, torch.from_numpy(x).to(dev), hi - lo, K, out_dtype=torch.float32))
        assert rel_max(y, ref[:, lo:hi]) < GEMV_TIGHT, (lo, hi)


@pytest.mark.parametrize("e_lo,e_hi,x_exp", [(0, 2, 100), (248, 252, -100), (117, 123, 0)])
def test_t64_gemv_extreme_scales(dev, e_lo, e_hi, x_exp):
    """Block-scaled MFMA over e8m0 scales at both ends of the range (2^-127 .. 2^127), with x
    scaled so that the float32 reference stays finite (its dequant overflows from e = 253 on with
    the larger codes): denormal-range weights, huge weights."""
    from helpers import MFMA_TOL
    from nurostream_amd.compute.kernels import T64Rows, fused_gemv, t64_pack
    rows, K = 128, 2880
    raw = _gemv_case("MXFP4", rows, K, seed=e_lo + 7, e_lo=e_lo, e_hi=e_hi)
    x = (np.random.default_rng(2).standard_normal((3, K)) * 2.0 ** x_exp).astype(np.float32)
    tiles = t64_pack(torch.from_numpy(raw).to(dev), OQ.MXFP4, rows, K)
    y = to_np(fused_gemv(T64Rows(tiles, OQ.MXFP4, rows, K, 0, rows), OQ.MXFP4, torch.from_numpy(x).to(dev), rows, K,
                         out_dtype=torch.float32))
    ref = OQ.gemv(raw, OQ.MXFP4, x, rows, K, f64=True)
    assert np.isfinite(ref).all() and np.isfinite(y).all()
    assert rel_max(y, ref) < MFMA_TOL


def test_t64_gemv_nan_scale_rows_are_non_finite(dev):
    """An e8m0 of 255 makes the reference's dequantized weights +-inf (quant.py:131-140), so its
    row products are non-finite; the block-scaled MFMA reads 255 as NaN: the same rows are
    non-finite and the other rows are unaffected."""
    from helpers import MFMA_TOL
    from nurostream_amd.compute.kernels import T64Rows, fused_gemv, t64_pack
    rows, K = 64, 256
    raw = _gemv_case("MXFP4", rows, K, seed=5).reshape(rows, K // 32, 17)
    bad = [3, 40]
    raw[bad, 2, 0] = 255
    raw[bad, 2, 1:] = 0x77  # codes 7 (LUT2 12): inf in the reference's float32 dequant
    raw = raw.reshape(-1)
    x = np.random.default_rng(3).standard_normal((1, K)).astype(np.float32)
    tiles = t64_pack(torch.from_numpy(raw).to(dev), OQ.MXFP4, rows, K)
    y = to_np(fused_gemv(T64Rows(tiles, OQ.MXFP4, rows, K, 0, rows), OQ.MXFP4, torch.from_numpy(x).to(dev), rows, K,
                         out_dtype=torch.float32))[0]
    with np.errstate(over="ignore", invalid="ignore"):
        ref = OQ.gemv(raw, OQ.MXFP4, x, rows, K)[0]
    assert not np.isfinite(ref[bad]).any() and not np.isfinite(y[bad]).any()
    ok = np.setdiff1d(np.arange(rows), bad)
    assert np.isfinite(y[ok]).all()
    assert rel_max(y[ok], ref[ok].astype(np.float64)) < MFMA_TOL


@pytest.mark.parametrize("T,n,resid,weight", [(1, 2880, True, False), (8, 2880, True, True), (3, 4096, False, True),
                                             (2, 100, True, True)])
def test_add_rmsnorm_matches_oracle(dev, T, n, resid, weight):
    """compute/ops.py:14-20 with the residual folded in (nsx_add_rmsnorm)."""
    from nurostream_amd.compute.ops import add_rms_norm
    g = torch.Generator().manual_seed(T * 7 + n)
    x = torch.randn(T, n, generator=g)
    r = torch.randn(T, n, generator=g) if resid else None
    w = torch.randn(n, generator=g) if weight else None
    y = add_rms_norm(x.to(dev), None if r is None else r.to(dev), None if w is None else w.to(dev), 1e-5)
    v = x.numpy() + (r.numpy() if resid else 0)
    ref = OM.rms_norm(v, None if w is None else w.numpy(), eps=1e-5)
    np.testing.assert_allclose(to_np(y), ref, rtol=2e-6, atol=2e-6)
    # in place (y aliases x), and the residual sum written back over x
    xd = x.to(dev)
    add_rms_norm(xd, None if r is None else r.to(dev), None if w is None else w.to(dev), 1e-5, out=xd)
    assert torch.equal(xd, y)
    xd, s = x.to(dev), torch.empty(T, n, device=dev)
    y2 = add_rms_norm(xd, None if r is None else r.to(dev), None if w is None else w.to(dev), 1e-5, sum_out=xd)
    assert torch.equal(y2, y)
    np.testing.assert_array_equal(to_np(xd), v.astype(np.float32))


@pytest.mark.parametrize("fmt,rows,K", [("Q8_0", 5120, 2880), ("Q8_0", 300, 4096), ("MXFP4", 700, 2880),
                                        ("Q4_0", 96, 4096), ("Q4_K", 64, 1536), ("Q6_K", 33, 2816),
                                        ("Q8_0", 40000, 256), ("Q4_0", 7, 64)])
@pytest.mark.parametrize("resid,weight", [(True, True), (False, True), (True, False)])
def test_fused_gemv_norm_equals_norm_then_gemv(dev, fmt, rows, K, resid, weight):
    """nsx_fused_gemv_norm (the block norm in the one-token GEMV's prologue) against
    nsx_add_rmsnorm followed by nsx_fused_gemv_ex: the same bits, norm and residual sum
    included (the prologue keeps add_rmsnorm_kernel's layout and sum order), and the
    product against the float64 oracle of the normed input. The 40000-row case gives
    every workgroup of the persistent grid several rows; only the first writes x + r."""
    from nurostream_amd.compute.kernels import fused_gemv, fused_gemv_norm
    from nurostream_amd.compute.ops import add_rms_norm
    t = getattr(OQ, fmt)
    raw = _gemv_case(fmt, rows, K, seed=rows + 3 * K)
    g = torch.Generator().manual_seed(rows + K)
    x = torch.randn(K, generator=g).to(dev)
    r = torch.randn(K, generator=g).to(dev) if resid else None
    w = (torch.rand(K, generator=g) + 0.5).to(dev) if weight else None
    b = torch.randn(rows, generator=g).to(dev)
    res = torch.randn(rows, generator=g).to(dev)
    raw_t = torch.from_numpy(raw).to(dev)
    s = torch.full((K,), float("nan"), device=dev) if resid else None
    y = fused_gemv_norm(raw_t, t, x, r, w, 1e-5, rows, K, sum_out=s, bias=b, resid=res)
    h = add_rms_norm(x.reshape(1, K), None if r is None else r.reshape(1, K), w, 1e-5)
    ref = fused_gemv(raw_t, t, h, rows, K, out_dtype=torch.float32, bias=b, resid=res.reshape(1, rows))
    assert torch.equal(y, ref)
    if resid:
        assert torch.equal(s, x + r)
    want = to_np(res) + (OQ.gemv(raw, t, to_np(h), rows, K, f64=True)[0] + to_np(b))
    assert rel_max(to_np(y)[0], want) < GEMV_TIGHT
    with pytest.raises(ValueError):  # the residual sum may not overwrite what other workgroups still read
        fused_gemv_norm(raw_t, t, x, r if resid else x.clone(), w, 1e-5, rows, K, sum_out=x)
