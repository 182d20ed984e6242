"""The C-ABI library loads and exports what include/nurostream_amd.h declares (CPU only).

Only host-side entry points (sizes, version, argument validation that
returns before any HIP call) are called here; compute calls need a GPU.
"""
from __future__ import annotations

import ctypes as C
import subprocess

import pytest

from nurostream_amd import _native as N
from nurostream_amd.format.gguf import GGMLType


@pytest.fixture(scope="module")
def lib():
    if not N.LIB_PATH.exists():
        from nurostream_amd import build
        build.build()
    return N.load()


def test_every_header_function_is_exported(lib):
    names = N.header_functions()
    assert len(names) >= 12, names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the ctypes binding covers every one of them
    assert sorted(N._SIGS) == names


def test_exported_symbols_are_the_header_set(lib):
    """nm: the .so exports no other nsx_* entry point than the header declares."""
    out = subprocess.run(["nm", "-D", "--defined-only", str(N.LIB_PATH)], capture_output=True, text=True, check=True)
    exported = sorted({ln.split()[-1] for ln in out.stdout.splitlines() if ln.split()[-1].startswith("nsx_")})
    assert exported == N.header_functions()


def test_abi_version_and_error_string(lib):
    assert lib.nsx_abi_version() == 3
    assert isinstance(lib.nsx_last_error(), bytes)


def test_t64_sizes(lib):
    # 64-row tiles: qs 1024 B per (tile, 32-column block) + e8m0 scales, rows padded to 64
    per = lib.nsx_t64_bytes(int(GGMLType.MXFP4), 2880, 2880)
    assert per >= 2880 * 90 * 17
    assert per < 2880 * 90 * 17 * 1.01
    assert lib.nsx_t64_bytes(int(GGMLType.MXFP4), 1, 32) > 0
    assert lib.nsx_t64_bytes(int(GGMLType.Q4_K), 64, 256) < 0  # MXFP4 only
    assert lib.nsx_t64_bytes(int(GGMLType.MXFP4), 64, 33) < 0  # K must be whole blocks


def _gptoss_layer(layout=N.LAYOUT_T64):
    L = N.MoeLayerC()
    L.ggml_type = int(GGMLType.MXFP4)
    L.layout = layout
    L.n_expert, L.top_k, L.n_embd, L.n_ff = 128, 4, 2880, 2880
    L.router_mode, L.act, L.alpha, L.limit = N.ROUTE_GPTOSS, N.ACT_CLAMPED_SWIGLU, 1.702, 7.0
    L.router_w = 1  # never dereferenced by the host-side checks
    L.router_dtype = int(GGMLType.BF16)
    L.gate_base = L.up_base = L.down_base = 1
    L.gate_stride = L.up_stride = L.down_stride = 1 << 22
    return L


def test_workspace_bytes(lib):
    L = _gptoss_layer()
    w1 = lib.nsx_moe_workspace_bytes(C.byref(L), 1)
    w8 = lib.nsx_moe_workspace_bytes(C.byref(L), 8)
    assert 0 < w1 < w8 < 64 << 20
    L.top_k = 0
    assert lib.nsx_moe_workspace_bytes(C.byref(L), 1) < 0


def test_workspace_bytes_by_dispatch(lib):
    """Grouped passes hold at most 4096 pairs: the workspace stops growing there."""
    L = _gptoss_layer()
    L.dispatch = N.DISPATCH_GROUPED
    w8, w1024, w4096 = (lib.nsx_moe_workspace_bytes(C.byref(L), T) for T in (8, 1024, 4096))
    assert 0 < w8 < w1024 == w4096
    L.dispatch = N.DISPATCH_PAIRS
    assert lib.nsx_moe_workspace_bytes(C.byref(L), 8) < w8  # no sort buffers or per-pair outputs
    L.dispatch = 9
    assert lib.nsx_moe_workspace_bytes(C.byref(L), 8) < 0
    L.dispatch = N.DISPATCH_GROUPED  # grouped needs t64, or stacked aligned Q4_K rows
    L.layout = N.LAYOUT_GGUF
    assert lib.nsx_moe_workspace_bytes(C.byref(L), 8) < 0
    assert b"grouped" in lib.nsx_last_error()
    L.ggml_type = int(GGMLType.Q4_K)
    L.n_embd, L.n_ff = 4096, 1536
    L.gate_stride = L.up_stride = L.down_stride = 1536 * 2304
    L.gate_base = L.up_base = L.down_base = 1 << 20
    wq = lib.nsx_moe_workspace_bytes(C.byref(L), 8)
    L.dispatch = N.DISPATCH_PAIRS
    wp = lib.nsx_moe_workspace_bytes(C.byref(L), 8)
    a8_h, a8_a = 8 * (4096 // 64 * 176), 32 * (1536 // 64 * 176)  # int8 terms: 8 tokens of h, 32 activations
    assert wp >= a8_a and wq >= wp + a8_h  # pairs: the activations' terms; grouped: also h's
    L.dispatch = N.DISPATCH_MFMA  # the matrix-core terms in their place
    terms = 8 * (4 * 4096 + 4096 // 8 + 16) + 32 * (4 * 1536 + 1536 // 8 + 16)
    assert lib.nsx_moe_workspace_bytes(C.byref(L), 8) >= wq - a8_h - a8_a + terms
    L.down_base = (1 << 20) + 8  # not 16-byte aligned: no Q4_K fast path, so no grouping
    assert lib.nsx_moe_workspace_bytes(C.byref(L), 8) < 0
    assert b"MFMA" in lib.nsx_last_error()
    L.dispatch = N.DISPATCH_GROUPED
    assert lib.nsx_moe_workspace_bytes(C.byref(L), 8) < 0


def test_validation_errors_return_codes(lib):
    # unsupported block type: NotImplemented, with a message
    rc = lib.nsx_dequantize(13, None, 176, 256, None, N.DT_F32, None)  # Q5_K
    assert rc == N.ENOTIMPL and b"Q6_K" in lib.nsx_last_error()
    rc = lib.nsx_fused_gemv(13, None, 1, 256, None, N.DT_F32, 1, None, None)
    assert rc == N.ENOTIMPL
    rc = lib.nsx_dequantize(int(GGMLType.Q8_0), None, 34, 64, None, N.DT_F32, None)
    assert rc == N.EINVAL  # more elements than blocks
    # router: top_k above n_expert
    rc = lib.nsx_router_topk(None, 1, 64, None, int(GGMLType.F32), None, 4, 5, N.ROUTE_GPTOSS, None, None, None, None)
    assert rc == N.EINVAL
    # layer phase out of range
    L = _gptoss_layer()
    rc = lib.nsx_moe_phase(C.byref(L), 7, None, 1, None, None, None, None, 0, None)
    assert rc == N.EINVAL
    with pytest.raises(ValueError):
        N.check(rc)


def test_static_workspace_limit(lib):
    """nsx_moe_forward_static takes no workspace: a call whose workspace would
    exceed the library's static array is refused on the host, before any HIP
    call (the pointers below are never dereferenced)."""
    L = _gptoss_layer()
    cap = N.STATIC_WORKSPACE_BYTES
    assert lib.nsx_moe_workspace_bytes(C.byref(L), 128) <= cap  # config 3 (T=128, grouped) fits
    T = 1024  # one grouped pass of 4096 pairs: per-pair outputs alone are 47 MB
    assert lib.nsx_moe_workspace_bytes(C.byref(L), T) > cap
    rc = lib.nsx_moe_forward_static(C.byref(L), 1, T, 1, 1, 1, None)
    assert rc == N.EINVAL and b"static workspace" in lib.nsx_last_error()
    with pytest.raises(ValueError):
        N.check(rc)
    rc = lib.nsx_moe_forward_static(C.byref(L), None, 1, 1, 1, 1, None)
    assert rc == N.EINVAL and b"null" in lib.nsx_last_error()


def test_moe_layer_rejects_bad_outputs():
    """MoELayer checks out / ids / weights before the native call writes
    through their pointers (shape, dtype, contiguity, device)."""
    import torch

    from nurostream_amd.moe.fused import MoELayer
    lay = MoELayer.__new__(MoELayer)
    lay.device, lay.n_embd, lay.top_k = torch.device("cpu"), 16, 2
    good = (torch.empty(3, 16), torch.empty(3, 2, dtype=torch.int32), torch.empty(3, 2))
    lay._check_buffers(3, *good)
    bad = [(torch.empty(3, 17), good[1], good[2]),
           (good[0], torch.empty(3, 2, dtype=torch.int64), good[2]),
           (good[0], good[1], torch.empty(2, 3).t()),
           (torch.empty(16, 3).t(), good[1], good[2]),
           (good[0], good[1], torch.empty(3, 2, dtype=torch.float16))]
    for out, ids, w in bad:
        with pytest.raises(ValueError):
            lay._check_buffers(3, out, ids, w)


def test_forward_norm_validation(lib):
    """nsx_moe_forward_norm folds the block norm into the router for t64 layers
    below 16 tokens (NotImplemented otherwise, so callers fall back), and
    refuses an x_out that overlaps x or r -- all checked on the host before any
    HIP call (the pointers below are never dereferenced)."""
    L = _gptoss_layer()
    args = lambda T, x_out: (C.byref(L), 1 << 20, 2 << 20, None, 1e-5, T, x_out, 4 << 20, 5 << 20, 6 << 20,  # noqa
                             7 << 20, 1 << 30, None)
    assert lib.nsx_moe_forward_norm(*args(16, 3 << 20)) == N.ENOTIMPL
    assert b"router" in lib.nsx_last_error()
    assert lib.nsx_moe_forward_norm(*args(1, (1 << 20) + 4)) == N.EINVAL
    assert b"overlaps" in lib.nsx_last_error()
    assert lib.nsx_moe_forward_norm(*args(1, (2 << 20) - 4)) == N.EINVAL
    L.layout = N.LAYOUT_GGUF
    assert lib.nsx_moe_forward_norm(*args(1, 3 << 20)) == N.ENOTIMPL


def test_forward_addnorm_validation(lib):
    """nsx_moe_forward_addnorm refuses an h_out that overlaps x or x_out and an x_out
    that overlaps x without being it -- checked on the host before any HIP call (the
    pointers below are never dereferenced)."""
    L = _gptoss_layer()
    T, row = 4, 4 * 2880 * 4
    args = lambda x, x_out, h_out: (C.byref(L), 1 << 20, T, x, None, 1e-5, x_out, h_out, 5 << 20, 6 << 20,  # noqa
                                    7 << 20, 1 << 30, None)
    x = 2 << 20
    assert lib.nsx_moe_forward_addnorm(*args(x, x, x + row // 2)) == N.EINVAL  # h_out over x
    assert b"h_out" in lib.nsx_last_error()
    assert lib.nsx_moe_forward_addnorm(*args(x, x + 4, 3 << 20)) == N.EINVAL  # x_out overlapping x, not x
    assert lib.nsx_moe_forward_addnorm(*args(x, 3 << 20, (3 << 20) + 8)) == N.EINVAL  # h_out over x_out


def test_gemv_norm_overlap_validation(lib):
    """nsx_fused_gemv_norm: workgroup 0 writes s and every workgroup its rows of y
    while the others still read x, r and resid, so s may overlap none of x, r,
    resid, y; y none of x, r; and y is resid exactly or apart from it -- byte
    ranges, checked on the host before any HIP call (the pointers below are
    never dereferenced)."""
    t, n_rows, K = int(GGMLType.Q8_0), 64, 256
    x, r, resid, y, s = 1 << 20, 2 << 20, 3 << 20, 4 << 20, 5 << 20

    def call(s=s, y=y, resid=resid, r=r):
        return lib.nsx_fused_gemv_norm(t, 6 << 20, n_rows, K, x, r, None, 1e-5, s, y, None, resid, None)

    for bad in (dict(s=x + 4), dict(s=x - 4 * K + 4), dict(s=r + 512), dict(s=resid + 8), dict(s=y + 16),
                dict(y=x + 1000), dict(y=r - 4 * n_rows + 4), dict(y=resid + 4), dict(resid=y - 4)):
        assert call(**bad) == N.EINVAL, bad
    assert b"overlap" in lib.nsx_last_error() or b"resid" in lib.nsx_last_error()
