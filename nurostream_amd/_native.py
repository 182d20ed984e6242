"""ctypes binding of libnsx.so (the C ABI declared in include/nurostream_amd.h).

The library is the only compute path for quantized weights: if it is missing,
or no GPU is present, the product functions raise instead of falling back to
a CPU implementation.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

from .format.gguf import GGMLType

LIB_PATH = Path(__file__).resolve().parent / "libnsx.so"
HEADER = Path(__file__).resolve().parents[1] / "include" / "nurostream_amd.h"

# status codes (nurostream_amd.h)
OK, EINVAL, ETYPE, ENOTIMPL, EHIP, EKERNEL, EIO, ETIMEDOUT = 0, 1, 2, 3, 4, 5, 6, 7
READ_DIRECT = 1
DT_F32, DT_F16, DT_BF16 = 0, 1, 2
LAYOUT_GGUF, LAYOUT_T64 = 0, 1
ROUTE_GPTOSS, ROUTE_QWEN3 = 0, 1
DISPATCH_AUTO, DISPATCH_PAIRS, DISPATCH_GROUPED, DISPATCH_MFMA = 0, 1, 2, 3
ACT_CLAMPED_SWIGLU, ACT_SILU_MUL = 0, 1

BLOCK_TYPES = frozenset({GGMLType.Q4_0, GGMLType.Q8_0, GGMLType.Q4_K, GGMLType.Q6_K, GGMLType.MXFP4})

_p = C.c_void_p
_i64 = C.c_int64
_i = C.c_int


class MoeLayerC(C.Structure):
    """nsx_moe_layer (field order and types follow the header)."""

    _fields_ = [
        ("ggml_type", C.c_int32), ("layout", C.c_int32), ("n_expert", C.c_int32),
        ("top_k", C.c_int32), ("n_embd", C.c_int32), ("n_ff", C.c_int32),
        ("router_mode", C.c_int32), ("act", C.c_int32), ("alpha", C.c_float),
        ("limit", C.c_float), ("router_w", _p), ("router_dtype", C.c_int32),
        ("dispatch", C.c_int32), ("router_bias", _p), ("gate_ptrs", _p),
        ("up_ptrs", _p), ("down_ptrs", _p), ("gate_bias", _p), ("up_bias", _p),
        ("down_bias", _p), ("gate_base", _p), ("up_base", _p), ("down_base", _p),
        ("gate_stride", C.c_int64), ("up_stride", C.c_int64), ("down_stride", C.c_int64),
        ("gate_tiles", _p), ("up_tiles", _p), ("down_tiles", _p),
    ]


class ReaderStatsC(C.Structure):
    """nsx_reader_stats."""

    _fields_ = [("requests", C.c_int64), ("bytes_read", C.c_int64), ("read_seconds", C.c_double),
                ("first_read", C.c_double), ("last_read", C.c_double), ("direct", C.c_int32),
                ("n_workers", C.c_int32)]


_SIGS = {
    "nsx_last_error": (C.c_char_p, []),
    "nsx_abi_version": (_i, []),
    "nsx_selftest": (_i, [_p, _p]),
    "nsx_read_probe": (_i, [_p, _i64, _i, _i, _p, _p]),
    "nsx_dequantize": (_i, [_i, _p, _i64, _i64, _p, _i, _p]),
    "nsx_fused_gemv": (_i, [_i, _p, _i64, _i64, _p, _i, _i64, _p, _p]),
    "nsx_fused_gemv_ex": (_i, [_i, _p, _i64, _i64, _p, _i, _i64, _p, _p, _p, _p]),
    "nsx_fused_gemv_norm": (_i, [_i, _p, _i64, _i64, _p, _p, _p, C.c_float, _p, _p, _p, _p, _p]),
    "nsx_t64_bytes": (_i64, [_i, _i64, _i64]),
    "nsx_t64_pack": (_i, [_i, _p, _i64, _i64, _p, _p]),
    "nsx_t64_unpack": (_i, [_i, _p, _i64, _i64, _p, _p]),
    "nsx_t64_gemv": (_i, [_i, _p, _i64, _i64, _i64, _i64, _p, _i, _i64, _p, _p]),
    "nsx_router_topk": (_i, [_p, _i64, _i64, _p, _i, _p, _i64, _i, _i, _p, _p, _p, _p]),
    "nsx_moe_workspace_bytes": (_i64, [C.POINTER(MoeLayerC), _i64]),
    "nsx_moe_forward": (_i, [C.POINTER(MoeLayerC), _p, _i64, _p, _p, _p, _p, _i64, _p]),
    "nsx_moe_forward_norm": (_i, [C.POINTER(MoeLayerC), _p, _p, _p, C.c_float, _i64, _p, _p, _p, _p, _p, _i64, _p]),
    "nsx_moe_forward_addnorm": (_i, [C.POINTER(MoeLayerC), _p, _i64, _p, _p, C.c_float, _p, _p, _p, _p, _p, _i64,
                                     _p]),
    "nsx_moe_chain_share_bytes": (_i64, [C.POINTER(MoeLayerC)]),
    "nsx_moe_chain_t1": (_i, [C.POINTER(MoeLayerC), _p, _p, C.c_float, _p, C.POINTER(MoeLayerC), _p, _p, _p, _p, _p,
                              _p, _i64, _i, _p]),
    "nsx_moe_phase": (_i, [C.POINTER(MoeLayerC), _i, _p, _i64, _p, _p, _p, _p, _i64, _p]),
    "nsx_moe_forward_static": (_i, [C.POINTER(MoeLayerC), _p, _i64, _p, _p, _p, _p]),
    "nsx_add_rmsnorm": (_i, [_p, _p, _i64, _i64, C.c_float, _p, _p, _p, _p]),
    "nsx_copy_blocks_async": (_i, [_i64, _p, _p, _p, _p, _p]),
    "nsx_gather_copy": (_i, [_i64, _p, _p, _p, _p]),
    "nsx_host_device_address": (_i, [_p, C.POINTER(C.c_uint64)]),
    "nsx_dequantize_rows": (_i, [_i, _p, _i64, _i64, _p, _i64, _p, _p]),
    "nsx_rope_kv_append": (_i, [_p, _p, _p, _p, _i, _i, _i, _p, C.c_float, _p, _p, _p, _i64, _p]),
    "nsx_attn_workspace_bytes": (_i64, [_i, _i, _i64]),
    "nsx_attn_decode": (_i, [_p, _p, _p, _p, _i, _i, _i, _p, _i64, _i, C.c_float, _p, _p, _p]),
    "nsx_attn_decode_qkv": (_i, [_p, _p, _p, _p, _p, C.c_float, _p, _i, _i, _i, _p, _p, _p, _i64, _i, C.c_float,
                                 _p, _p, _p]),
    "nsx_pos_advance": (_i, [_p, C.c_int32, _p]),
    "nsx_reader_open": (_i, [C.c_char_p, _i, _i, _i, _i64, _i, _p, C.POINTER(_p)]),
    "nsx_reader_submit": (_i, [_p, _i64, _i64, _p, _i, _p, C.POINTER(C.c_uint64)]),
    "nsx_reader_poll": (_i, [_p, C.c_uint64]),
    "nsx_reader_wait": (_i, [_p, C.c_uint64, _i64, _p]),
    "nsx_reader_get_stats": (_i, [_p, C.POINTER(ReaderStatsC)]),
    "nsx_reader_close": (_i, [_p]),
}
PHASE_ROUTER, PHASE_GATE_UP, PHASE_DOWN, PHASE_COMBINE = 0, 1, 2, 3
CHAIN_GATE_UP, CHAIN_DOWN = 1, 2  # nsx_moe_chain_t1 phases
STATIC_WORKSPACE_BYTES = 32 << 20  # NSX_STATIC_WORKSPACE_BYTES


class NativeError(RuntimeError):
    pass


_lib = None
_load_error: Exception | None = None


def header_functions() -> list[str]:
    """Every function the public header declares."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(nsx_\w+)\s*\(", text, re.M)))


def load():
    """The ctypes handle of libnsx.so; raises if it was never built."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise NativeError(
            f"{LIB_PATH} is missing: build it with `python -m nurostream_amd.build` "
            "(the HIP library is the only compute path for quantized weights)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.nsx_abi_version() != 3:
        raise NativeError("libnsx.so ABI version mismatch")
    _lib = lib
    return lib


def check(rc: int, what: str = "") -> None:
    if rc == OK:
        return
    msg = load().nsx_last_error().decode(errors="replace")
    if what:
        msg = f"{what}: {msg}"
    if rc == EINVAL:
        raise ValueError(msg)
    if rc == ETYPE:
        raise TypeError(msg)
    if rc == ENOTIMPL:
        raise NotImplementedError(msg)
    if rc == EIO:
        raise (EOFError if "short read" in msg else OSError)(msg)
    if rc == ETIMEDOUT:
        raise TimeoutError(msg)
    raise NativeError(msg)


def require_device(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise NativeError(
                "the nurostream_amd compute path runs on the GPU only "
                f"(got a {t.device} tensor); there is no CPU fallback")


def stream_ptr(device=None) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream


def act_dtype_code(dtype) -> int:
    import torch

    if dtype == torch.float32:
        return DT_F32
    if dtype == torch.float16:
        return DT_F16
    if dtype == torch.bfloat16:
        return DT_BF16
    raise TypeError(f"unsupported activation dtype {dtype}")


_selftested: set = set()


def ensure_selftest(device) -> None:
    """Run the FP4 conversion self test once per device."""
    import torch

    idx = torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    if idx in _selftested:
        return
    scratch = torch.zeros(1, dtype=torch.int32, device=f"cuda:{idx}")
    with torch.cuda.device(idx):
        check(load().nsx_selftest(scratch.data_ptr(), stream_ptr(idx)), "selftest")
    _selftested.add(idx)
