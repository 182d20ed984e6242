"""GGML block layouts, tensor coordinates and a minimal GGUF v3 container.

Mirrors the reference's `neurostream/format/gguf.py`:
  * `GGMLType` / `TYPE_LAYOUT` / `nbytes_for`  -> format/gguf.py:19-68
  * `TensorInfo` (ggml-order shape, torch_shape, memoised geometry) -> :102-128
  * `GGUFFile` (header, metadata and tensor index; no tensor data) -> :162-245

The writer (`GGUFWriter`) has no counterpart in the reference package (the
reference's tests use the third-party gguf-py writer); it exists so that
synthetic models can be written to and re-read from a real GGUF file.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from enum import IntEnum
from pathlib import Path
from typing import Any, BinaryIO

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32


class GGMLType(IntEnum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    BF16 = 30
    MXFP4 = 39


# (elements per block, bytes per block) -- the ggml values, format/gguf.py:39-55
TYPE_LAYOUT: dict[GGMLType, tuple[int, int]] = {
    GGMLType.F32: (1, 4),
    GGMLType.F16: (1, 2),
    GGMLType.BF16: (1, 2),
    GGMLType.MXFP4: (32, 17),
    GGMLType.Q4_0: (32, 18),
    GGMLType.Q4_1: (32, 20),
    GGMLType.Q5_0: (32, 22),
    GGMLType.Q5_1: (32, 24),
    GGMLType.Q8_0: (32, 34),
    GGMLType.Q2_K: (256, 84),
    GGMLType.Q3_K: (256, 110),
    GGMLType.Q4_K: (256, 144),
    GGMLType.Q5_K: (256, 176),
    GGMLType.Q6_K: (256, 210),
    GGMLType.Q8_K: (256, 292),
}

FLOAT_TYPES = frozenset({GGMLType.F32, GGMLType.F16, GGMLType.BF16})


def nbytes_for(dtype: GGMLType, n_elements: int) -> int:
    """Byte size of `n_elements` stored as `dtype` (format/gguf.py:58-68)."""
    if dtype not in TYPE_LAYOUT:
        raise NotImplementedError(f"unsupported ggml type: {dtype!r}")
    block_elems, block_bytes = TYPE_LAYOUT[dtype]
    if n_elements % block_elems:
        raise ValueError(
            f"{n_elements} elements is not a multiple of {dtype.name} "
            f"block size {block_elems}"
        )
    return (n_elements // block_elems) * block_bytes


@dataclass(slots=True)
class TensorInfo:
    """Where a tensor lives in the file: coordinates only, no data."""

    name: str
    shape: tuple[int, ...]  # ggml order: fastest-varying dimension first
    dtype: GGMLType
    offset: int  # relative to the start of the data section
    nbytes: int
    # (n_rows, row_elems, row_bytes), memoised on the instance (never keyed by
    # id(): a recycled address would hand one model's strides to another).
    geom: tuple[int, int, int] | None = None

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    @property
    def torch_shape(self) -> tuple[int, ...]:
        """Row-major shape: ggml dims reversed."""
        return tuple(reversed(self.shape))


def tensor_info(name: str, torch_shape, dtype: GGMLType, offset: int = 0) -> TensorInfo:
    """Build a TensorInfo from a row-major (torch-order) shape."""
    n = 1
    for d in torch_shape:
        n *= int(d)
    return TensorInfo(name, tuple(int(d) for d in reversed(tuple(torch_shape))),
                      GGMLType(dtype), offset, nbytes_for(GGMLType(dtype), n))


def row_geometry(info: TensorInfo) -> tuple[int, int, int]:
    """(n_rows, row_elements, row_bytes), flattening all leading dimensions.

    Expert e of a stacked (n_expert, out, in) tensor owns rows
    [e*out, (e+1)*out). Follows io/source.py:38-62.
    """
    if info.geom is not None:
        return info.geom
    shape = info.torch_shape
    if len(shape) == 1:
        out = (1, shape[0], info.nbytes)
    else:
        row_elems = shape[-1]
        n_rows = 1
        for d in shape[:-1]:
            n_rows *= d
        out = (n_rows, row_elems, nbytes_for(info.dtype, row_elems))
    info.geom = out
    return out


# ---------------------------------------------------------------------------
# GGUF v3 container (format/gguf.py:71-245)

class _ValueType(IntEnum):
    UINT8 = 0
    INT8 = 1
    UINT16 = 2
    INT16 = 3
    UINT32 = 4
    INT32 = 5
    FLOAT32 = 6
    BOOL = 7
    STRING = 8
    ARRAY = 9
    UINT64 = 10
    INT64 = 11
    FLOAT64 = 12


_SCALAR_FMT = {
    _ValueType.UINT8: "<B", _ValueType.INT8: "<b",
    _ValueType.UINT16: "<H", _ValueType.INT16: "<h",
    _ValueType.UINT32: "<I", _ValueType.INT32: "<i",
    _ValueType.FLOAT32: "<f", _ValueType.BOOL: "<?",
    _ValueType.UINT64: "<Q", _ValueType.INT64: "<q",
    _ValueType.FLOAT64: "<d",
}


class _Cursor:
    def __init__(self, fh: BinaryIO) -> None:
        self.fh = fh

    def read(self, n: int) -> bytes:
        b = self.fh.read(n)
        if len(b) != n:
            raise EOFError(f"truncated GGUF: wanted {n} bytes, got {len(b)}")
        return b

    def scalar(self, vt: _ValueType) -> Any:
        fmt = _SCALAR_FMT[vt]
        return struct.unpack(fmt, self.read(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        (n,) = struct.unpack("<Q", self.read(8))
        return self.read(n).decode("utf-8", errors="replace")

    def value(self, vt: _ValueType) -> Any:
        if vt == _ValueType.STRING:
            return self.string()
        if vt == _ValueType.ARRAY:
            (elem_t,) = struct.unpack("<I", self.read(4))
            (count,) = struct.unpack("<Q", self.read(8))
            elem_t = _ValueType(elem_t)
            return [self.value(elem_t) for _ in range(count)]
        return self.scalar(vt)


class GGUFFile:
    """Parsed GGUF index. Holds no tensor data (format/gguf.py:162-245)."""

    def __init__(self, path: str | Path) -> None:
        self.path = Path(path)
        self.metadata: dict[str, Any] = {}
        self.tensors: dict[str, TensorInfo] = {}
        self.alignment = DEFAULT_ALIGNMENT
        self.data_offset = 0
        self._parse()

    def _parse(self) -> None:
        with open(self.path, "rb") as fh:
            cur = _Cursor(fh)
            magic = cur.read(4)
            if magic != GGUF_MAGIC:
                raise ValueError(f"not a GGUF file (magic={magic!r}): {self.path}")
            version, n_tensors, n_kv = struct.unpack("<IQQ", cur.read(20))
            if version != 3:
                raise ValueError(f"unsupported GGUF version {version} (need 3)")
            self.version = version
            for _ in range(n_kv):
                key = cur.string()
                (vt,) = struct.unpack("<I", cur.read(4))
                self.metadata[key] = cur.value(_ValueType(vt))
            self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
            infos = []
            for _ in range(n_tensors):
                name = cur.string()
                (n_dims,) = struct.unpack("<I", cur.read(4))
                dims = struct.unpack(f"<{n_dims}Q", cur.read(8 * n_dims))
                (raw_t,) = struct.unpack("<I", cur.read(4))
                (offset,) = struct.unpack("<Q", cur.read(8))
                infos.append((name, dims, GGMLType(raw_t), offset))
            pos = fh.tell()
            pad = (self.alignment - (pos % self.alignment)) % self.alignment
            self.data_offset = pos + pad
        for name, dims, dtype, offset in infos:
            n = 1
            for d in dims:
                n *= d
            self.tensors[name] = TensorInfo(name, tuple(dims), dtype, offset, nbytes_for(dtype, n))

    def arch(self) -> str:
        return str(self.metadata.get("general.architecture", "unknown"))

    def cfg(self, suffix: str, default: Any = None) -> Any:
        return self.metadata.get(f"{self.arch()}.{suffix}", default)

    def file_offset(self, info: TensorInfo) -> int:
        return self.data_offset + info.offset

    def total_tensor_bytes(self) -> int:
        return sum(t.nbytes for t in self.tensors.values())

    def __repr__(self) -> str:
        return (f"<GGUFFile {self.path.name} arch={self.arch()} "
                f"tensors={len(self.tensors)} data={self.total_tensor_bytes() / 1e9:.2f}GB>")


class GGUFWriter:
    """Write a GGUF v3 file from already-encoded tensor bytes.

    Tensors are given as (name, torch_shape, GGMLType, bytes-like); metadata as
    python scalars/strings/lists. Data is aligned to `alignment` bytes.
    """

    def __init__(self, path: str | Path, arch: str, alignment: int = DEFAULT_ALIGNMENT):
        self.path = Path(path)
        self.alignment = alignment
        self.kv: list[tuple[str, _ValueType, Any]] = [
            ("general.architecture", _ValueType.STRING, arch)]
        self.tensors: list[tuple[str, tuple[int, ...], GGMLType, bytes]] = []

    def add(self, key: str, value: Any) -> None:
        if isinstance(value, bool):
            vt = _ValueType.BOOL
        elif isinstance(value, int):
            vt = _ValueType.UINT32 if 0 <= value < (1 << 32) else _ValueType.INT64
        elif isinstance(value, float):
            vt = _ValueType.FLOAT32
        elif isinstance(value, str):
            vt = _ValueType.STRING
        elif isinstance(value, (list, tuple)):
            vt = _ValueType.ARRAY
        else:
            raise TypeError(f"unsupported metadata value for {key}: {type(value)}")
        self.kv.append((key, vt, value))

    def add_tensor(self, name: str, torch_shape, dtype: GGMLType, data) -> None:
        data = bytes(memoryview(data).cast("B"))
        n = 1
        for d in torch_shape:
            n *= int(d)
        if len(data) != nbytes_for(GGMLType(dtype), n):
            raise ValueError(f"{name}: {len(data)} bytes for shape {tuple(torch_shape)} {GGMLType(dtype).name}")
        self.tensors.append((name, tuple(int(d) for d in torch_shape), GGMLType(dtype), data))

    @staticmethod
    def _enc_str(s: str) -> bytes:
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def _enc_value(self, vt: _ValueType, v: Any) -> bytes:
        if vt == _ValueType.STRING:
            return self._enc_str(v)
        if vt == _ValueType.ARRAY:
            items = list(v)
            if items and isinstance(items[0], str):
                et = _ValueType.STRING
            elif items and isinstance(items[0], float):
                et = _ValueType.FLOAT32
            else:
                et = _ValueType.INT32
            return (struct.pack("<IQ", int(et), len(items))
                    + b"".join(self._enc_value(et, x) for x in items))
        return struct.pack(_SCALAR_FMT[vt], v)

    def write(self) -> None:
        head = bytearray()
        head += GGUF_MAGIC + struct.pack("<IQQ", 3, len(self.tensors), len(self.kv))
        for key, vt, v in self.kv:
            head += self._enc_str(key) + struct.pack("<I", int(vt)) + self._enc_value(vt, v)
        offset = 0
        offsets = []
        for name, shape, dtype, data in self.tensors:
            offsets.append(offset)
            offset += len(data)
            offset += (self.alignment - offset % self.alignment) % self.alignment
        for (name, shape, dtype, data), off in zip(self.tensors, offsets):
            dims = tuple(reversed(shape))
            head += self._enc_str(name) + struct.pack("<I", len(dims))
            head += struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", int(dtype), off)
        head += b"\0" * ((self.alignment - len(head) % self.alignment) % self.alignment)
        with open(self.path, "wb") as fh:
            fh.write(head)
            pos = 0
            for (name, shape, dtype, data), off in zip(self.tensors, offsets):
                fh.write(b"\0" * (off - pos))
                fh.write(data)
                pos = off + len(data)
