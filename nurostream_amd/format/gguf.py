"""GGML block layouts, tensor coordinates and a minimal GGUF v3 container.

The interface of the reference's `neurostream/format/gguf.py`:
  * `GGMLType` / `TYPE_LAYOUT` / `nbytes_for`  -> format/gguf.py:19-68 (the
    type ids and block layouts are ggml's file format)
  * `TensorInfo` (ggml-order shape, torch_shape, memoised geometry) -> :102-128
  * `GGUFFile` (header, metadata and tensor index; no tensor data) -> :162-245;
    here decoded from a read-only memory map of the header, field by field at
    offsets

The writer (`GGUFWriter`) has no counterpart in the reference package (the
reference's tests use the third-party gguf-py writer); it exists so that
synthetic models can be written to and re-read from a real GGUF file.
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass
from enum import IntEnum
from pathlib import Path
from typing import Any

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
    """Bytes that `n_elements` values of `dtype` occupy: whole blocks only
    (the contract of format/gguf.py:58-68: NotImplementedError for a type
    without a known block layout, ValueError for a partial block)."""
    layout = TYPE_LAYOUT.get(dtype)
    if layout is None:
        raise NotImplementedError(f"no block layout known for ggml type {dtype!r}")
    per, size = layout
    blocks, rest = divmod(int(n_elements), per)
    if rest:
        raise ValueError(f"{GGMLType(dtype).name} stores whole blocks of {per} values; "
                         f"{n_elements} values leave {rest} over")
    return blocks * size


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
    """GGUF metadata value type ids (part of the file format)."""
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


# little-endian struct codes of the fixed-size value types
_SCALAR_FMT = {
    _ValueType.UINT8: "<B", _ValueType.INT8: "<b",
    _ValueType.UINT16: "<H", _ValueType.INT16: "<h",
    _ValueType.UINT32: "<I", _ValueType.INT32: "<i",
    _ValueType.FLOAT32: "<f", _ValueType.BOOL: "<?",
    _ValueType.UINT64: "<Q", _ValueType.INT64: "<q",
    _ValueType.FLOAT64: "<d",
}
_SCALAR = {vt: struct.Struct(f) for vt, f in _SCALAR_FMT.items()}
_U32, _U64 = struct.Struct("<I"), struct.Struct("<Q")
_HEAD = struct.Struct("<4sIQQ")  # magic, version, tensor count, metadata count


class _HeaderView:
    """Decodes the header region of a GGUF file in place, from a read-only
    memory map: every field is unpacked at an offset, so no stream position
    or intermediate copies are involved."""

    def __init__(self, buf, path) -> None:
        self.buf = buf
        self.pos = 0
        self.path = path

    def _take(self, n: int) -> int:
        at = self.pos
        if at + n > len(self.buf):
            raise EOFError(f"{self.path}: the GGUF header ends early ({n} bytes needed at offset {at}, "
                           f"the file has {len(self.buf)})")
        self.pos = at + n
        return at

    def unpack(self, st: struct.Struct):
        return st.unpack_from(self.buf, self._take(st.size))

    def u32(self) -> int:
        return self.unpack(_U32)[0]

    def u64(self) -> int:
        return self.unpack(_U64)[0]

    def text(self) -> str:
        n = self.u64()
        at = self._take(n)
        return bytes(self.buf[at:at + n]).decode("utf-8", errors="replace")

    def value(self, vt: int) -> Any:
        vt = _ValueType(vt)
        if vt == _ValueType.STRING:
            return self.text()
        if vt == _ValueType.ARRAY:
            inner = _ValueType(self.u32())
            count = self.u64()
            if inner in _SCALAR:  # a run of fixed-size values: one unpack
                st = _SCALAR[inner]
                at = self._take(st.size * count)
                return list(struct.unpack_from(f"<{count}{st.format[1:]}", self.buf, at))
            return [self.value(inner) for _ in range(count)]
        return self.unpack(_SCALAR[vt])[0]


class GGUFFile:
    """Header, metadata and tensor index of a GGUF v3 file; holds no tensor
    data (the reader contract of format/gguf.py:162-245: `metadata`,
    `tensors`, `alignment`, `data_offset`, `arch()`, `cfg()`, `file_offset()`)."""

    def __init__(self, path: str | Path) -> None:
        self.path = Path(path)
        self.metadata: dict[str, Any] = {}
        self.tensors: dict[str, TensorInfo] = {}
        self.alignment = DEFAULT_ALIGNMENT
        self.data_offset = 0
        self.version = 0
        with open(self.path, "rb") as fh:
            size = os.fstat(fh.fileno()).st_size
            if size < _HEAD.size:
                raise EOFError(f"{self.path}: {size} bytes is too short for a GGUF header")
            with mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ) as mm:
                self._index(_HeaderView(memoryview(mm), self.path))

    def _index(self, hv: _HeaderView) -> None:
        try:
            magic, version, n_tensors, n_kv = hv.unpack(_HEAD)
            if magic != GGUF_MAGIC:
                raise ValueError(f"{self.path} is not a GGUF file (starts with {magic!r})")
            if version != 3:
                raise ValueError(f"{self.path}: GGUF version {version}; this reader handles version 3")
            self.version = version
            for _ in range(n_kv):
                key = hv.text()
                self.metadata[key] = hv.value(hv.u32())
            self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
            for _ in range(n_tensors):
                name = hv.text()
                n_dims = hv.u32()
                dims = tuple(hv.u64() for _ in range(n_dims))
                dtype = GGMLType(hv.u32())
                offset = hv.u64()
                n = 1
                for d in dims:
                    n *= d
                self.tensors[name] = TensorInfo(name, dims, dtype, offset, nbytes_for(dtype, n))
            # tensor data starts at the next multiple of the alignment
            self.data_offset = -(-hv.pos // self.alignment) * self.alignment
        finally:
            hv.buf.release()

    def arch(self) -> str:
        return str(self.metadata.get("general.architecture", "unknown"))

    def cfg(self, suffix: str, default: Any = None) -> Any:
        """Metadata key `<arch>.<suffix>`."""
        return self.metadata.get(f"{self.arch()}.{suffix}", default)

    def file_offset(self, info: TensorInfo) -> int:
        """Absolute file offset of a tensor's first byte."""
        return self.data_offset + info.offset

    def total_tensor_bytes(self) -> int:
        return sum(t.nbytes for t in self.tensors.values())

    def __repr__(self) -> str:
        return (f"GGUFFile({self.path.name!r}, arch={self.arch()!r}, {len(self.tensors)} tensors, "
                f"{self.total_tensor_bytes() / 2**30:.2f} GiB of tensor data)")


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
