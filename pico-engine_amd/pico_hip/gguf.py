"""GGUF v2/v3 reader and writer (host side).

Reader: same result type as the reference's ``gguf.load`` (gguf.py:79-115): ``GGUF(path,
version, metadata, tensors, data_start, alignment)`` with ``TensorInfo(name, shape, ggml_type,
offset, n_elements, n_bytes)``; shapes are ggml ``ne`` order (fastest dimension first), the
data section starts at the next multiple of ``general.alignment`` (default 32).
Writer: produces the synthetic models the benchmarks and tests run on (the reference ships no
writer; the format is the public GGUF spec).
"""

from __future__ import annotations

import struct
from dataclasses import dataclass
from pathlib import Path
from typing import BinaryIO, Iterable

import numpy as np

from .dequant import nbytes_for

GGUF_MAGIC = 0x46554747  # b"GGUF" little-endian

# metadata value types (GGUF spec "Value Types")
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}
_NUMPY = {U8: "<u1", I8: "<i1", U16: "<u2", I16: "<i2", U32: "<u4", I32: "<i4", F32: "<f4",
          U64: "<u8", I64: "<i8", F64: "<f8"}


@dataclass
class TensorInfo:
    name: str
    shape: tuple[int, ...]   # ggml ne order: shape[0] is the contiguous dimension
    ggml_type: int
    offset: int              # relative to data_start
    n_elements: int
    n_bytes: int


@dataclass
class GGUF:
    path: Path
    version: int
    metadata: dict[str, object]
    tensors: list[TensorInfo]
    data_start: int
    alignment: int

    def tensor(self, name: str) -> TensorInfo:
        for t in self.tensors:
            if t.name == name:
                return t
        raise KeyError(name)


def _read_str(f: BinaryIO) -> str:
    (n,) = struct.unpack("<Q", f.read(8))
    return f.read(n).decode("utf-8", errors="replace")


def _read_value(f: BinaryIO, vtype: int):
    if vtype in _SCALAR:
        fmt = _SCALAR[vtype]
        return struct.unpack(fmt, f.read(struct.calcsize(fmt)))[0]
    if vtype == STR:
        return _read_str(f)
    if vtype == ARR:
        etype, n = struct.unpack("<IQ", f.read(12))
        if etype in _NUMPY:  # numeric arrays in one read
            arr = np.frombuffer(f.read(n * np.dtype(_NUMPY[etype]).itemsize), dtype=_NUMPY[etype])
            return [bool(v) for v in arr] if etype == BOOL else arr.tolist()
        return [_read_value(f, etype) for _ in range(n)]
    raise ValueError(f"unknown GGUF value type {vtype}")


def load(path: str | Path) -> GGUF:
    """Parse header, metadata and tensor infos (tensor data is not read)."""
    path = Path(path)
    with open(path, "rb") as f:
        magic, version, n_tensors, n_kv = struct.unpack("<IIQQ", f.read(24))
        if magic != GGUF_MAGIC:
            raise ValueError(f"{path}: first four bytes {magic:#010x} are not the GGUF signature")
        if version not in (2, 3):
            raise ValueError(f"{path}: GGUF format version {version} is not 2 or 3")
        metadata: dict[str, object] = {}
        for _ in range(n_kv):
            key = _read_str(f)
            (vtype,) = struct.unpack("<I", f.read(4))
            metadata[key] = _read_value(f, vtype)
        alignment = int(metadata.get("general.alignment", 32))
        tensors = []
        for _ in range(n_tensors):
            name = _read_str(f)
            (ndim,) = struct.unpack("<I", f.read(4))
            shape = struct.unpack(f"<{ndim}Q", f.read(8 * ndim))
            ggml_type, offset = struct.unpack("<IQ", f.read(12))
            n = int(np.prod(shape, dtype=np.int64)) if ndim else 1
            tensors.append(TensorInfo(name, tuple(int(s) for s in shape), ggml_type, offset, n,
                                      nbytes_for(ggml_type, n)))
        data_start = f.tell()
        data_start += (alignment - data_start % alignment) % alignment
    return GGUF(path, version, metadata, tensors, data_start, alignment)


def read_tensor_bytes(g: GGUF, t: TensorInfo) -> np.ndarray:
    """The tensor's raw bytes as a uint8 array (a read-only memory map of the file). Raises
    ValueError when the file ends before the tensor does (a truncated file or a bad offset)."""
    mm = np.memmap(g.path, dtype=np.uint8, mode="r")
    start = g.data_start + t.offset
    if t.offset < 0 or start + t.n_bytes > mm.size:
        raise ValueError(f"{g.path}: tensor {t.name} spans bytes [{start}, {start + t.n_bytes}) "
                         f"but the file has {mm.size}")
    return mm[start:start + t.n_bytes]


# ---- writer -------------------------------------------------------------------------------

def _w_str(f: BinaryIO, s: str) -> None:
    b = s.encode("utf-8")
    f.write(struct.pack("<Q", len(b)))
    f.write(b)


def _infer(value) -> int:
    if isinstance(value, bool):
        return BOOL
    if isinstance(value, int):
        return U32 if 0 <= value < 2**32 else I64
    if isinstance(value, float):
        return F32
    if isinstance(value, str):
        return STR
    if isinstance(value, (list, tuple)):
        return ARR
    raise TypeError(f"cannot store {type(value)} in GGUF metadata")


def _w_value(f: BinaryIO, vtype: int, value) -> None:
    if vtype in _SCALAR:
        f.write(struct.pack(_SCALAR[vtype], value))
    elif vtype == STR:
        _w_str(f, value)
    elif vtype == ARR:
        etype = _infer(value[0]) if len(value) else I32
        if etype == U32 and any(v < 0 for v in value):
            etype = I32
        f.write(struct.pack("<IQ", etype, len(value)))
        if etype in _NUMPY and etype != BOOL:
            f.write(np.asarray(value, dtype=_NUMPY[etype]).tobytes())
        else:
            for v in value:
                _w_value(f, etype, v)
    else:
        raise ValueError(vtype)


def write(path: str | Path, metadata: dict[str, object],
          tensors: Iterable[tuple[str, tuple[int, ...], int, bytes | np.ndarray]],
          alignment: int = 32) -> None:
    """Write a GGUF v3 file. ``tensors`` = (name, ne-shape, ggml_type, raw bytes)."""
    tensors = list(tensors)
    meta = dict(metadata)
    if alignment != 32:
        meta["general.alignment"] = alignment
    offsets, off = [], 0
    for name, shape, gtype, raw in tensors:
        n = int(np.prod(shape, dtype=np.int64))
        nbytes = nbytes_for(gtype, n)
        if len(memoryview(raw).cast("B")) != nbytes:
            raise ValueError(f"{name}: {len(memoryview(raw).cast('B'))} bytes, expected {nbytes}")
        off += (alignment - off % alignment) % alignment
        offsets.append(off)
        off += nbytes
    with open(path, "wb") as f:
        f.write(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(meta)))
        for key, value in meta.items():
            _w_str(f, key)
            vt = _infer(value)
            f.write(struct.pack("<I", vt))
            _w_value(f, vt, value)
        for (name, shape, gtype, _), o in zip(tensors, offsets):
            _w_str(f, name)
            f.write(struct.pack("<I", len(shape)))
            f.write(struct.pack(f"<{len(shape)}Q", *shape))
            f.write(struct.pack("<IQ", gtype, o))
        pos = f.tell()
        f.write(b"\0" * ((alignment - pos % alignment) % alignment))
        base = f.tell()
        for (name, shape, gtype, raw), o in zip(tensors, offsets):
            pad = base + o - f.tell()
            f.write(b"\0" * pad)
            f.write(memoryview(raw).cast("B"))
