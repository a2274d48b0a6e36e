"""GGUF v2/v3 model files: reading (memory-mapped) and writing.

Reads what the reference's loaders read (src/loader/gguf_loader.c:84-190,
src/runtime/generate.py:38-88): the 24-byte header (magic "GGUF", version,
tensor count, key/value count), the metadata key/value pairs, the tensor
descriptors (name, dims, type, offset relative to the data section) and the
data section, which starts at the descriptors' end rounded up to
``general.alignment`` (32 when absent; gguf_loader.c:151-155 -- generate.py
always uses 32).  Unlike the reference, every metadata value is kept, not
only the vocabulary, and tensors are numpy views of a read-only memory map,
so a multi-GB model is not copied before its one-time upload to the GPU.

Tensor layouts (generate.py:169-180): dims[0] is the fastest (K) dimension,
dims[1] the row count; Q4_0/Q5_0/Q8_0 tensors come back as
[rows][K/32][18|22|34] uint8 blocks, F32/F16 as arrays of shape dims[::-1].
"""

from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .gguf import Q4_0_BYTES, Q5_0_BYTES, Q8_0_BYTES, QK

GGUF_MAGIC = 0x46554747  # "GGUF" little-endian
DEFAULT_ALIGNMENT = 32

# value types (gguf_loader.h:22-36)
T_UINT8, T_INT8, T_UINT16, T_INT16, T_UINT32, T_INT32, T_FLOAT32, T_BOOL, T_STRING, T_ARRAY, T_UINT64, T_INT64, \
    T_FLOAT64 = range(13)
_SCALAR = {T_UINT8: "<B", T_INT8: "<b", T_UINT16: "<H", T_INT16: "<h", T_UINT32: "<I", T_INT32: "<i",
           T_FLOAT32: "<f", T_BOOL: "<?", T_UINT64: "<Q", T_INT64: "<q", T_FLOAT64: "<d"}

# tensor types (GGUF / ggml numbering, generate.py:170-180; Q5_0 is ggml's 6)
F32, F16, Q4_0, Q5_0, Q8_0 = 0, 1, 2, 6, 8
_BLOCK_BYTES = {Q4_0: Q4_0_BYTES, Q5_0: Q5_0_BYTES, Q8_0: Q8_0_BYTES}


class GGUFError(ValueError):
    """The file is not a GGUF v2/v3 model this reader understands."""


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dims: tuple[int, ...]
    type: int
    offset: int  # relative to the data section

    @property
    def nbytes(self) -> int:
        n = int(np.prod(self.dims, dtype=np.int64)) if self.dims else 1
        if self.type == F32:
            return 4 * n
        if self.type == F16:
            return 2 * n
        if self.type in _BLOCK_BYTES:
            if self.dims[0] % QK:
                raise GGUFError(f"{self.name}: K = {self.dims[0]} is not a multiple of 32")
            return n // QK * _BLOCK_BYTES[self.type]
        raise GGUFError(f"{self.name}: tensor type {self.type} is not supported")


class _Reader:
    def __init__(self, buf, size: int):
        self.buf, self.size, self.pos = buf, size, 0

    def take(self, n: int) -> bytes:
        if self.pos + n > self.size:
            raise GGUFError(f"truncated file: need {n} bytes at offset {self.pos} of {self.size}")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return bytes(b)

    def scalar(self, t: int):
        fmt = _SCALAR[t]
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar(T_UINT64)
        return self.take(n).decode("utf-8", errors="replace")

    def value(self, t: int):
        if t in _SCALAR:
            return self.scalar(t)
        if t == T_STRING:
            return self.string()
        if t == T_ARRAY:
            et = self.scalar(T_UINT32)
            count = self.scalar(T_UINT64)
            if et == T_ARRAY:
                raise GGUFError("nested arrays are not supported")
            return [self.value(et) for _ in range(count)]
        raise GGUFError(f"unknown metadata value type {t} at offset {self.pos}")


class GGUFFile:
    """A parsed GGUF file; ``tensor(name)`` returns views of its data."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        size = self.path.stat().st_size
        if size < 24:
            raise GGUFError(f"{self.path}: {size} bytes, smaller than a GGUF header")
        with open(self.path, "rb") as f:
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        r = _Reader(self._mm, size)
        magic, self.version = r.scalar(T_UINT32), r.scalar(T_UINT32)
        if magic != GGUF_MAGIC:
            raise GGUFError(f"{self.path}: bad magic 0x{magic:08x}")
        if not 2 <= self.version <= 3:  # gguf_loader.c:15-24
            raise GGUFError(f"{self.path}: GGUF version {self.version} (supported: 2, 3)")
        n_tensors, n_kv = r.scalar(T_UINT64), r.scalar(T_UINT64)
        self.metadata: dict[str, object] = {}
        self.metadata_types: dict[str, int] = {}
        for _ in range(n_kv):
            key = r.string()
            t = r.scalar(T_UINT32)
            self.metadata[key] = r.value(t)
            self.metadata_types[key] = t
        self.tensors: dict[str, TensorInfo] = {}
        for _ in range(n_tensors):
            name = r.string()
            n_dims = r.scalar(T_UINT32)
            dims = tuple(r.scalar(T_UINT64) for _ in range(n_dims))
            ttype, offset = r.scalar(T_UINT32), r.scalar(T_UINT64)
            self.tensors[name] = TensorInfo(name, dims, ttype, offset)
        align = self.metadata.get("general.alignment", DEFAULT_ALIGNMENT)
        if not isinstance(align, int) or isinstance(align, bool) or align <= 0:
            raise GGUFError(f"{self.path}: general.alignment = {align!r}")
        self.alignment = align
        self.data_offset = (r.pos + align - 1) // align * align
        self.size = size
        for t in self.tensors.values():
            end = self.data_offset + t.offset + t.nbytes
            if end > size:
                raise GGUFError(f"{self.path}: tensor {t.name} ends at {end}, past the file ({size} bytes)")

    def tensor(self, name: str) -> np.ndarray:
        """Read-only numpy view of one tensor (see the module docstring for shapes)."""
        try:
            t = self.tensors[name]
        except KeyError:
            raise KeyError(f"{self.path}: no tensor {name!r}") from None
        start = self.data_offset + t.offset
        raw = np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=start)
        if t.type == F32:
            return raw.view(np.float32).reshape(t.dims[::-1])
        if t.type == F16:
            return raw.view(np.float16).reshape(t.dims[::-1])
        rows = int(np.prod(t.dims[1:], dtype=np.int64)) if len(t.dims) > 1 else 1
        return raw.reshape(rows, t.dims[0] // QK, _BLOCK_BYTES[t.type])

    def vocab(self) -> list[str]:
        """tokenizer.ggml.tokens (generate.py:71-76)."""
        return list(self.metadata.get("tokenizer.ggml.tokens", []))

    def close(self) -> None:
        if getattr(self, "_mm", None) is not None:
            try:
                self._mm.close()
            except BufferError:  # views still alive: the map closes when they go
                pass
            self._mm = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _value_bytes(t: int, v) -> bytes:
    if t in _SCALAR:
        return struct.pack(_SCALAR[t], v)
    if t == T_STRING:
        b = v.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    raise GGUFError(f"cannot write value type {t}")


def write_gguf(path: str | Path, metadata: dict, tensors: dict[str, tuple[int, tuple[int, ...], np.ndarray]],
               alignment: int = DEFAULT_ALIGNMENT, version: int = 3) -> None:
    """Writes a GGUF file.

    metadata: key -> (value type, value), arrays as (T_ARRAY, (element type,
    [values])).  tensors: name -> (tensor type, dims with dims[0] fastest,
    bytes/array whose raw bytes are the tensor).  When alignment differs from
    32 it is also recorded as general.alignment (uint32).  Tensor data are
    padded to the alignment, as GGUF writers do.
    """
    if alignment != DEFAULT_ALIGNMENT and "general.alignment" not in metadata:
        metadata = {**metadata, "general.alignment": (T_UINT32, alignment)}
    out = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(metadata)))
    for key, (t, v) in metadata.items():
        out += _value_bytes(T_STRING, key) + struct.pack("<I", t)
        if t == T_ARRAY:
            et, values = v
            out += struct.pack("<IQ", et, len(values))
            for e in values:
                out += _value_bytes(et, e)
        else:
            out += _value_bytes(t, v)
    blobs, offset = [], 0
    for name, (ttype, dims, data) in tensors.items():
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        info = TensorInfo(name, tuple(dims), ttype, offset)
        if info.nbytes != raw.size:
            raise GGUFError(f"{name}: {raw.size} bytes for dims {dims} type {ttype} ({info.nbytes} expected)")
        out += _value_bytes(T_STRING, name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ttype, offset)
        blobs.append(raw)
        offset += (raw.size + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    with open(path, "wb") as f:
        f.write(out)
        for raw in blobs:
            f.write(raw.tobytes())
            f.write(b"\0" * ((-raw.size) % alignment))
