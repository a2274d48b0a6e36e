"""ctypes binding of the reference's own GGUF loader (TEST INFRASTRUCTURE ONLY).

oracle/_ref/libgguf_ref.so is src/loader/gguf_loader.c compiled unchanged
from the reference tree by oracle/Makefile; it is the checker of
asmllm_amd.gguf_file.  The structures below restate gguf_loader.h:13-69 for
ctypes.  Absent (None) where the reference tree was not there to build from.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, Structure, c_char, c_char_p, c_int, c_size_t, c_uint32, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_ref" / "libgguf_ref.so"


class Header(Structure):  # gguf_loader.h:17-22
    _fields_ = [("magic", c_uint32), ("version", c_uint32), ("tensor_count", c_uint64), ("kv_count", c_uint64)]


class TensorInfo(Structure):  # gguf_loader.h:38-44
    _fields_ = [("name", c_char * 128), ("n_dims", c_uint32), ("dims", c_uint64 * 4), ("type", c_uint32),
                ("offset", c_uint64)]


class Context(Structure):  # gguf_loader.h:62-69
    _fields_ = [("header", Header), ("kv_pairs", c_void_p), ("tensors", POINTER(TensorInfo)),
                ("file_data", c_void_p), ("file_size", c_size_t), ("data_offset", c_size_t)]


_LIB = None


def lib():
    """The loaded reference loader, or None when it was not built."""
    global _LIB
    if _LIB is None and LIB_PATH.exists():
        L = ctypes.CDLL(str(LIB_PATH))
        L.gguf_load_from_file.argtypes = [c_char_p, POINTER(POINTER(Context))]
        L.gguf_load_from_file.restype = c_int
        L.gguf_find_tensor.argtypes = [POINTER(Context), c_char_p, POINTER(POINTER(TensorInfo))]
        L.gguf_find_tensor.restype = c_int
        L.gguf_get_tensor_data.argtypes = [POINTER(Context), POINTER(TensorInfo)]
        L.gguf_get_tensor_data.restype = c_void_p
        L.gguf_free.argtypes = [POINTER(Context)]
        L.gguf_free.restype = None
        _LIB = L
    return _LIB


def load(path) -> dict | None:
    """What the reference loader makes of a file: header counts, data offset
    and, per tensor, (dims, type, offset, byte offset of its data in the
    file); None when it refuses the file."""
    L = lib()
    ctx = POINTER(Context)()
    if not L.gguf_load_from_file(str(path).encode(), ctypes.byref(ctx)):
        return None
    try:
        c = ctx.contents
        out = {"version": c.header.version, "tensor_count": c.header.tensor_count,
               "kv_count": c.header.kv_count, "data_offset": c.data_offset, "file_size": c.file_size,
               "tensors": {}}
        for i in range(c.header.tensor_count):
            t = c.tensors[i]
            name = t.name.decode()
            found = POINTER(TensorInfo)()
            assert L.gguf_find_tensor(ctx, name.encode(), ctypes.byref(found))
            data = L.gguf_get_tensor_data(ctx, found)
            out["tensors"][name] = (tuple(t.dims[d] for d in range(t.n_dims)), t.type, t.offset,
                                    None if data is None else data - c.file_data)
        return out
    finally:
        L.gguf_free(ctx)
