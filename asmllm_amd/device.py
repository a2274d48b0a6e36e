"""Device memory, streams and events over libasmllm's plumbing entry points.

The reference keeps every tensor in numpy arrays and passes raw pointers
through ctypes (src/runtime/generate.py:268-317).  Here weights and
activations live in HBM; these wrappers own the allocations and move numpy
data in and out.
"""

from __future__ import annotations

import ctypes

import numpy as np

from .native import check, lib

H2D, D2H, D2D = 1, 2, 3


class DeviceBuffer:
    """One device allocation.  Freed on close() or garbage collection."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        ptr = lib().asmhip_malloc(max(self.nbytes, 1))
        if not ptr:
            check(-2, f"device allocation of {self.nbytes} bytes")
        self.ptr = int(ptr)

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("upload exceeds the allocation")
        check(lib().asmhip_memcpy(self.ptr + offset, arr.ctypes.data, arr.nbytes, H2D), "memcpy h2d")

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download exceeds the allocation")
        check(lib().asmhip_memcpy(out.ctypes.data, self.ptr + offset, out.nbytes, D2H), "memcpy d2h")
        return out

    def copy_from(self, other: "DeviceBuffer", nbytes: int | None = None) -> None:
        n = other.nbytes if nbytes is None else nbytes
        check(lib().asmhip_memcpy(self.ptr, other.ptr, n, D2D), "memcpy d2d")

    def close(self) -> None:
        if getattr(self, "ptr", 0):
            lib().asmhip_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    def __init__(self):
        handle = lib().asmhip_stream_create()
        if not handle:
            check(-2, "stream create")
        self.handle = int(handle)

    def synchronize(self) -> None:
        check(lib().asmhip_stream_synchronize(self.handle), "stream synchronize")

    def close(self) -> None:
        if getattr(self, "handle", 0):
            lib().asmhip_stream_destroy(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    """A HIP event.  timing=True: an event used only to time stream work
    (asmhip_event_create_timing): its record does no system-scope cache
    writeback / invalidate, which would otherwise slow the work after it."""

    def __init__(self, timing: bool = False):
        handle = lib().asmhip_event_create_timing() if timing else lib().asmhip_event_create()
        if not handle:
            check(-2, "event create")
        self.handle = int(handle)

    def record(self, stream: Stream | None = None) -> None:
        check(lib().asmhip_event_record(self.handle, stream.handle if stream else None), "event record")

    def synchronize(self) -> None:
        check(lib().asmhip_event_synchronize(self.handle), "event synchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().asmhip_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)), "event elapsed")
        return float(ms.value)

    def close(self) -> None:
        if getattr(self, "handle", 0):
            lib().asmhip_event_destroy(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def device_count() -> int:
    return int(lib().asmhip_device_count())


def device_info() -> dict:
    name = ctypes.create_string_buffer(128)
    cus, clk, mem = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
    check(lib().asmhip_device_info(name, 128, ctypes.byref(cus), ctypes.byref(clk), ctypes.byref(mem)), "device info")
    return {"arch": name.value.decode(), "compute_units": cus.value, "clock_khz": clk.value, "memory": mem.value}


def synchronize() -> None:
    check(lib().asmhip_synchronize(), "device synchronize")


class Graph:
    """A captured, instantiated HIP graph (replayed with launch())."""

    def __init__(self, handle: int):
        self.handle = handle

    @classmethod
    def capture(cls, stream: Stream, enqueue) -> "Graph":
        check(lib().asmhip_stream_begin_capture(stream.handle), "begin capture")
        try:
            enqueue()
        finally:
            out = ctypes.c_void_p()
            rc = lib().asmhip_stream_end_capture(stream.handle, ctypes.byref(out))
        check(rc, "end capture")
        return cls(int(out.value))

    def launch(self, stream: Stream) -> None:
        check(lib().asmhip_graph_launch(self.handle, stream.handle), "graph launch")

    def close(self) -> None:
        if getattr(self, "handle", 0):
            lib().asmhip_graph_destroy(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
