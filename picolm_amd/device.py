"""Device (HBM) buffers over the library's allocator and stream."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._native import PicolmHipError, check, lib


_initialised = False


def init(device: int = 0) -> None:
    """Selects the gfx950 device and creates the library stream (idempotent)."""
    global _initialised
    check(lib.plh_init(device), "plh_init")
    _initialised = True


def synchronize() -> None:
    check(lib.plh_synchronize(), "plh_synchronize")


class DeviceBuffer:
    """A raw HBM allocation.  `ptr` is the device address as an int."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = lib.plh_malloc(self.nbytes)
        if not p:
            raise PicolmHipError(f"plh_malloc({self.nbytes}) failed: {lib.plh_last_error()}")
        self.ptr = int(p)

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        check(lib.plh_memcpy_htod(self.ptr + offset, arr.ctypes.data, arr.nbytes), "htod")

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        check(lib.plh_memcpy_dtoh(out.ctypes.data, self.ptr + offset, out.nbytes), "dtoh")
        return out

    def copy_from(self, other: "DeviceBuffer", nbytes: int | None = None) -> None:
        n = self.nbytes if nbytes is None else nbytes
        check(lib.plh_memcpy_dtod(self.ptr, other.ptr, n), "dtod")

    def zero(self) -> None:
        check(lib.plh_memset(self.ptr, 0, self.nbytes), "memset")

    def free(self) -> None:
        if self.ptr:
            lib.plh_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    """hipEvent recorded on the library stream."""

    def __init__(self):
        self.h = lib.plh_event_create()
        if not self.h:
            raise PicolmHipError("plh_event_create failed")

    def record(self) -> None:
        check(lib.plh_event_record(self.h), "plh_event_record")

    def elapsed_ms(self, later: "Event") -> float:
        ms = lib.plh_event_elapsed_ms(self.h, later.h)
        if ms < 0:
            raise PicolmHipError("plh_event_elapsed_ms failed")
        return float(ms)

    def __del__(self):
        try:
            lib.plh_event_destroy(self.h)
        except Exception:
            pass


class Graph:
    """Captures what is queued on the library stream inside a `with` block."""

    def __init__(self):
        self.h = None

    def __enter__(self):
        check(lib.plh_capture_begin(), "plh_capture_begin")
        return self

    def __exit__(self, exc_type, exc, tb):
        h = lib.plh_capture_end()
        if exc_type is None and not h:
            raise PicolmHipError(f"graph capture failed: {lib.plh_last_error()}")
        self.h = h
        return False

    def launch(self) -> None:
        check(lib.plh_graph_launch(self.h), "plh_graph_launch")

    def __del__(self):
        try:
            if self.h:
                lib.plh_graph_destroy(self.h)
        except Exception:
            pass
