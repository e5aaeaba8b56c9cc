"""Weight GEMV (the path picolm's gpu_try_matmul offloads, gpu.c:579-702):
out = W @ x for GGUF Q4_K, Q6_K and Q8_0 matrices held in HBM, bit-identical
to the reference's matmul (tensor.c:200-215) in its x86-64 AVX2 build."""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._native import check, lib
from .device import DeviceBuffer

TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 8, 12, 14
BLOCK = {TYPE_Q8_0: (32, 34), TYPE_Q4_K: (256, 144), TYPE_Q6_K: (256, 210)}


def row_bytes(qtype: int, n: int) -> int:
    """gguf_type_row_size (quant.c:321-326) of the supported types."""
    if qtype not in BLOCK:
        raise ValueError(f"no GEMV for type {qtype}")
    w, b = BLOCK[qtype]
    return n // w * b


def pack_host(qtype: int, n: int, d: int, rows: np.ndarray) -> np.ndarray:
    """The device layout of a d x n matrix, built on the host (no GPU use)."""
    rows = np.ascontiguousarray(rows, np.uint8)
    if rows.size != d * row_bytes(qtype, n):
        raise ValueError("rows must hold d * row_bytes(qtype, n) bytes")
    size = lib.plh_gemv_packed_bytes(qtype, n, d)
    if size == 0:
        raise ValueError(f"no GEMV for type {qtype} with n={n}")
    out = np.empty(size, np.uint8)
    check(lib.plh_gemv_pack_host(qtype, n, d, rows.ctypes.data, out.ctypes.data),
          "plh_gemv_pack_host")
    return out


class QMatrix:
    """A d x n GGUF weight matrix uploaded (packed) into HBM."""

    def __init__(self, qtype: int, n: int, d: int, rows: np.ndarray):
        rows = np.ascontiguousarray(rows, np.uint8)
        if rows.size != d * row_bytes(qtype, n):
            raise ValueError("rows must hold d * row_bytes(qtype, n) bytes")
        size = lib.plh_gemv_packed_bytes(qtype, n, d)
        if size == 0:
            raise ValueError(f"no GEMV for type {qtype} with n={n}")
        self.qtype, self.n, self.d = qtype, n, d
        self.buf = DeviceBuffer(size)
        check(lib.plh_gemv_upload(qtype, n, d, rows.ctypes.data, self.buf.ptr),
              "plh_gemv_upload")

    @property
    def ptr(self) -> int:
        return self.buf.ptr

    def free(self) -> None:
        self.buf.free()


def matmul(out: int, x: int, W: QMatrix) -> None:
    """Queues out[d] = W @ x[n] (device pointers)."""
    check(lib.plh_gemv(W.qtype, W.n, W.d, C.c_void_p(W.ptr), C.c_void_p(x), C.c_void_p(out)),
          "plh_gemv")
