"""Loads the product library lib/libpicolm_hip.so and declares its C ABI
(include/picolm_hip.h, include/gpu_hip.h).

There is no fallback: if the library is missing this import fails loudly.
Build it with `python -c "import __graft_entry__ as g; g.build()"` or
`make -C picolm_amd`.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# PICOLM_HIP_LIB points at a libpicolm_hip.so built elsewhere (same ABI).
LIB_PATH = os.environ.get("PICOLM_HIP_LIB") or os.path.join(HERE, "lib", "libpicolm_hip.so")


class PicolmHipError(RuntimeError):
    """A call into libpicolm_hip returned -1 (not handled / failed)."""


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `make -C {HERE}` (hipcc, gfx950)")
    return C.CDLL(LIB_PATH, mode=C.RTLD_GLOBAL)


lib = _load()

_vp = C.c_void_p
_i = C.c_int
_sz = C.c_size_t


# plh_model and its parts (include/picolm_hip.h)
class PlhMatrix(C.Structure):
    _fields_ = [("qtype", C.c_int), ("w", _vp)]


class PlhLayer(C.Structure):
    _fields_ = [("attn_norm", _vp), ("ffn_norm", _vp),
                ("q", PlhMatrix), ("k", PlhMatrix), ("v", PlhMatrix), ("o", PlhMatrix),
                ("gate", PlhMatrix), ("up", PlhMatrix), ("down", PlhMatrix),
                ("q_bias", _vp), ("k_bias", _vp), ("v_bias", _vp), ("o_bias", _vp),
                ("q_norm", _vp), ("k_norm", _vp)]


class PlhModel(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("n_embd", C.c_int), ("n_ffn", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int),
                ("vocab_size", C.c_int), ("max_seq_len", C.c_int), ("rope_type", C.c_int),
                ("rms_norm_eps", C.c_float), ("embd_type", C.c_int), ("token_embd", _vp),
                ("output_norm", _vp), ("output", PlhMatrix), ("key_cache", _vp),
                ("val_cache", _vp), ("rope_cos", _vp), ("rope_sin", _vp),
                ("layers", C.POINTER(PlhLayer))]


_SIGS = {
    # lifecycle
    "plh_init": (_i, [_i]),
    "plh_shutdown": (None, []),
    "plh_available": (_i, []),
    "plh_last_error": (C.c_char_p, []),
    "plh_device_count": (_i, []),
    # memory
    "plh_malloc": (_vp, [_sz]),
    "plh_free": (_i, [_vp]),
    "plh_memcpy_htod": (_i, [_vp, _vp, _sz]),
    "plh_memcpy_dtoh": (_i, [_vp, _vp, _sz]),
    "plh_memcpy_dtod": (_i, [_vp, _vp, _sz]),
    "plh_memcpy2d_dtoh": (_i, [_vp, _sz, _vp, _sz, _sz, _sz]),
    "plh_memcpy2d_htod": (_i, [_vp, _sz, _vp, _sz, _sz, _sz]),
    "plh_memset": (_i, [_vp, _i, _sz]),
    "plh_synchronize": (_i, []),
    "plh_host_alloc": (_vp, [_sz]),
    "plh_host_free": (_i, [_vp]),
    "plh_memcpy_htod_async": (_i, [_vp, _vp, _sz]),
    "plh_memcpy_dtoh_async": (_i, [_vp, _vp, _sz]),
    "plh_memcpy2d_dtoh_async": (_i, [_vp, _sz, _vp, _sz, _sz, _sz]),
    "plh_copy2d_batch_async": (_i, [_vp, _i]),
    # events
    "plh_event_create": (_vp, []),
    "plh_event_record": (_i, [_vp]),
    "plh_event_elapsed_ms": (C.c_float, [_vp, _vp]),
    "plh_event_destroy": (None, [_vp]),
    # graphs
    "plh_capture_begin": (_i, []),
    "plh_capture_end": (_vp, []),
    "plh_graph_launch": (_i, [_vp]),
    "plh_graph_destroy": (None, [_vp]),
    # tables, conversion
    "plh_rope_tables_host": (None, [_vp, _vp, _i, _i, C.c_float]),
    "plh_f32_to_f16": (_i, [_vp, _vp, _sz]),
    "plh_f16_checksum": (_i, [C.c_uint64, C.c_uint64, C.POINTER(C.c_uint64)]),
    # attention
    "plh_attn_decode": (_i, [_i] * 9 + [_vp] * 8),
    "plh_attn_decode_noalloc": (_i, [_i] * 9 + [_vp] * 8),
    "plh_attn_prefill": (_i, [_i] * 10 + [_vp] * 8 + [_i]),
    "plh_attn_decode_qknorm": (_i, [_i] * 9 + [_vp] * 10 + [C.c_float]),
    "plh_attn_decode_rows": (_i, [_i] * 9 + [_vp] * 10 + [C.c_float] + [_vp] * 2),
    "plh_attn_prefill_qknorm": (_i, [_i] * 10 + [_vp] * 8 + [_i, _vp, _vp, C.c_float]),
    # weight GEMV
    "plh_gemv_packed_bytes": (_sz, [_i, _i, _i]),
    "plh_gemv_upload": (_i, [_i, _i, _i, _vp, _vp]),
    "plh_gemv_pack_host": (_i, [_i, _i, _i, _vp, _vp]),
    "plh_gemv": (_i, [_i, _i, _i, _vp, _vp, _vp]),
    "plh_gemv_ex": (_i, [_i, _i, _i, _vp, _vp, _vp, _vp, C.c_float, _vp, _i, _vp, _vp]),
    "plh_gemv_swiglu": (_i, [_i, _i, _i, _vp, _vp, _vp, _vp, _vp, C.c_float]),
    "plh_matmul_batch": (_i, [_i, _i, _i, _vp, _vp, _i, _vp]),
    # forward pass
    "plh_rmsnorm": (_i, [_vp, _vp, _vp, _i, C.c_float]),
    "plh_dequantize_row": (_i, [_i, _vp, _vp, _i]),
    "plh_forward_workspace_bytes": (_sz, [C.POINTER(PlhModel)]),
    "plh_forward": (_i, [C.POINTER(PlhModel), _i, _i, _vp, _vp, _vp]),
    "plh_forward_prefill": (_i, [C.POINTER(PlhModel), _vp, _i, _i, _vp, _vp, _vp]),
    "plh_set_tuning": (_i, [_i, _i]),
}

for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args


def last_error() -> str:
    msg = lib.plh_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise PicolmHipError(f"{what} failed: {last_error()}")
