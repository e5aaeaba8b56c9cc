"""ctypes front-end of the test oracle (oracle/build/liboracle.so) and of the
reference harness (oracle/_ref/libpicolm_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke entry and the bench's
CPU-baseline leg, to check results against.  The product package never
imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libpicolm_ref.so")
REF_SRC = "/root/reference/picolm"

ROPE_LLAMA = 0
ROPE_QWEN = 1

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")

# GGUF type ids (quant.h:49-63) of the GEMV path
TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 2, 8, 12, 14
BLOCK = {TYPE_F32: (1, 4), TYPE_F16: (1, 2), TYPE_Q4_0: (32, 18), TYPE_Q8_0: (32, 34),
         TYPE_Q4_K: (256, 144), TYPE_Q6_K: (256, 210)}   # (weights, bytes) per block


def build(ref: bool | None = None) -> None:
    """Compile the oracle (and the reference harness when its sources exist)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if ref is None:
        ref = os.path.isdir(REF_SRC)
    if ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


class OrcMatrix(C.Structure):
    _fields_ = [("qtype", C.c_int), ("rows", C.c_void_p)]


class OrcLayer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
                ("q", OrcMatrix), ("k", OrcMatrix), ("v", OrcMatrix), ("o", OrcMatrix),
                ("gate", OrcMatrix), ("up", OrcMatrix), ("down", OrcMatrix),
                ("q_bias", C.c_void_p), ("k_bias", C.c_void_p), ("v_bias", C.c_void_p),
                ("o_bias", C.c_void_p), ("q_norm", C.c_void_p), ("k_norm", C.c_void_p)]


class OrcModel(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("n_embd", C.c_int), ("n_ffn", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int),
                ("vocab_size", C.c_int), ("max_seq_len", C.c_int), ("rope_type", C.c_int),
                ("rms_norm_eps", C.c_float), ("token_embd", OrcMatrix),
                ("output_norm", C.c_void_p), ("output", OrcMatrix), ("key_cache", C.c_void_p),
                ("val_cache", C.c_void_p), ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
                ("layers", C.POINTER(OrcLayer))]


_nf = C.POINTER(C.c_float)   # nullable float*
_lib = None
_ref = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(ref=False)
        L = C.CDLL(LIB_PATH)
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16_array.argtypes = [_f32p, _u16p, C.c_size_t]
        L.orc_f32_to_f16_array.restype = None
        L.orc_f16_to_f32_array.argtypes = [_u16p, _f32p, C.c_size_t]
        L.orc_f16_to_f32_array.restype = None
        L.orc_f16_checksum.argtypes = [C.c_uint64, C.c_uint64, C.c_int]
        L.orc_f16_checksum.restype = C.c_uint64
        L.orc_rope_tables.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_float]
        L.orc_rope_tables.restype = None
        L.orc_rope.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int, _f32p, _f32p, C.c_int]
        L.orc_rope.restype = None
        dims = [C.c_int] * 8
        L.orc_attn_decode.argtypes = dims + [_f32p, _f32p, _f32p, _u16p, _u16p, _f32p, _f32p, _f32p]
        L.orc_attn_decode.restype = C.c_int
        L.orc_attn_decode_mt.argtypes = dims + [_f32p, _f32p, _f32p, _u16p, _u16p, _f32p, _f32p,
                                                _f32p, C.c_int]
        L.orc_attn_decode_mt.restype = C.c_int
        L.orc_attn_prefill.argtypes = dims + [C.c_int, _f32p, _f32p, _f32p, _u16p, _u16p,
                                              _f32p, _f32p, _f32p, C.c_int]
        L.orc_attn_prefill.restype = C.c_int
        L.orc_attn_core.argtypes = [C.c_int] * 6 + [_f32p, _u16p, _u16p, _f32p]
        L.orc_attn_core.restype = C.c_int
        L.orc_attn_decode_qkn.argtypes = dims + [_f32p, _f32p, _f32p, _u16p, _u16p, _f32p, _f32p,
                                                 _f32p, _nf, _nf, C.c_float]
        L.orc_attn_decode_qkn.restype = C.c_int
        L.orc_attn_prefill_qkn.argtypes = dims + [C.c_int, _f32p, _f32p, _f32p, _u16p, _u16p,
                                                  _f32p, _f32p, _f32p, C.c_int, _nf, _nf,
                                                  C.c_float]
        L.orc_attn_prefill_qkn.restype = C.c_int
        L.orc_attn_prefill_mt.argtypes = dims + [C.c_int, _f32p, _f32p, _f32p, _u16p, _u16p,
                                                 _f32p, _f32p, _f32p, C.c_int, _nf, _nf,
                                                 C.c_float, C.c_int]
        L.orc_attn_prefill_mt.restype = C.c_int
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_float]
        L.orc_rmsnorm.restype = None
        for name in ("orc_vec_dot_q4_K", "orc_vec_dot_q6_K", "orc_vec_dot_q8_0",
                     "orc_vec_dot_f32"):
            getattr(L, name).argtypes = [_u8p, _f32p, C.c_int]
            getattr(L, name).restype = C.c_float
        L.orc_dequantize_row.argtypes = [C.c_int, _u8p, _f32p, C.c_int]
        L.orc_dequantize_row.restype = None
        L.orc_matmul.argtypes = [_f32p, _f32p, _u8p, C.c_int, C.c_int, C.c_int]
        L.orc_matmul.restype = C.c_int
        L.orc_matmul_mt.argtypes = [_f32p, _f32p, _u8p, C.c_int, C.c_int, C.c_int, C.c_int]
        L.orc_matmul_mt.restype = C.c_int
        L.orc_silu.argtypes = [C.c_float]
        L.orc_silu.restype = C.c_float
        L.orc_forward.argtypes = [C.POINTER(OrcModel), C.c_int, C.c_int, _f32p, _nf, C.c_int]
        L.orc_forward.restype = C.c_int
        L.orc_forward_prefill.argtypes = [C.POINTER(OrcModel), _i32p, C.c_int, C.c_int, _f32p,
                                          _nf, C.c_int]
        L.orc_forward_prefill.restype = C.c_int
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> C.CDLL:
    global _ref
    if _ref is None:
        R = C.CDLL(REF_PATH)
        R.fp32_to_fp16.argtypes = [C.c_float]
        R.fp32_to_fp16.restype = C.c_uint16
        R.fp16_to_fp32.argtypes = [C.c_uint16]
        R.fp16_to_fp32.restype = C.c_float
        R.rope.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int, _f32p, _f32p, C.c_int]
        R.rope.restype = None
        R.ref_model_new.argtypes = [C.c_int] * 5 + [C.c_float, C.c_int, C.c_int, C.c_ulonglong, C.c_float]
        R.ref_model_new.restype = C.c_void_p
        R.ref_model_free.argtypes = [C.c_void_p]
        R.ref_model_free.restype = None
        R.ref_cache_ptrs.argtypes = [C.c_void_p] + [C.POINTER(C.c_void_p)] * 4
        R.ref_cache_ptrs.restype = None
        R.ref_set_decode_qkv.argtypes = [C.c_void_p, C.c_int, _f32p, _f32p, _f32p]
        R.ref_set_decode_qkv.restype = None
        R.ref_decode.argtypes = [C.c_void_p, C.c_int, C.c_int, _f32p]
        R.ref_decode.restype = None
        R.ref_prefill.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_int, _f32p]
        R.ref_prefill.restype = None
        R.ref_embed.argtypes = [C.c_void_p, _i32p, C.c_int, _f32p]
        R.ref_embed.restype = None
        R.ref_layer_inputs.argtypes = [C.c_void_p, C.c_int, _f32p, C.c_int, _f32p, _f32p, _f32p]
        R.ref_layer_inputs.restype = None
        R.ref_final_norm.argtypes = [C.c_void_p, _f32p, _f32p]
        R.ref_final_norm.restype = None
        R.ref_set_qk_norm.argtypes = [C.c_void_p, C.c_int, _f32p, _f32p, C.c_float]
        R.ref_set_qk_norm.restype = None
        R.ref_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_float]
        R.ref_rmsnorm.restype = None
        for name in ("vec_dot_q4_K_f32", "vec_dot_q6_K_f32", "vec_dot_q8_0_f32",
                     "vec_dot_f32_f32"):
            getattr(R, name).argtypes = [_u8p, _f32p, C.c_int]
            getattr(R, name).restype = C.c_float
        R.vec_dot.argtypes = [_u8p, _f32p, C.c_int, C.c_int]
        R.vec_dot.restype = C.c_float
        R.dequantize_row.argtypes = [_u8p, _f32p, C.c_int, C.c_int]
        R.dequantize_row.restype = None
        R.ref_model_new_full.argtypes = [_i32p, C.c_float, C.c_float, C.POINTER(C.c_void_p),
                                         _i32p]
        R.ref_model_new_full.restype = C.c_void_p
        R.ref_forward.argtypes = [C.c_void_p, C.c_int, C.c_int, _f32p, _f32p]
        R.ref_forward.restype = None
        R.ref_forward_prefill.argtypes = [C.c_void_p, _i32p, C.c_int, C.c_int, _f32p, _f32p]
        R.ref_forward_prefill.restype = None
        R.ref_silu.argtypes = [_f32p, C.c_int]
        R.ref_silu.restype = None
        R.ref_set_threads.argtypes = [C.c_int]
        R.ref_set_threads.restype = None
        _ref = R
    return _ref


# ---------------------------------------------------------------------------
# numpy conveniences
# ---------------------------------------------------------------------------

def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(h.reshape(-1), out.reshape(-1), h.size)
    return out


def rope_tables(max_seq_len: int, head_dim: int, base: float):
    half = head_dim // 2
    c = np.empty((max_seq_len, half), dtype=np.float32)
    s = np.empty((max_seq_len, half), dtype=np.float32)
    lib().orc_rope_tables(c.reshape(-1), s.reshape(-1), max_seq_len, head_dim, base)
    return c, s


def rope(q, k, head_dim, n_heads, n_kv_heads, cos_row, sin_row, rope_type):
    """In-place RoPE of one token's q [n_heads*D] and k [n_kv_heads*D]."""
    lib().orc_rope(q, k, head_dim, n_heads, n_kv_heads,
                   np.ascontiguousarray(cos_row, np.float32),
                   np.ascontiguousarray(sin_row, np.float32), rope_type)


class Shape:
    """Attention shape: n_layers, n_heads, n_kv_heads, head_dim, max_seq_len."""

    def __init__(self, n_layers, n_heads, n_kv_heads, head_dim, max_seq_len,
                 rope_base=10000.0, rope_type=ROPE_LLAMA):
        self.n_layers = n_layers
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.rope_base = rope_base
        self.rope_type = rope_type

    @property
    def q_dim(self):
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    def cache_elems(self):
        return self.n_layers * self.max_seq_len * self.kv_dim

    def dims(self):
        return (self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim,
                self.max_seq_len, self.rope_type)


def _nullable(a):
    if a is None:
        return None
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a.ctypes.data_as(C.POINTER(C.c_float))


def attn_decode(shp: Shape, layer, pos, q, k, v, kc, vc, cos_t, sin_t,
                q_norm=None, k_norm=None, eps=0.0):
    """Oracle decode step; q, k rotated in place, caches appended in place.
    q_norm / k_norm ([head_dim] each) apply Qwen3's QK-norm with epsilon eps."""
    out = np.empty(shp.q_dim, dtype=np.float32)
    if q_norm is None and k_norm is None:
        rc = lib().orc_attn_decode(*shp.dims(), layer, pos, q, k, v, kc, vc,
                                   cos_t.reshape(-1), sin_t.reshape(-1), out)
    else:
        qn = None if q_norm is None else np.ascontiguousarray(q_norm, np.float32)
        kn = None if k_norm is None else np.ascontiguousarray(k_norm, np.float32)
        rc = lib().orc_attn_decode_qkn(*shp.dims(), layer, pos, q, k, v, kc, vc,
                                       cos_t.reshape(-1), sin_t.reshape(-1), out,
                                       _nullable(qn), _nullable(kn), eps)
    if rc != 0:
        raise ValueError("orc_attn_decode rejected its arguments")
    return out


def rmsnorm(x, w, eps):
    """The reference's rmsnorm (x86-64 AVX2 build order) of one vector."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm(out, x, np.ascontiguousarray(w, np.float32), x.size, eps)
    return out


def attn_decode_mt(shp: Shape, layer, pos, q, k, v, kc, vc, cos_t, sin_t, n_threads):
    """attn_decode with the q heads split over n_threads host threads
    (bit-identical output); the CPU baseline's head-parallel upper bound."""
    out = np.empty(shp.q_dim, dtype=np.float32)
    rc = lib().orc_attn_decode_mt(*shp.dims(), layer, pos, q, k, v, kc, vc,
                                  cos_t.reshape(-1), sin_t.reshape(-1), out, n_threads)
    if rc != 0:
        raise ValueError("orc_attn_decode_mt rejected its arguments")
    return out


def attn_prefill(shp: Shape, layer, start_pos, n_tokens, q, k, v, kc, vc,
                 cos_t, sin_t, out_stride=None, q_norm=None, k_norm=None, eps=0.0):
    stride = shp.q_dim if out_stride is None else out_stride
    out = np.zeros(max(n_tokens, 1) * stride, dtype=np.float32)
    if q_norm is None and k_norm is None:
        rc = lib().orc_attn_prefill(*shp.dims(), layer, start_pos, n_tokens,
                                    q.reshape(-1), k.reshape(-1), v.reshape(-1),
                                    kc, vc, cos_t.reshape(-1), sin_t.reshape(-1),
                                    out, stride)
    else:
        qn = None if q_norm is None else np.ascontiguousarray(q_norm, np.float32)
        kn = None if k_norm is None else np.ascontiguousarray(k_norm, np.float32)
        rc = lib().orc_attn_prefill_qkn(*shp.dims(), layer, start_pos, n_tokens,
                                        q.reshape(-1), k.reshape(-1), v.reshape(-1),
                                        kc, vc, cos_t.reshape(-1), sin_t.reshape(-1),
                                        out, stride, _nullable(qn), _nullable(kn), eps)
    if rc != 0:
        raise ValueError("orc_attn_prefill rejected its arguments")
    return out[: n_tokens * stride].reshape(n_tokens, stride)


def attn_prefill_mt(shp: Shape, layer, start_pos, n_tokens, q, k, v, kc, vc, cos_t, sin_t,
                    n_threads, q_norm=None, k_norm=None, eps=0.0):
    """attn_prefill with the attention split by q head over n_threads host
    threads (bit-identical output); the CPU baseline's head-parallel upper
    bound."""
    stride = shp.q_dim
    out = np.zeros(max(n_tokens, 1) * stride, dtype=np.float32)
    qn = None if q_norm is None else np.ascontiguousarray(q_norm, np.float32)
    kn = None if k_norm is None else np.ascontiguousarray(k_norm, np.float32)
    rc = lib().orc_attn_prefill_mt(*shp.dims(), layer, start_pos, n_tokens,
                                   q.reshape(-1), k.reshape(-1), v.reshape(-1),
                                   kc, vc, cos_t.reshape(-1), sin_t.reshape(-1),
                                   out, stride, _nullable(qn), _nullable(kn), eps, n_threads)
    if rc != 0:
        raise ValueError("orc_attn_prefill_mt rejected its arguments")
    return out[: n_tokens * stride].reshape(n_tokens, stride)


def attn_core(shp: Shape, layer, pos, q, kc, vc):
    out = np.empty(shp.q_dim, dtype=np.float32)
    rc = lib().orc_attn_core(shp.n_heads, shp.n_kv_heads, shp.head_dim,
                             shp.max_seq_len, layer, pos,
                             np.ascontiguousarray(q, np.float32), kc, vc, out)
    if rc != 0:
        raise ValueError("orc_attn_core rejected its arguments")
    return out


class RefModel:
    """The reference's own forward pass on a tiny model (oracle/ref_harness.c)."""

    def __init__(self, shp: Shape, mode: int, seed: int = 1, w_scale: float = 0.25):
        R = ref()
        self.shp = shp
        self.h = R.ref_model_new(shp.n_layers, shp.n_heads, shp.n_kv_heads,
                                 shp.head_dim, shp.max_seq_len, shp.rope_base,
                                 shp.rope_type, mode, seed, w_scale)
        if not self.h:
            raise MemoryError("ref_model_new failed")
        ptrs = [C.c_void_p() for _ in range(4)]
        R.ref_cache_ptrs(self.h, *[C.byref(p) for p in ptrs])
        n = shp.cache_elems()
        half = shp.head_dim // 2
        self.kc = np.ctypeslib.as_array(C.cast(ptrs[0], C.POINTER(C.c_uint16)), (n,))
        self.vc = np.ctypeslib.as_array(C.cast(ptrs[1], C.POINTER(C.c_uint16)), (n,))
        self.cos = np.ctypeslib.as_array(C.cast(ptrs[2], C.POINTER(C.c_float)),
                                         (shp.max_seq_len, half))
        self.sin = np.ctypeslib.as_array(C.cast(ptrs[3], C.POINTER(C.c_float)),
                                         (shp.max_seq_len, half))

    def close(self):
        if self.h:
            ref().ref_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


# ---------------------------------------------------------------------------
# weight GEMV (gpu_try_matmul's path)
# ---------------------------------------------------------------------------

def row_bytes(qtype: int, n: int) -> int:
    w, b = BLOCK[qtype]
    return n // w * b


def matmul(W: np.ndarray, x: np.ndarray, n: int, d: int, qtype: int) -> np.ndarray:
    """out[i] = vec_dot(row i of W, x) in the reference's x86-64 (AVX2) order."""
    out = np.empty(d, np.float32)
    rc = lib().orc_matmul(out, np.ascontiguousarray(x, np.float32),
                          np.ascontiguousarray(W, np.uint8).reshape(-1), n, d, qtype)
    if rc != 0:
        raise ValueError(f"no fused dot product for type {qtype}")
    return out


def matmul_mt(W: np.ndarray, x: np.ndarray, n: int, d: int, qtype: int,
              n_threads: int) -> np.ndarray:
    """matmul with rows split over n_threads host threads (bit-identical)."""
    out = np.empty(d, np.float32)
    rc = lib().orc_matmul_mt(out, np.ascontiguousarray(x, np.float32),
                             np.ascontiguousarray(W, np.uint8).reshape(-1), n, d, qtype,
                             n_threads)
    if rc != 0:
        raise ValueError(f"no fused dot product for type {qtype}")
    return out


def dequantize(W: np.ndarray, n: int, d: int, qtype: int) -> np.ndarray:
    W = np.ascontiguousarray(W, np.uint8).reshape(d, -1)
    out = np.empty((d, n), np.float32)
    for i in range(d):
        lib().orc_dequantize_row(qtype, np.ascontiguousarray(W[i]), out[i], n)
    return out


# ---------------------------------------------------------------------------
# whole forward pass (model_forward / model_forward_prefill)
# ---------------------------------------------------------------------------

LAYER_MATRICES = ("q", "k", "v", "o", "gate", "up", "down")


def _ptr(a):
    return None if a is None else a.ctypes.data


class OracleForward:
    """The oracle's forward pass over a host model (attributes as in the
    product's synth.SynthModel: config ints, rope_base, eps, embd_type,
    token_embd, output_norm, output_type, output, layers), with its own
    zero-filled host KV caches and RoPE tables."""

    def __init__(self, h):
        self.h = h
        self.kc = np.zeros(h.cache_elems(), np.uint16)
        self.vc = np.zeros(h.cache_elems(), np.uint16)
        self.cos, self.sin = rope_tables(h.max_seq_len, h.head_dim, h.rope_base)
        self.layers = (OrcLayer * h.n_layers)()
        for li, L in enumerate(h.layers):
            ol = self.layers[li]
            ol.attn_norm, ol.ffn_norm = _ptr(L["attn_norm"]), _ptr(L["ffn_norm"])
            for name in LAYER_MATRICES:
                qt, rows = L[name]
                setattr(ol, name, OrcMatrix(qt, rows.ctypes.data))
            for name in ("q_bias", "k_bias", "v_bias", "o_bias", "q_norm", "k_norm"):
                setattr(ol, name, _ptr(L[name]))
        self.m = OrcModel(h.n_layers, h.n_embd, h.n_ffn, h.n_heads, h.n_kv_heads, h.head_dim,
                          h.vocab_size, h.max_seq_len, h.rope_type, h.eps,
                          OrcMatrix(h.embd_type, h.token_embd.ctypes.data),
                          h.output_norm.ctypes.data, OrcMatrix(h.output_type, h.output.ctypes.data),
                          self.kc.ctypes.data, self.vc.ctypes.data, self.cos.ctypes.data,
                          self.sin.ctypes.data, C.cast(self.layers, C.POINTER(OrcLayer)))

    def forward(self, token: int, pos: int, n_threads: int = 1):
        logits = np.empty(self.h.vocab_size, np.float32)
        x = np.empty(self.h.n_embd, np.float32)
        rc = lib().orc_forward(C.byref(self.m), token, pos, logits,
                               x.ctypes.data_as(_nf), n_threads)
        if rc != 0:
            raise ValueError("orc_forward rejected its arguments")
        return logits, x

    def prefill(self, tokens, start_pos: int, n_threads: int = 1):
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.h.vocab_size, np.float32)
        x = np.empty(self.h.n_embd, np.float32)
        rc = lib().orc_forward_prefill(C.byref(self.m), t, len(t), start_pos, logits,
                                       x.ctypes.data_as(_nf), n_threads)
        if rc != 0:
            raise ValueError("orc_forward_prefill rejected its arguments")
        return logits, x


class RefForward:
    """The reference's own model_forward / model_forward_prefill on the same
    host buffers (oracle/_ref, ref_harness.c ref_model_new_full)."""

    def __init__(self, h):
        R = ref()
        self.h = h
        cfg = np.array([h.n_layers, h.n_embd, h.n_ffn, h.n_heads, h.n_kv_heads, h.head_dim,
                        h.vocab_size, h.max_seq_len, h.rope_type], np.int32)
        ptrs = [h.token_embd, h.output_norm, h.output]
        types = [h.embd_type, TYPE_F32, h.output_type]
        for L in h.layers:
            ptrs += [L["attn_norm"], L["q"][1], L["k"][1], L["v"][1], L["o"][1], L["q_norm"],
                     L["k_norm"], L["ffn_norm"], L["gate"][1], L["down"][1], L["up"][1],
                     L["q_bias"], L["k_bias"], L["v_bias"], L["o_bias"]]
            types += [TYPE_F32, L["q"][0], L["k"][0], L["v"][0], L["o"][0], TYPE_F32, TYPE_F32,
                      TYPE_F32, L["gate"][0], L["down"][0], L["up"][0], TYPE_F32, TYPE_F32,
                      TYPE_F32, TYPE_F32]
        self._ptrs = (C.c_void_p * len(ptrs))(*[_ptr(a) for a in ptrs])
        self.handle = R.ref_model_new_full(cfg, h.rope_base, h.eps, self._ptrs,
                                           np.array(types, np.int32))
        if not self.handle:
            raise MemoryError("ref_model_new_full failed")
        p = [C.c_void_p() for _ in range(4)]
        R.ref_cache_ptrs(self.handle, *[C.byref(x) for x in p])
        n = h.cache_elems()
        self.kc = np.ctypeslib.as_array(C.cast(p[0], C.POINTER(C.c_uint16)), (n,))
        self.vc = np.ctypeslib.as_array(C.cast(p[1], C.POINTER(C.c_uint16)), (n,))

    def forward(self, token: int, pos: int):
        logits = np.empty(self.h.vocab_size, np.float32)
        x = np.empty(self.h.n_embd, np.float32)
        ref().ref_forward(self.handle, token, pos, logits, x)
        return logits, x

    def prefill(self, tokens, start_pos: int):
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.h.vocab_size, np.float32)
        x = np.empty(self.h.n_embd, np.float32)
        ref().ref_forward_prefill(self.handle, t, len(t), start_pos, logits, x)
        return logits, x

    def close(self):
        if self.handle:
            ref().ref_model_free(self.handle)
            self.handle = None

    def __del__(self):
        self.close()
