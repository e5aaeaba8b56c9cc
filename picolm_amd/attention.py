"""Host-side mirror of picolm's attention operator (Python view of the C ABI).

Names follow the reference: `AttnConfig` carries the model_config_t fields the
block reads (model.h:22-36), `KVCache` is the FP16 cache of run_state_t
(model.h:98-106) resident in HBM, and `decode` / `prefill` are the attention
blocks of model_forward_ex (model.c:819-892) and model_forward_prefill
(model.c:1039-1089).  Every call goes to libpicolm_hip; nothing here computes
attention on the CPU.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._native import check, lib
from .device import DeviceBuffer

ROPE_LLAMA = 0
ROPE_QWEN = 1


@dataclass(frozen=True)
class AttnConfig:
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    max_seq_len: int
    rope_freq_base: float = 10000.0
    rope_type: int = ROPE_LLAMA

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def cache_elems(self) -> int:
        return self.n_layers * self.max_seq_len * self.kv_dim


def rope_tables(max_seq_len: int, head_dim: int, base: float):
    """Host tables of model.c:545-556, computed by the library's C11 host code."""
    half = head_dim // 2
    cos_t = np.empty((max_seq_len, half), dtype=np.float32)
    sin_t = np.empty((max_seq_len, half), dtype=np.float32)
    lib.plh_rope_tables_host(cos_t.ctypes.data, sin_t.ctypes.data, max_seq_len, head_dim,
                             C.c_float(base))
    return cos_t, sin_t


class KVCache:
    """FP16 K and V caches [n_layers][max_seq_len][kv_dim] in HBM, zero-filled
    like the reference's calloc (model.c:612-619), plus device RoPE tables."""

    def __init__(self, cfg: AttnConfig):
        self.cfg = cfg
        nbytes = cfg.cache_elems * 2
        self.key = DeviceBuffer(nbytes)
        self.val = DeviceBuffer(nbytes)
        self.key.zero()
        self.val.zero()
        cos_t, sin_t = rope_tables(cfg.max_seq_len, cfg.head_dim, cfg.rope_freq_base)
        self.cos_host, self.sin_host = cos_t, sin_t
        self.cos = DeviceBuffer.from_numpy(cos_t)
        self.sin = DeviceBuffer.from_numpy(sin_t)

    def load(self, key_bits: np.ndarray, val_bits: np.ndarray) -> None:
        """Replaces the whole device cache with host fp16 bit patterns."""
        assert key_bits.dtype == np.uint16 and key_bits.size == self.cfg.cache_elems
        assert val_bits.dtype == np.uint16 and val_bits.size == self.cfg.cache_elems
        self.key.upload(key_bits)
        self.val.upload(val_bits)

    def fetch(self):
        shape = (self.cfg.cache_elems,)
        return self.key.download(np.uint16, shape), self.val.download(np.uint16, shape)

    def free(self) -> None:
        for b in (self.key, self.val, self.cos, self.sin):
            b.free()


def decode(cache: KVCache, layer0: int, pos: int, q: int, k: int, v: int, out: int,
           n_launch_layers: int = 1, q_norm: int | None = None, k_norm: int | None = None,
           norm_eps: float = 0.0) -> None:
    """Queues one decode step (device pointers q, k, v, out) for
    `n_launch_layers` layers starting at `layer0`.  q_norm / k_norm (device
    pointers to [n_launch_layers][head_dim] fp32) add Qwen3's QK-norm."""
    c = cache.cfg
    if q_norm is None and k_norm is None:
        check(lib.plh_attn_decode(c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.max_seq_len,
                                  c.rope_type, layer0, n_launch_layers, pos, q, k, v,
                                  cache.key.ptr, cache.val.ptr, cache.cos.ptr, cache.sin.ptr,
                                  out),
              "plh_attn_decode")
    else:
        check(lib.plh_attn_decode_qknorm(c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim,
                                         c.max_seq_len, c.rope_type, layer0, n_launch_layers,
                                         pos, q, k, v, cache.key.ptr, cache.val.ptr,
                                         cache.cos.ptr, cache.sin.ptr, out, q_norm, k_norm,
                                         norm_eps),
              "plh_attn_decode_qknorm")


def decode_rows(cache: KVCache, layer0: int, pos: int, q: int, k: int, v: int, out: int,
                k_rows: int, v_rows: int, n_launch_layers: int = 1, q_norm: int | None = None,
                k_norm: int | None = None, norm_eps: float = 0.0) -> None:
    """decode() that also writes the appended rows' fp16 bits to k_rows /
    v_rows ([n_launch_layers][kv_dim] uint16 each; any device-accessible
    pointers, pinned host memory included)."""
    c = cache.cfg
    check(lib.plh_attn_decode_rows(c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim,
                                   c.max_seq_len, c.rope_type, layer0, n_launch_layers, pos,
                                   q, k, v, cache.key.ptr, cache.val.ptr, cache.cos.ptr,
                                   cache.sin.ptr, out, q_norm, k_norm, norm_eps, k_rows, v_rows),
          "plh_attn_decode_rows")


def prefill(cache: KVCache, layer0: int, start_pos: int, n_tokens: int, q: int, k: int, v: int,
            out: int, out_stride: int | None = None, n_launch_layers: int = 1,
            q_norm: int | None = None, k_norm: int | None = None,
            norm_eps: float = 0.0) -> None:
    """Queues a causal prefill of n_tokens tokens at positions start_pos..
    (device pointers q [L][N][q_dim], k/v [L][N][kv_dim], out [L][N][stride]);
    q_norm / k_norm as in decode."""
    c = cache.cfg
    stride = c.q_dim if out_stride is None else out_stride
    if q_norm is None and k_norm is None:
        check(lib.plh_attn_prefill(c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim,
                                   c.max_seq_len, c.rope_type, layer0, n_launch_layers,
                                   start_pos, n_tokens, q, k, v, cache.key.ptr, cache.val.ptr,
                                   cache.cos.ptr, cache.sin.ptr, out, stride),
              "plh_attn_prefill")
    else:
        check(lib.plh_attn_prefill_qknorm(c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim,
                                          c.max_seq_len, c.rope_type, layer0, n_launch_layers,
                                          start_pos, n_tokens, q, k, v, cache.key.ptr,
                                          cache.val.ptr, cache.cos.ptr, cache.sin.ptr, out,
                                          stride, q_norm, k_norm, norm_eps),
              "plh_attn_prefill_qknorm")


def f32_to_f16(src: int, dst: int, n: int) -> None:
    """Device fp32 -> fp16 bits with the reference's rounding (quant.c:41-78)."""
    check(lib.plh_f32_to_f16(src, dst, n), "plh_f32_to_f16")


def f16_checksum(first: int, count: int) -> int:
    out = C.c_uint64(0)
    check(lib.plh_f16_checksum(first, count, C.byref(out)), "plh_f16_checksum")
    return int(out.value)
