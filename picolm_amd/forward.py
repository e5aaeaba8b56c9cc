"""Whole forward pass on the device (picolm's model_forward_ex,
model.c:746-925): embedding, every layer's norms, projections, attention and
SwiGLU, the final norm and the logits, queued on the library stream by
plh_forward (include/picolm_hip.h).

DeviceModel uploads a model held in host buffers (the reference's GGUF rows,
e.g. a synth.SynthModel) once: packed projection matrices, fp32 norms and
biases, the raw embedding rows, the FP16 KV caches and the RoPE tables.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._native import PlhLayer, PlhMatrix, PlhModel, check, lib
from .attention import rope_tables
from .device import DeviceBuffer
from .gemv import QMatrix

LAYER_MATRICES = ("q", "k", "v", "o", "gate", "up", "down")


class DeviceModel:
    """A host model (attributes as in synth.SynthModel) resident in HBM."""

    def __init__(self, host):
        self.host = host
        h = host
        self._keep = []          # device buffers the descriptor points into

        def dev(arr):
            if arr is None:
                return None
            b = DeviceBuffer.from_numpy(arr)
            self._keep.append(b)
            return b.ptr

        self.layers = (PlhLayer * h.n_layers)()
        for li, L in enumerate(h.layers):
            pl = self.layers[li]
            pl.attn_norm, pl.ffn_norm = dev(L["attn_norm"]), dev(L["ffn_norm"])
            shapes = dict(q=(h.n_embd, h.q_dim), k=(h.n_embd, h.kv_dim), v=(h.n_embd, h.kv_dim),
                          o=(h.q_dim, h.n_embd), gate=(h.n_embd, h.n_ffn),
                          up=(h.n_embd, h.n_ffn), down=(h.n_ffn, h.n_embd))
            for name in LAYER_MATRICES:
                qt, rows = L[name]
                # every layer gets its own copy, also when the host bytes are
                # shared, so a token streams every layer's weights from HBM
                W = QMatrix(qt, *shapes[name], rows)
                self._keep.append(W)
                setattr(pl, name, PlhMatrix(qt, W.ptr))
            for name in ("q_bias", "k_bias", "v_bias", "o_bias", "q_norm", "k_norm"):
                setattr(pl, name, dev(L[name]))
        self.out_matrix = QMatrix(h.output_type, h.n_embd, h.vocab_size, h.output)
        self.embd = DeviceBuffer.from_numpy(h.token_embd)
        self.output_norm = DeviceBuffer.from_numpy(h.output_norm)
        nkv = h.cache_elems() * 2
        self.key = DeviceBuffer(nkv)
        self.val = DeviceBuffer(nkv)
        self.key.zero()
        self.val.zero()
        self.cos_host, self.sin_host = rope_tables(h.max_seq_len, h.head_dim, h.rope_base)
        self.cos = DeviceBuffer.from_numpy(self.cos_host)
        self.sin = DeviceBuffer.from_numpy(self.sin_host)
        self.desc = PlhModel(h.n_layers, h.n_embd, h.n_ffn, h.n_heads, h.n_kv_heads,
                             h.head_dim, h.vocab_size, h.max_seq_len, h.rope_type, h.eps,
                             h.embd_type, self.embd.ptr, self.output_norm.ptr,
                             PlhMatrix(h.output_type, self.out_matrix.ptr), self.key.ptr,
                             self.val.ptr, self.cos.ptr, self.sin.ptr,
                             C.cast(self.layers, C.POINTER(PlhLayer)))
        ws = lib.plh_forward_workspace_bytes(C.byref(self.desc))
        self.workspace = DeviceBuffer(ws)
        self.logits = DeviceBuffer(h.vocab_size * 4)
        self.x_out = DeviceBuffer(h.n_embd * 4)

    def forward(self, token: int, pos: int, logits: int | None = None,
                x_out: int | None = None) -> None:
        """Queues model_forward(token, pos); logits / x_out default to this
        model's own device buffers."""
        check(lib.plh_forward(C.byref(self.desc), int(token), int(pos), self.workspace.ptr,
                              self.logits.ptr if logits is None else logits,
                              self.x_out.ptr if x_out is None else x_out), "plh_forward")

    def prefill(self, tokens, start_pos: int, logits: int | None = None,
                x_out: int | None = None) -> None:
        """Queues model_forward_prefill(tokens, start_pos): logits of the
        last token."""
        t = np.ascontiguousarray(tokens, np.int32)
        check(lib.plh_forward_prefill(C.byref(self.desc), t.ctypes.data, len(t), int(start_pos),
                                      self.workspace.ptr,
                                      self.logits.ptr if logits is None else logits,
                                      self.x_out.ptr if x_out is None else x_out),
              "plh_forward_prefill")

    def fetch_logits(self) -> np.ndarray:
        return self.logits.download(np.float32, (self.host.vocab_size,))

    def fetch_x(self) -> np.ndarray:
        return self.x_out.download(np.float32, (self.host.n_embd,))

    def fetch_cache(self):
        n = self.host.cache_elems()
        return self.key.download(np.uint16, (n,)), self.val.download(np.uint16, (n,))

    def load_cache(self, key_bits: np.ndarray, val_bits: np.ndarray) -> None:
        self.key.upload(np.ascontiguousarray(key_bits, np.uint16))
        self.val.upload(np.ascontiguousarray(val_bits, np.uint16))

    def free(self) -> None:
        for b in self._keep:
            b.free()
        for b in (self.out_matrix, self.embd, self.output_norm, self.key, self.val, self.cos,
                  self.sin, self.workspace, self.logits, self.x_out):
            b.free()
        self._keep = []
