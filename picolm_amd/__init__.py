"""picolm_amd -- MI355X-native attention block of picolm (decode + prefill).

The product is libpicolm_hip.so (HIP kernels for gfx950 behind a C ABI,
include/picolm_hip.h and include/gpu_hip.h).  This package is its Python
view: `_native` binds the ABI (and fails loudly when the library is absent),
`device` wraps HBM buffers and events, `attention` mirrors the reference's
attention operator, `gemv` its weight matmul (the gpu_try_matmul path), `forward` the whole
forward pass (model_forward) and `synth` random models in GGUF layout.
"""
from ._native import LIB_PATH, PicolmHipError, check, lib  # noqa: F401
from .attention import (ROPE_LLAMA, ROPE_QWEN, AttnConfig, KVCache, decode, decode_rows,  # noqa: F401
                        f16_checksum, f32_to_f16, prefill, rope_tables)
from .device import DeviceBuffer, Event, Graph, init, synchronize  # noqa: F401
from .forward import DeviceModel  # noqa: F401
from .gemv import QMatrix, matmul  # noqa: F401
