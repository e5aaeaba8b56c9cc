"""Head dims without a tuned kernel: the reference runs every even head_dim
up to 256 (model.c:408 sets head_dim = n_embd / n_heads; its accumulator is
acc[256], model.c:856), the tuned kernels cover 64 and 128, and every other
one runs on attn_generic.hip through the same entry points.  Decode, prefill,
QK-norm and the decode-rows variant against the oracle: outputs within the
attention tolerance of tests/attn_check.py, K/V caches bit for bit."""
import pytest

import test_gpu_decode as TD
import test_gpu_decode_rows as TR
import test_gpu_prefill as TP
import test_gpu_qknorm as TQ

pytestmark = pytest.mark.gpu

# (n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, theta, rope_type, pos)
DECODE = [
    (2, 32, 32, 80, 300, 1e4, 0, 257),   # 80: MHA, one 256-row chunk and a tail
    (2, 32, 8, 96, 600, 1e4, 0, 513),    # 96: GQA 4, three chunks
    (2, 8, 4, 256, 300, 1e4, 0, 299),    # 256: the largest, last cache row
    (2, 6, 6, 48, 300, 1e4, 0, 0),       # position 0: only the appended row
    (2, 8, 2, 32, 600, 1e4, 1, 511),     # QWEN rotation, 32
    (1, 4, 2, 18, 100, 1e4, 0, 77),      # 18: rmsnorm tail of 2, odd pair count
    (1, 4, 1, 2, 50, 1e4, 1, 20),        # 2: one rope pair
]

# (n_layers, n_heads, n_kv_heads, head_dim, max_seq_len, theta, rope_type, start, n)
PREFILL = [
    (2, 32, 8, 96, 600, 1e4, 0, 0, 300),
    (2, 8, 4, 256, 400, 1e4, 1, 37, 200),
    (1, 6, 6, 48, 300, 1e4, 0, 230, 60),    # crosses the 256-position chunk
    (1, 4, 2, 18, 64, 1e4, 0, 5, 59),       # fills the cache to its last row
]


@pytest.mark.parametrize("case", DECODE, ids=[f"d{c[3]}_pos{c[7]}" for c in DECODE])
def test_decode_generic_head_dim(gpu, oracle_mod, case):
    L, Hq, Hkv, D, S, theta, rt, pos = case
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    TD.run_decode(gpu, oracle_mod, cfg, pos, seed=pos + 3 * D)


def test_decode_generic_per_layer_and_subrange(gpu, oracle_mod):
    cfg = gpu.AttnConfig(4, 12, 4, 80, 400, 1e4, 0)
    TD.run_decode(gpu, oracle_mod, cfg, 300, seed=8, per_layer=True)
    TD.run_decode(gpu, oracle_mod, cfg, 301, seed=9, layer_range=(1, 2))


def test_decode_generic_ignores_rows_past_pos(gpu, oracle_mod):
    cfg = gpu.AttnConfig(2, 8, 2, 96, 400, 1e4, 0)
    TD.run_decode(gpu, oracle_mod, cfg, 200, seed=10, poison=True)


@pytest.mark.parametrize("case", PREFILL, ids=[f"d{c[3]}_start{c[7]}_n{c[8]}" for c in PREFILL])
def test_prefill_generic_head_dim(gpu, oracle_mod, case):
    L, Hq, Hkv, D, S, theta, rt, start, n = case
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    TP.run_prefill(gpu, oracle_mod, cfg, start, n, seed=start + n + D)


def test_prefill_generic_strided_output(gpu, oracle_mod):
    cfg = gpu.AttnConfig(2, 4, 2, 18, 128, 1e4, 0)
    TP.run_prefill(gpu, oracle_mod, cfg, 10, 50, seed=4, out_stride=cfg.q_dim + 4, per_layer=True)


@pytest.mark.parametrize("dims", [(2, 8, 4, 96, 1024, 1e6, 1), (2, 6, 2, 36, 1024, 1e4, 0)],
                         ids=["d96_qwen", "d36_llama"])
@pytest.mark.parametrize("pos", [0, 300, 900])
def test_decode_qknorm_generic(gpu, oracle_mod, dims, pos):
    TQ.test_decode_qknorm(gpu, oracle_mod, dims, pos)


@pytest.mark.parametrize("dims", [(2, 8, 4, 96, 1024, 1e6, 1), (2, 6, 2, 36, 1024, 1e4, 0)],
                         ids=["d96_qwen", "d36_llama"])
def test_prefill_qknorm_generic(gpu, oracle_mod, dims):
    TQ.test_prefill_qknorm_chunks_then_decode(gpu, oracle_mod, dims)


@pytest.mark.parametrize("host_rows", [False, True], ids=["device_rows", "pinned_host_rows"])
def test_decode_rows_generic(gpu, host_rows):
    TR.test_decode_rows_match_plain_decode(gpu, (2, 8, 2, 96, 300, 1, 0, 2, 250, True),
                                           host_rows)


# Shapes the tuned prefill kernel does not take, routed to the generic kernels
# by plh_attn_prefill instead of being refused: an output row of 5 heads x 18
# floats (q_dim = 90, not a multiple of 4), and a GQA group of 136 q heads
# (more columns than one tuned workgroup holds) at the tuned head_dim 64.
@pytest.mark.parametrize("case", [(1, 5, 1, 18, 64, 1e4, 0, 3, 40),
                                  (1, 5, 5, 18, 64, 1e4, 1, 0, 33),
                                  (1, 136, 1, 64, 48, 1e4, 0, 2, 20)],
                         ids=["h5_d18_gqa5", "h5_d18_mha", "g136_d64"])
def test_prefill_untuned_shapes_use_generic(gpu, oracle_mod, case):
    L, Hq, Hkv, D, S, theta, rt, start, n = case
    cfg = gpu.AttnConfig(L, Hq, Hkv, D, S, theta, rt)
    TP.run_prefill(gpu, oracle_mod, cfg, start, n, seed=start + n + Hq)
