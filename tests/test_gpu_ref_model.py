"""The drop-in check: picolm's OWN model_t through the gpu.h-style boundary.

tests/c/test_ref_model is built here against the reference's model.h, with
gpu_hip.c compiled in and the reference's model.c / tensor.c / quant.c linked
from oracle/_ref (make -C tests/c ref).  Every model_t it uses comes from the
reference's allocate_run_state, and every CPU result from the reference's
own model_forward_ex / model_forward / model_forward_prefill / matmul /
kvcache_save / kvcache_load, so a field-offset mismatch between this
package's host/model.h and picolm's would show here as a wrong result.

Checks, attention hooks (injection model: q/k/v exact through the biases):
gpu_init / gpu_upload_model return 0; gpu_try_attention_prefill and
gpu_try_attention match the reference within the attention tolerance (and
the tight PREC bound); the host caches equal the CPU model's bit for bit;
gpu_kv_download restores cleared host caches; kvcache_save of the GPU model
writes the same bytes as the CPU model's; a fresh model that kvcache_load's
that file and gpu_kv_upload's it continues decoding on the device in step
with the CPU model.  Whole forward pass: gpu_try_forward(_prefill) logits
and state.x against the reference's, caches (layer 0 bit-exact), and
gpu_try_matmul bit-exact against the reference's matmul on every matrix."""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from picolm_amd import synth as S
from test_gpu_boundary_forward import CFG, QWEN, write_model, normwise, FWD_TOL

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "tests", "c", "test_ref_model")
needs_exe = pytest.mark.skipif(
    not os.path.exists(EXE),
    reason="tests/c/test_ref_model not built (make -C oracle ref && make -C tests/c ref, "
           "needs the reference sources)")
PREC = 5e-5


def run_attn(tmp_path, L, Hq, Hkv, D, S_, rt, P, T, R, seed, env_extra=None):
    out = tmp_path / "attn.txt"
    args = [EXE, "attn"] + [str(a) for a in (L, Hq, Hkv, D, S_, rt, P, T, R, seed)] + [str(out)]
    env = dict(os.environ)
    env["PICOLM_HIP_GEMV_EXACT"] = "1"   # gpu_try_matmul bit-exact against the reference
    env.update(env_extra or {})
    print(f"[case] ref-model attn {args[2:-1]} env {env_extra}", flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=240, env=env)
    assert r.returncode == 0, r.stderr
    kv = dict(item.split("=") for item in out.read_text().split())
    return {k: float(v) if "err" in k else int(v) for k, v in kv.items()}


ATTN_CASES = [
    # L, Hq, Hkv, D, S, rope, prompt, decode, resume
    (2, 32, 4, 64, 64, 0, 9, 4, 3),     # TinyLlama heads
    (2, 12, 2, 64, 48, 0, 7, 3, 2),     # GQA 6
    (2, 4, 4, 128, 40, 1, 5, 3, 2),     # MHA, D 128, QWEN rotation
]


@needs_exe
@pytest.mark.parametrize("case", ATTN_CASES, ids=["gqa8_d64", "gqa6_d64", "mha_d128_qwen"])
def test_attention_hooks_with_reference_model(tmp_path, case):
    r = run_attn(tmp_path, *case, seed=11)
    P, T, R = case[6], case[7], case[8]
    assert r["rc_init"] == 0 and r["rc_upload"] == 0
    assert r["prefill_rc"] == 0 and r["decode_rc"] == 0 and r["resume_rc"] == 0
    for phase in ("prefill", "decode", "resume"):
        assert r[f"{phase}_err"] <= PREC, (phase, r)
        assert r[f"{phase}_bad"] == 0, (phase, r)
    assert r["prefill_cache_eq"] == 1 and r["decode_cache_eq"] == 1
    # persistence with the reference's own file code
    assert r["rc_download"] == 0 and r["download_eq"] == 1
    assert r["rc_save"] == 0 and r["file_eq"] == 1
    assert r["rc_reinit"] == 0 and r["rc_reupload"] == 0
    assert r["loaded"] == P + T and r["rc_kv_upload"] == 0
    assert r["resume_cache_eq"] == 1
    assert r["prefill_fallback"] == 0 and r["decode_fallback"] == 0 and r["resume_fallback"] == 0


@needs_exe
@pytest.mark.parametrize("fail_after", [1, 3, 8])
def test_injected_failure_falls_back_to_the_reference(tmp_path, fail_after):
    """PICOLM_HIP_FAIL_AFTER=N: the attention hook call after N successful
    ones fails after its kernels ran (device cache ahead of the host's), the
    backend is lost, and the harness answers every later -1 as picolm's call
    sites do, with the reference's CPU block on the same model_t.  Outputs stay
    within the bound and the host caches -- the only copy once the device is
    lost -- equal the CPU model's bit for bit; kvcache_save writes the same
    file, and a fresh model (whose own gpu_init re-arms the switch) resumes
    from it.  Calls: prefill 2 layers, then 4 tokens x 2 layers, then 3 x 2."""
    L, P, T, R = 2, 9, 4, 3
    r = run_attn(tmp_path, L, 32, 4, 64, 64, 0, P, T, R, seed=13,
                 env_extra={"PICOLM_HIP_FAIL_AFTER": str(fail_after)})
    assert r["rc_init"] == 0 and r["rc_upload"] == 0
    for phase in ("prefill", "decode", "resume"):
        assert r[f"{phase}_err"] <= PREC, (phase, r)
        assert r[f"{phase}_bad"] == 0, (phase, r)
    # hook calls before the failure succeed; the failing call and all later
    # ones of the same backend fall back
    calls = [L] + [T * L]
    pre_ok = min(fail_after, L)
    dec_ok = min(max(fail_after - L, 0), T * L)
    assert r["prefill_fallback"] == L - pre_ok
    assert r["decode_fallback"] == T * L - dec_ok
    assert (r["prefill_rc"] == 0) == (pre_ok == L)
    assert (r["decode_rc"] == 0) == (dec_ok == T * L)
    assert r["prefill_cache_eq"] == 1 and r["decode_cache_eq"] == 1
    lost = fail_after < sum(calls)
    assert r["rc_download"] == (-1 if lost else 0) and r["download_eq"] == 1
    assert r["rc_save"] == 0 and r["file_eq"] == 1
    assert r["rc_reinit"] == 0 and r["rc_reupload"] == 0
    assert r["loaded"] == P + T and r["rc_kv_upload"] == 0
    assert r["resume_fallback"] == R * L - min(fail_after, R * L)
    assert r["resume_cache_eq"] == 1


def run_forward(tmp_path, h, steps):
    fin, fout = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(fin, "wb") as f:
        write_model(f, h)
        np.array([len(steps)], np.int32).tofile(f)
        for kind, start, toks in steps:
            np.array([kind, start, len(toks)] + list(toks), np.int32).tofile(f)
    print(f"[case] ref-model forward {h.n_layers}x{h.n_embd} steps {len(steps)}", flush=True)
    env = dict(os.environ)
    env["PICOLM_HIP_GEMV_EXACT"] = "1"   # gpu_try_matmul bit-exact against the reference
    r = subprocess.run([EXE, "forward", str(fin), str(fout)], capture_output=True, text=True,
                       timeout=240, env=env)
    assert r.returncode == 0, r.stderr
    buf = open(fout, "rb").read()
    off = 0

    def take(dtype, count):
        nonlocal off
        a = np.frombuffer(buf, dtype=dtype, count=count, offset=off)
        off += a.nbytes
        return a
    rcs = tuple(int(v) for v in take(np.int32, 2))
    res = []
    for _ in steps:
        rc = int(take(np.int32, 1)[0])
        res.append((rc, take(np.float32, h.vocab_size), take(np.float32, h.n_embd),
                    take(np.float32, h.vocab_size), take(np.float32, h.n_embd)))
    calls, exact = (int(v) for v in take(np.int32, 2))
    n = h.cache_elems()
    caches = [take(np.uint16, n) for _ in range(4)]
    return rcs, res, calls, exact, caches


@needs_exe
@pytest.mark.parametrize("cfg", [CFG, QWEN], ids=["llama", "qwen"])
def test_forward_hooks_with_reference_model(tmp_path, oracle_mod, cfg):
    O = oracle_mod
    h = S.SynthModel(**cfg, seed=41)
    rng = np.random.default_rng(42)
    p1 = rng.integers(0, h.vocab_size, 6).tolist()
    steps = [(1, 0, p1), (0, 6, [11]), (0, 7, [h.vocab_size - 1])]
    rcs, res, calls, exact, (kg, vg, kc, vc) = run_forward(tmp_path, h, steps)
    assert rcs == (0, 0)
    for (kind, start, _), (rc, lg, xg, lc, xc) in zip(steps, res):
        assert rc == 0, (kind, start)
        assert max(normwise(lg, lc), normwise(xg, xc)) <= FWD_TOL, (kind, start)
        assert int(np.argmax(lg)) == int(np.argmax(lc))
    assert calls == 7 * h.n_layers and exact == calls
    kv_layer = h.max_seq_len * h.kv_dim
    assert np.array_equal(kg[:kv_layer], kc[:kv_layer])
    assert np.array_equal(vg[:kv_layer], vc[:kv_layer])
    for dev_bits, ref_bits in ((kg, kc), (vg, vc)):
        a, b = O.f16_to_f32(dev_bits[kv_layer:]), O.f16_to_f32(ref_bits[kv_layer:])
        step = np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float16)).astype(np.float32)
        assert np.all(np.abs(a - b) <= step + 2e-5 * np.max(np.abs(b)))
