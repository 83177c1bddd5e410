"""The reference's own specializer-emitted forward pass over this build.

`verum-slice --generate/--benchmark` does not call the bridge itself: it
compiles the model into a C module (src/vbs_engine.c:174-223: graph ->
planner -> vbs_specializer_emit_source -> system C compiler ->
vbs_specializer_load -> verum_init) and runs its verum_forward, whose
forward_token calls the bridge (src/vbs_specializer.c:231-366). These tests
run that chain from the reference sources (oracle/_ref/libvbs_callers*_ref.so)
in a child process (tests/specializer_run.py) and decode greedily through the
emitted module:

* the unpatched specializer over an allow-listed weight mix (Q8_0, Q4_0,
  Q4_1, F16, Q6_K: src/vbs_specializer.c:69-71) -- no reference-side change;
* the specializer with oracle/specializer_q4k.patch over the Q4_K_M mix --
  the reference-side change a Q4_K_M model needs, with the bridge's two Q4_K
  entries of oracle/ref_callers.c;
* the unpatched specializer refusing the Q4_K_M model, as it does today.

CPU: over the reference's own CPU backend the module reproduces the golden
tiny-model decode (tokens and final logits bit for bit) and the bridge
sequence tests/ref_callers.py restates. GPU: over g_vbs_hip_backend every
step's logits equal host/vbs_decode.c's over the same table, bit for bit.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import vbs_gfx950 as V
from oracle_lib import REF_CALLERS_Q4K_SO, REF_CALLERS_SO, REF_SO

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
RUNNER = os.path.join(HERE, "specializer_run.py")
TINY = dict(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
            max_ctx=64)
# weight types the unpatched specializer has dispatch for (src/vbs_specializer.c:69-71)
ALLOWED_MIX = {"q": V.Q8_0, "k": V.Q4_0, "v": V.Q4_1, "o": V.F16, "gate": V.Q4_0,
               "up": V.Q8_0, "down": V.Q6_K, "embd": V.Q8_0, "head": V.Q6_K}

have_jit = pytest.mark.skipif(
    not all(os.path.exists(p) for p in (REF_CALLERS_SO, REF_CALLERS_Q4K_SO, REF_SO)),
    reason="oracle/_ref not built here (make -C oracle ref)")


def tiny_gguf(host, tmp_path, name, mix=None, seed=99):
    model = V.SynthModel(host, **TINY, seed=seed, mix=mix)
    path = str(tmp_path / name)
    V.write_gguf(host, path, model)
    return model, path


def run_module(tmp_path, backend, lib, gguf, start, steps, expect_ok=True):
    """One child run; returns (result npz or None, combined output)."""
    work = tmp_path / f"jit_{backend}_{lib}"
    work.mkdir(exist_ok=True)
    out = str(work / "out.npz")
    cmd = [sys.executable, "-u", RUNNER, "--backend", backend, "--lib", lib, "--gguf", gguf,
           "--workdir", str(work), "--start", str(start), "--steps", str(steps), "--out", out]
    print("child:", " ".join(cmd), flush=True)
    p = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    text = p.stdout + p.stderr
    print(text, flush=True)
    if not expect_ok:
        assert p.returncode != 0, "the specializer was expected to refuse"
        return None, text
    assert p.returncode == 0, text
    r = np.load(out)
    src = str(r["module"])[:-3] + ".c"
    with open(src) as f:
        emitted = f.read()
    return dict(tokens=[int(t) for t in r["tokens"]], logits=r["logits"],
                n_plans=int(r["n_plans"]), source=emitted), text


def reference_cpu_backend():
    import ctypes as C
    be = V.Backend(C.CDLL(REF_SO), "g_vbs_cpu_backend")
    assert be.init()
    return be


@have_jit
def test_module_q4k_patch_over_reference_cpu_backend_matches_golden(host, tmp_path):
    """The Q4_K-patched specializer's module for the tiny Q4_K_M model, over
    the reference CPU backend: the golden greedy tokens and final logits
    (tests/golden/tiny_model.json, written by the reference's C) bit for bit."""
    meta = json.load(open(os.path.join(GOLD, "tiny_model.json")))
    assert meta["config"] == TINY and meta["seed"] == 99
    _, path = tiny_gguf(host, tmp_path, "tiny.gguf")
    r, _ = run_module(tmp_path, "cpu", "q4k", path, meta["start_token"], len(meta["tokens"]))
    assert "vbs_gpu_dispatch_vram_q4_k(" in r["source"]
    # 2 layers x 9 tensors + token_embd + output_norm + output
    assert r["n_plans"] == 2 * 9 + 3
    assert r["tokens"] == meta["tokens"]
    assert np.array_equal(r["logits"][-1].view(np.uint32),
                          np.array(meta["last_logits_f32_bits"], np.uint32))


@have_jit
def test_unpatched_specializer_refuses_q4k(host, tmp_path):
    """Without the patch the specializer refuses a Q4_K_M model before any
    bridge call (src/vbs_specializer.c:140-145)."""
    _, path = tiny_gguf(host, tmp_path, "tiny.gguf")
    _, text = run_module(tmp_path, "cpu", "plain", path, 1, 2, expect_ok=False)
    assert "no GPU dispatch exists for weight type q4_k" in text


@have_jit
def test_module_allowlisted_mix_over_reference_cpu_backend(host, tmp_path):
    """The unpatched specializer's module for a Q8_0/Q4_0/Q4_1/F16/Q6_K model,
    over the reference CPU backend: every step's logits bit-equal to the
    bridge sequence tests/ref_callers.py restates, over the same backend."""
    import ref_callers as rc
    _, path = tiny_gguf(host, tmp_path, "mix.gguf", mix=ALLOWED_MIX, seed=21)
    r, _ = run_module(tmp_path, "cpu", "plain", path, 7, 12)
    for f in ("vram_q8_0", "vram_q4_0", "vram_q4_1", "vram_f16", "vram_q6_k", "embed_q8_0"):
        assert f"vbs_gpu_dispatch_{f}(g_blocks" in r["source"], f
    L = rc.load_callers("cpu_mix")
    eng = rc.RefEngine(L, reference_cpu_backend(), path)
    try:
        eng.zero_kv()
        tok = 7
        for i, lg in enumerate(r["logits"]):
            want = eng.step(tok, i)
            assert np.array_equal(lg.view(np.uint32), want.view(np.uint32)), i
            tok = int(np.argmax(want))
    finally:
        eng.close()


def _decode_driver_equal(host, backend, model, r, start):
    d = V.Decoder(host, backend, model)
    try:
        tok = start
        for i, lg in enumerate(r["logits"]):
            want = d.step(tok, i)
            assert np.array_equal(lg.view(np.uint32), want.view(np.uint32)), i
            tok = int(np.argmax(want))
    finally:
        d.close()


@pytest.mark.gpu
@have_jit
def test_gpu_module_q4k_patch_equals_decode_driver(host, backend, tmp_path):
    """The Q4_K-patched specializer's module over g_vbs_hip_backend: 24
    greedy steps, each step's logits bit-equal to host/vbs_decode.c's, and
    the tokens the reference CPU backend's golden ones."""
    meta = json.load(open(os.path.join(GOLD, "tiny_model.json")))
    model, path = tiny_gguf(host, tmp_path, "tiny.gguf")
    r, _ = run_module(tmp_path, "gfx950", "q4k", path, meta["start_token"], len(meta["tokens"]))
    assert r["tokens"] == meta["tokens"]
    _decode_driver_equal(host, backend, model, r, meta["start_token"])


@pytest.mark.gpu
@have_jit
def test_gpu_module_allowlisted_mix_equals_decode_driver(host, backend, tmp_path):
    """The unpatched specializer's module (no reference-side change at all)
    over g_vbs_hip_backend: 16 greedy steps of the Q8_0/Q4_0/Q4_1/F16/Q6_K
    model, each step's logits bit-equal to host/vbs_decode.c's."""
    model, path = tiny_gguf(host, tmp_path, "mix.gguf", mix=ALLOWED_MIX, seed=21)
    r, _ = run_module(tmp_path, "gfx950", "plain", path, 7, 16)
    _decode_driver_equal(host, backend, model, r, 7)
