"""The synthetic GGUF models through the reference's own model-level CPU
inference (src/vbs_cpu.c, compiled into oracle/_ref with the sources its
Makefile links it with).

* vbs_cpu_open accepts the file: its strict llama-metadata, tensor-type and
  shape checks (src/vbs_cpu.c:396-476) pin the GGUF writer further.
* Its logits agree with the decode-step oracle (vbs_oracle_forward_token) to
  within the CPU model's own quantisation: it runs Q8_0 shadows of the
  K-quant weights with Q8 activations and an f32 KV cache (src/vbs_cpu.c:
  166-219, 312-346, 572-640) where the GPU path keeps the weights, f32
  activations and an f16 cache. The two share nothing but the model file, so
  agreement also pins the oracle's tensor roles, RoPE pairing, GQA head map
  and norm placement against a second, independent reading of the same
  architecture.
"""
import os

import numpy as np
import pytest

import vbs_gfx950 as V
from oracle_lib import REF_CPU_SO, Oracle, cpu_model_logits, reference_cpu_model

pytestmark = pytest.mark.skipif(not os.path.exists(REF_CPU_SO),
                                reason="oracle/_ref CPU model not built")

TINY = dict(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
            max_ctx=64)
TOKENS = [1, 17, 300, 5, 42]


def oracle_logits(host, model, tokens):
    orc = Oracle()
    c = model.cfg
    n = c["n_layers"] * c["max_ctx"] * c["n_kv_heads"] * c["head_dim"]
    kc, vc = np.zeros(n, np.uint16), np.zeros(n, np.uint16)
    om = orc.model(model, kc, vc)
    return [orc.forward(om, t, p, c["vocab"]) for p, t in enumerate(tokens)]


@pytest.mark.parametrize("mix", [None, {"q": V.Q8_0, "k": V.Q4_0, "v": V.Q4_1, "o": V.Q8_0,
                                        "gate": V.Q4_0, "up": V.Q8_0, "down": V.Q4_1,
                                        "embd": V.Q8_0, "head": V.Q8_0}],
                         ids=["q4_k_m", "q8_q4_mix"])
def test_reference_cpu_model_runs_the_synthetic_file(host, tmp_path, mix):
    model = V.SynthModel(host, seed=31, mix=mix, **TINY)
    path = tmp_path / "tiny.gguf"
    V.write_gguf(host, str(path), model, context_length=2176)
    got = cpu_model_logits(reference_cpu_model(), path, TOKENS)
    want = oracle_logits(host, model, TOKENS)
    for step, (a, b) in enumerate(zip(got, want)):
        assert a.shape == (TINY["vocab"],) and np.all(np.isfinite(a))
        rel = np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b.astype(np.float64))
        cos = float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b)))
        assert cos > 0.995 and rel < 0.08, (step, cos, rel)


def test_reference_cpu_model_capacity_and_vocab(host, tmp_path):
    import ctypes as C
    model = V.SynthModel(host, seed=32, **TINY)
    path = tmp_path / "tiny.gguf"
    V.write_gguf(host, str(path), model, context_length=2176)
    lib = reference_cpu_model()
    err = C.create_string_buffer(512)
    m = lib.vbs_cpu_open(str(path).encode(), 16, err, 512)
    assert m, err.value
    try:
        assert lib.vbs_cpu_vocab_size(m) == TINY["vocab"]
        assert lib.vbs_cpu_context_capacity(m) == 16
    finally:
        lib.vbs_cpu_close(m)
