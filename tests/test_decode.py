"""Decode-step parity: the bridge-order driver (host/vbs_decode.c) over a
backend table against the oracle's forward pass (oracle/vbs_oracle.c,
vbs_oracle_forward_token, following src/vbs_specializer.c:231-349).

* CPU: the driver over the reference's own CPU backend (oracle/_ref, compiled
  from src/vbs_backend_cpu.c) must give bit-identical logits to the oracle --
  this pins the oracle's forward pass and the driver's sequencing on the real
  reference code.
* GPU: the driver over g_vbs_hip_backend must produce the oracle's greedy
  token sequence, with logits within 1e-4 relative L2 per step.
"""
import numpy as np
import pytest

import vbs_gfx950 as V
from oracle_lib import REF_SO, Oracle

TINY = dict(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
            max_ctx=64)


def full_cache(model, kc_pref, vc_pref, n_pos):
    """[L][n_pos][kvd] prefill -> [L][max_ctx][kvd] oracle cache."""
    c = model.cfg
    kvd = c["n_kv_heads"] * c["head_dim"]
    shape = (c["n_layers"], c["max_ctx"], kvd)
    kc, vc = np.zeros(shape, np.uint16), np.zeros(shape, np.uint16)
    if n_pos:
        kc[:, :n_pos] = kc_pref.reshape(c["n_layers"], n_pos, kvd)
        vc[:, :n_pos] = vc_pref.reshape(c["n_layers"], n_pos, kvd)
    return kc, vc


def oracle_greedy(oracle, model, kc, vc, token, pos, n, threads=16):
    om = oracle.model(model, kc, vc)
    toks, logits = [], []
    for i in range(n):
        lg = oracle.forward(om, token, pos + i, model.cfg["vocab"], threads)
        token = int(np.argmax(lg))  # numpy argmax returns the first maximum
        toks.append(token)
        logits.append(lg)
    return np.array(toks, np.uint32), logits


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b.astype(np.float64)))


@pytest.fixture(scope="module")
def tiny(host):
    return V.SynthModel(host, **TINY, seed=99)


def test_driver_on_reference_cpu_backend_matches_oracle(host, tiny):
    import ctypes
    import os
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref not built (reference sources absent)")
    ref = V.Backend(ctypes.CDLL(REF_SO), "g_vbs_cpu_backend")
    assert ref.init()
    oracle = Oracle()
    kc_p, vc_p = tiny.kv_prefill(host, 5)
    d = V.Decoder(host, ref, tiny)
    d.load_kv(kc_p, vc_p, 5)
    kc, vc = full_cache(tiny, kc_p, vc_p, 5)
    om = oracle.model(tiny, kc, vc)
    tok = 3
    for pos in range(5, 13):
        got = d.step(tok, pos)
        want = oracle.forward(om, tok, pos, tiny.cfg["vocab"], threads=4)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"pos {pos}"
        tok = int(np.argmax(want))
    # the driver's KV stores equal the oracle's, bit for bit
    gk, gv = d.read_kv(13)
    c = tiny.cfg
    kvd = c["n_kv_heads"] * c["head_dim"]
    assert np.array_equal(gk.reshape(c["n_layers"], 13, kvd), kc[:, :13])
    assert np.array_equal(gv.reshape(c["n_layers"], 13, kvd), vc[:, :13])
    d.close()


@pytest.mark.gpu
def test_gpu_tiny_model_greedy(host, backend, tiny):
    oracle = Oracle()
    d = V.Decoder(host, backend, tiny)
    kc, vc = full_cache(tiny, None, None, 0)
    want_toks, want_logits = oracle_greedy(oracle, tiny, kc, vc, 1, 0, 24)
    tok = 1
    for i in range(24):
        lg = d.step(tok, i)
        assert rel_l2(lg, want_logits[i]) <= 1e-4, f"step {i}"
        tok = int(np.argmax(lg))
        assert tok == want_toks[i], f"step {i}"
    d.close()


@pytest.mark.gpu
@pytest.mark.parametrize("n_layers,n_tok", [(4, 12), (32, 3)], ids=["7b_4layers", "7b_full"])
def test_gpu_7b_shape_greedy(host, backend, n_layers, n_tok):
    """7B geometry (config 4), KV prefilled N(0,1) to 2048, greedy from 2048."""
    ctx = 2048
    model = V.SynthModel(host, n_layers=n_layers, hidden=4096, ffn=11008, n_heads=32,
                         n_kv_heads=8, head_dim=128, vocab=32000, max_ctx=ctx + n_tok + 1,
                         seed=7)
    kc_p, vc_p = model.kv_prefill(host, ctx)
    d = V.Decoder(host, backend, model)
    d.load_kv(kc_p, vc_p, ctx)
    toks, margins = d.greedy(1, ctx, n_tok)
    d.close()
    kc, vc = full_cache(model, kc_p, vc_p, ctx)
    want, _ = oracle_greedy(Oracle(), model, kc, vc, 1, ctx, n_tok)
    assert np.array_equal(toks, want), (toks, want, margins)
