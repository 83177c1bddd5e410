"""The drop-in driven by the reference's own callers of the backend table:
its specializer bridge (src/vbs_specializer_bridge.c:83-206, with the two
Q4_K entries of oracle/ref_callers.c), its memory fabric
(src/vbs_fabric.c:63-154), its slice executor (src/vbs_slice_executor.c:42-107,
convention B) and its GGUF loader, compiled from the reference sources into
oracle/_ref/libvbs_callers_ref.so (tests/ref_callers.py drives them).

* CPU: the same callers over the reference's own CPU backend reproduce the
  golden tiny-model decode bit for bit -- this pins the emitted call sequence
  the GPU tests replay, and the executor's tiling against the oracle.
* GPU: the bridge sequence over g_vbs_hip_backend gives logits equal, bit for
  bit, to this build's decode driver (host/vbs_decode.c) at every step, with
  the golden tokens; a Q4_K-embedding model whose blocks the fabric faults in
  on first use does the same; the slice executor's convention-B tiles
  (row and column splits, accumulation) match the oracle's matvec.
"""
import json
import os

import numpy as np
import pytest

import vbs_gfx950 as V
from oracle_lib import REF_CALLERS_SO, REF_SO, Oracle

have_callers = pytest.mark.skipif(not (os.path.exists(REF_CALLERS_SO) and os.path.exists(REF_SO)),
                                  reason="oracle/_ref not built here (make -C oracle ref)")
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TINY = dict(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
            max_ctx=64)
ALL_Q4K = {r: V.Q4_K for r in ("q", "k", "v", "o", "gate", "up", "down", "embd", "head")}


def rc():
    import ref_callers
    return ref_callers


def tiny_gguf(host, tmp_path, name, mix=None, seed=99):
    model = V.SynthModel(host, **TINY, seed=seed, mix=mix)
    path = str(tmp_path / name)
    V.write_gguf(host, path, model)
    return model, path


def reference_cpu_backend():
    import ctypes as C
    be = V.Backend(C.CDLL(REF_SO), "g_vbs_cpu_backend")
    assert be.init()
    return be


def greedy(engine, n, tok=1, pos=0):
    toks, logits = [], []
    for i in range(n):
        lg = engine.step(tok, pos + i)
        tok = int(np.argmax(lg))
        toks.append(tok)
        logits.append(lg)
    return toks, logits


@have_callers
def test_bridge_sequence_over_reference_cpu_backend_matches_golden(host, tmp_path):
    """F5 again, now through the reference's bridge, fabric and GGUF loader:
    the emitted token step over the reference CPU backend gives the golden
    greedy tokens and final logits bit for bit."""
    meta = json.load(open(os.path.join(GOLD, "tiny_model.json")))
    assert meta["config"] == TINY and meta["seed"] == 99
    _, path = tiny_gguf(host, tmp_path, "tiny.gguf")
    L = rc().load_callers("cpu")
    eng = rc().RefEngine(L, reference_cpu_backend(), path)
    try:
        eng.zero_kv()
        toks, logits = greedy(eng, len(meta["tokens"]), meta["start_token"])
    finally:
        eng.close()
    assert toks == meta["tokens"]
    assert np.array_equal(logits[-1].view(np.uint32),
                          np.array(meta["last_logits_f32_bits"], np.uint32))


@have_callers
def test_slice_executor_over_reference_cpu_backend(host, tmp_path):
    """The executor's tiles over the reference CPU backend equal the oracle's
    whole matvec (the tiling itself is exact: each tile accumulates whole
    blocks in the reference's order only within one row's column range)."""
    import ctypes as C
    model, path = tiny_gguf(host, tmp_path, "tiny_se.gguf")
    L = rc().load_callers("cpu_se")
    be = reference_cpu_backend()
    gm = rc().GgufModel(L, path)
    orc = Oracle()
    try:
        se = rc().SliceExecutor(L, be, gm, 4096)
        for name in ("blk.0.ffn_gate.weight", "blk.1.ffn_down.weight", "output.weight"):
            rows, cols, t = gm.shape(name)
            x = V.synth_normal(host, cols, 5, rows)
            bx, by = be.upload(x), be.upload(np.zeros(rows, np.float32))
            ok, err = se.run_linear(name, bx, by)
            assert ok, err
            got = be.download(by, rows, np.float32)
            w = np.ctypeslib.as_array(C.cast(L.vbs_callers_tensor_data(gm.ptr, gm.tensor(name)),
                                             C.POINTER(C.c_uint8)),
                                      (rows * V.row_bytes(t, cols),)).copy()
            want = orc.linear(t, w, x, cols, rows)
            assert float(np.linalg.norm(got - want) / np.linalg.norm(want)) <= 1e-6, name
        se.close()
    finally:
        gm.close()


@pytest.mark.gpu
@have_callers
def test_gpu_bridge_sequence_equals_decode_driver(host, backend, tmp_path):
    """The reference's bridge over g_vbs_hip_backend: 24 greedy steps of the
    tiny Q4_K_M model (vbs_gpu_dispatch_vram_q4_k for Q/K/V/O/gate/up), the
    logits of every step bit-equal to host/vbs_decode.c's over the same
    table, and the tokens the reference CPU backend's golden ones."""
    meta = json.load(open(os.path.join(GOLD, "tiny_model.json")))
    model, path = tiny_gguf(host, tmp_path, "tiny_gpu.gguf")
    L = rc().load_callers("gpu")
    eng = rc().RefEngine(L, backend, path)
    d = V.Decoder(host, backend, model)
    try:
        eng.zero_kv()
        toks, logits = greedy(eng, len(meta["tokens"]), meta["start_token"])
        tok = meta["start_token"]
        for i, lg in enumerate(logits):
            want = d.step(tok, i)
            assert np.array_equal(lg.view(np.uint32), want.view(np.uint32)), i
            tok = int(np.argmax(want))
    finally:
        d.close()
        eng.close()
    assert toks == meta["tokens"]


@pytest.mark.gpu
@have_callers
def test_gpu_bridge_q4k_embedding_with_fabric_fault_in(host, backend, tmp_path):
    """Every weight Q4_K, embedding and head included (the bridge's added
    vbs_gpu_dispatch_embed_q4_k), registered on the host tier so that
    vbs_bridge_get_block_dptr faults each block into device memory through
    the table (vbs_fabric_fault_in_to_device): 12 steps bit-equal to the
    decode driver's."""
    model, path = tiny_gguf(host, tmp_path, "tiny_q4k.gguf", mix=ALL_Q4K, seed=5)
    L = rc().load_callers("gpu_q4k")
    eng = rc().RefEngine(L, backend, path, tier=rc().TIER_HOST_PAGED)
    d = V.Decoder(host, backend, model)
    try:
        assert set(eng.tiers_at_registration) == {5}  # VBS_TIER_FILE_SOURCE
        assert set(eng.tiers_after_init) == {0}  # VBS_TIER_VRAM
        eng.zero_kv()
        tok = 3
        for pos in range(12):
            got, want = eng.step(tok, pos), d.step(tok, pos)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), pos
            tok = int(np.argmax(want))
    finally:
        d.close()
        eng.close()


@pytest.mark.gpu
@have_callers
@pytest.mark.parametrize("geometry,window,names", [
    ("tiny", 4096, ["blk.0.ffn_gate.weight", "blk.1.ffn_down.weight", "output.weight"]),
    ("7b_1layer", 8 << 20, ["blk.0.ffn_down.weight", "blk.0.ffn_gate.weight", "output.weight"]),
], ids=["tiny_4KiB", "7b_8MiB"])
def test_gpu_slice_executor_convention_b(host, backend, tmp_path, geometry, window, names):
    """src/vbs_slice_executor.c over g_vbs_hip_backend: each tensor streamed
    through two `window`-byte staging windows as convention-B tiles (several
    row tiles, and column tiles accumulated for the wide ones), against the
    oracle's matvec over the whole tensor within 1e-5 relative L2."""
    import ctypes as C
    if geometry == "tiny":
        _, path = tiny_gguf(host, tmp_path, "se.gguf")
    else:
        path = str(tmp_path / "se7b.gguf")
        V.write_gguf_geometry(host, path, n_layers=1, hidden=4096, ffn=11008, n_heads=32,
                              n_kv_heads=8, head_dim=128, vocab=32000, context_length=64, seed=7)
    L = rc().load_callers(f"gpu_se_{geometry}")
    gm = rc().GgufModel(L, path)
    orc = Oracle()
    try:
        se = rc().SliceExecutor(L, backend, gm, window)
        for name in names:
            rows, cols, t = gm.shape(name)
            x = V.synth_normal(host, cols, 9, rows)
            bx, by = backend.upload(x), backend.upload(np.full(rows, np.nan, np.float32))
            ok, err = se.run_linear(name, bx, by)
            assert ok, (name, err, backend.last_error())
            got = backend.download(by, rows, np.float32)
            w = np.ctypeslib.as_array(C.cast(L.vbs_callers_tensor_data(gm.ptr, gm.tensor(name)),
                                             C.POINTER(C.c_uint8)),
                                      (rows * V.row_bytes(t, cols),)).copy()
            want = orc.linear(t, w, x, cols, rows, threads=16)
            err = float(np.linalg.norm(got - want) / np.linalg.norm(want))
            print(f"{name} {rows}x{cols} {V.TYPE_NAMES[t]}: rel L2 {err:.2e}")
            assert err <= 1e-5, (name, err)
            backend.ops.free_buffer(bx)
            backend.ops.free_buffer(by)
        se.close()
    finally:
        gm.close()


def engine_kv_capacity(free_vram, total_vram, geo, n_layers, ctx, mix=None):
    """vbs_engine_create's KV budget (src/vbs_engine.c:94-140) for a Q4_K_M
    llama model of this geometry: positions that fit in the free VRAM after
    the model and the runtime buffers, capped at the context length."""
    mix = dict(V.Q4_K_M_MIX if mix is None else mix)
    H, F, nq, nkv, hd, vocab = (geo[k] for k in ("hidden", "ffn", "n_heads", "n_kv_heads",
                                                 "head_dim", "vocab"))
    qd, kvd = nq * hd, nkv * hd
    shapes = {"q": (qd, H), "k": (kvd, H), "v": (kvd, H), "o": (H, qd),
              "gate": (F, H), "up": (F, H), "down": (H, F)}
    model = (n_layers * sum(r * V.row_bytes(mix[n], c) for n, (r, c) in shapes.items())
             + n_layers * 2 * H * 4 + H * 4
             + vocab * V.row_bytes(mix["embd"], H) + vocab * V.row_bytes(mix["head"], H))
    scratch = 4 * (qd + kvd + kvd + qd + F + F + F + H + qd + kvd)
    runtime = 2 * H * 4 + vocab * 4 + scratch
    kv_pos = n_layers * nkv * hd * 2
    base = free_vram or total_vram
    fit = (base - model - runtime) // (2 * kv_pos) if base > model + runtime else 0
    return min(fit, ctx), kv_pos, model


@pytest.mark.gpu
@have_callers
def test_gpu_device_info_feeds_profiler_fabric_and_kv_budget(host, backend, tmp_path):
    """The reference's selection, profiler and engine read the shim's device
    struct: VBS_BACKEND=hip takes the table when its init succeeds, and logs
    device 0's name (src/vbs_backend_select.c:42-85; that file links the
    Vulkan and CUDA backends, which the image cannot build, so the test
    checks the conditions it reads: init, a device, a name); the profiler's HIP
    branch turns max_working_set_bytes / max_buffer_bytes into the system
    profile (src/vbs_profiler.c:194-210, restated in oracle/ref_callers.c:
    vbs_profiler.c itself does not link here); the engine sizes its KV cache
    from that profile (src/vbs_engine.c:94-140). With this device's figures
    the 7B model gets its whole 2176-position context and the 70B model its
    8320 (config 5 at ctx 8192 plus 128 tokens), the planner's VRAM budget
    (src/vbs_planner.c:57) holds the whole 70B model, and the 70B caches of
    that capacity allocate through the table. The reference fabric over the
    same profile places the tiny model in device memory and its bridge
    sequence equals the decode driver's."""
    import ctypes as C
    ops = backend.ops
    assert ops.init() and ops.get_device_count() >= 1
    devp = ops.get_device(0)
    dev = devp.contents
    assert dev.name and dev.type == 2  # VBS_BACKEND_HIP
    L = rc().load_callers("gpu_profile")
    prof = L.vbs_callers_profile_hip(C.cast(devp, C.c_void_p))
    import ref_callers as rcm
    total, free = dev.max_working_set_bytes, dev.max_working_set_bytes * 85 // 100
    print(f"device {dev.name.decode()}: max_working_set {total / 2**30:.1f} GiB, "
          f"max_buffer {dev.max_buffer_bytes / 2**30:.1f} GiB")
    assert total >= 256 << 30 and dev.max_buffer_bytes >= 64 << 30
    from test_decode import GEO_70B, GEO_7B
    cap7, _, m7 = engine_kv_capacity(free, total, GEO_7B, 32, 2176)
    cap70, kvpos70, m70 = engine_kv_capacity(free, total, GEO_70B, 80, 8320)
    print(f"KV capacity: 7B {cap7} (model {m7 / 1e9:.2f} GB), 70B {cap70} "
          f"(model {m70 / 1e9:.2f} GB)")
    assert cap7 == 2176 and cap70 == 8320
    assert free * 90 // 100 >= m70  # every 70B tensor planned IN_VRAM
    kv = [backend.alloc(kvpos70 * cap70) for _ in range(2)]
    for b in kv:
        ops.free_buffer(b)
    model, path = tiny_gguf(host, tmp_path, "tiny_prof.gguf")
    eng = rcm.RefEngine(L, backend, path, profile="hip")
    d = V.Decoder(host, backend, model)
    try:
        assert set(eng.tiers_after_init) == {0}  # VBS_TIER_VRAM
        eng.zero_kv()
        tok = 1
        for pos in range(6):
            got, want = eng.step(tok, pos), d.step(tok, pos)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), pos
            tok = int(np.argmax(want))
    finally:
        d.close()
        eng.close()
