#!/usr/bin/env python3
"""Write the golden fixtures of tests/golden/ by running the reference's own
CPU code: oracle/_ref/libvbs_ref.so, compiled by `make -C oracle ref` from
src/vbs_backend_cpu.c, src/vbs_dequant.c and src/vbs_gguf.c where they lie
under the mounted reference tree. Only data is written (inputs and the
reference's outputs); no reference source is copied.

  dequant_blocks.npz   F1: random + edge blocks per hot-path type ->
                       vbs_dequant_block outputs (f32 bit patterns)
  half.json            F2: digest of vbs_f16_to_f32 over all 65536 halves,
                       digest of vbs_f32_to_f16 over all 2^32 floats, and
                       explicit edge conversions
  linear.npz           F3: vbs_host_linear_tile (through the reference CPU
                       backend's dispatch_linear_tile) at 8x4096, 8x11008
                       and an offsets + accumulate tile pair
  prims.npz            F4: rms_norm, rope, kv store, silu*up, add and GQA
                       attention through the reference dispatch_primitive
  tiny_model.json      F5: greedy tokens and last logits of the tiny
                       Q4_K_M-mix model, decoded in the bridge's order
                       through the reference CPU backend

Run from the repository root after `make -C oracle` and a build of the
package (the synthetic generator and the decode driver come from
libvbs_backend_gfx950.so):  python tests/golden/gen_golden.py
"""
import ctypes as C
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "verum-bespoke-singularity_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import vbs_gfx950 as V  # noqa: E402
from oracle_lib import REF_SO, F16FN, Oracle  # noqa: E402

SEED = 77
TYPES = [V.Q4_0, V.Q4_1, V.Q8_0, V.Q4_K, V.Q6_K]


def ref_lib():
    if not os.path.exists(REF_SO):
        sys.exit(f"{REF_SO} missing: run `make -C oracle ref` with the reference mounted")
    lib = C.CDLL(REF_SO)
    lib.vbs_f16_to_f32.restype, lib.vbs_f16_to_f32.argtypes = C.c_float, [C.c_uint16]
    lib.vbs_f32_to_f16.restype, lib.vbs_f32_to_f16.argtypes = C.c_uint16, [C.c_float]
    lib.vbs_dequant_block.restype = C.c_int
    lib.vbs_dequant_block.argtypes = [C.c_int, C.c_void_p, C.c_void_p]
    return lib


def edge_blocks(t, nbytes, rng):
    """Hand-made blocks: all 0x00, all 0xFF, alternating, max scales, special d."""
    out = [np.zeros(nbytes, np.uint8), np.full(nbytes, 0xFF, np.uint8),
           np.tile(np.array([0x55, 0xAA], np.uint8), nbytes // 2)]
    specials = [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x3C00, 0xBC00, 0x8001]  # subnormal, max, 1, -1
    dpos = {V.Q4_0: [0], V.Q4_1: [0, 2], V.Q8_0: [0], V.Q4_K: [0, 2], V.Q6_K: [208]}[t]
    for sv in specials:
        b = rng.integers(0, 256, nbytes, dtype=np.uint8)
        for p in dpos:
            b[p:p + 2] = np.frombuffer(np.uint16(sv).tobytes(), np.uint8)
        out.append(b)
    return out


def gen_dequant(lib, host):
    rng = np.random.default_rng(SEED)
    arrays = {}
    for t in TYPES:
        e, nb = V.GEOMETRY[t]
        synth = V.synth_matrix(host, t, 1, e * 48, SEED, 900 + t).reshape(48, nb)
        rnd = rng.integers(0, 256, (16, nb), dtype=np.uint8)  # arbitrary bytes (finite d not required)
        blocks = np.concatenate([synth, rnd, np.stack(edge_blocks(t, nb, rng))])
        outs = np.empty((blocks.shape[0], e), np.float32)
        for i, b in enumerate(blocks):
            b = np.ascontiguousarray(b)
            assert lib.vbs_dequant_block(t, b.ctypes.data, outs[i].ctypes.data) == e
        arrays[f"t{t}_in"] = blocks
        arrays[f"t{t}_out"] = outs.view(np.uint32)
    np.savez_compressed(os.path.join(HERE, "dequant_blocks.npz"), **arrays)


def gen_half(lib):
    # all 65536 halves as one F16 embedding row through the reference CPU
    # backend, so the converted floats are stored to memory untouched (a float
    # return value through ctypes would quiet signalling-NaN payloads)
    be = ref_backend()
    table = np.arange(65536, dtype=np.uint16)
    f = np.zeros(65536, np.float32)
    keep = []
    pipe = be.ops.compile_embed_pipeline(be.device(), V.F16, None, 0)
    assert be.dispatch(pipe, [V.VbsArg(0, table.ctypes.data, 0), be.u32_arg(keep, 0),
                              V.VbsArg(0, f.ctypes.data, 0), be.u32_arg(keep, 65536)])
    d16 = hashlib.sha256(f.view(np.uint32).astype("<u4").tobytes()).hexdigest()
    orc = Oracle()
    ref_fn = F16FN(("vbs_f32_to_f16", lib))
    d32 = orc._digest_f32_to_f16(ref_fn, os.cpu_count() or 4)
    edges = [0.0, -0.0, 1.0, -2.5, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.103515625e-05,
             6.1e-05, 3.0517578125e-05, 2.98e-08, 2.9802322387695312e-08, 2.99e-08, 5.96e-08,
             1e-10, float("inf"), float("-inf"), float("nan"), 0.1, 1.0 / 3.0, 2049.0, 2051.0,
             -1.00048828125, 1.00048828125, 1.0004882812500002]
    ev = [[float(np.float32(v)), int(np.float32(v).view(np.uint32)),
           int(lib.vbs_f32_to_f16(float(np.float32(v))))] for v in edges]
    with open(os.path.join(HERE, "half.json"), "w") as fh:
        json.dump({"f16_to_f32_sha256": d16, "f32_to_f16_digest": f"{d32:016x}",
                   "digest_note": "FNV-1a 64 over 256 ranges of 2^24 floats, see "
                                  "vbs_oracle_digest_f32_to_f16",
                   "f32_to_f16_edges": ev}, fh, indent=1)


def ref_backend():
    be = V.Backend(C.CDLL(REF_SO), "g_vbs_cpu_backend")
    assert be.init()
    return be


def hbuf(be, a):
    a = np.ascontiguousarray(a)
    return V.VbsBuffer(a.ctypes.data, a.ctypes.data, a.nbytes, be.device()), a


def gen_linear(host):
    be = ref_backend()
    arrays = {}
    cases = [(V.Q4_0, 8, 4096), (V.Q4_1, 8, 4096), (V.Q8_0, 8, 4096), (V.Q4_K, 8, 4096),
             (V.Q4_K, 8, 11008), (V.Q6_K, 8, 11008), (V.Q6_K, 8, 4096), (V.F16, 8, 512),
             (V.F32, 8, 300)]
    for i, (t, rows, cols) in enumerate(cases):
        w = V.synth_matrix(host, t, rows, cols, SEED, 1000 + i)
        x = V.synth_normal(host, cols, SEED, 2000 + i)
        y = np.zeros(rows, np.float32)
        pipe = be.ops.compile_linear_pipeline(be.device(), t, None, 0)
        bw, _ = hbuf(be, w)
        bx, _ = hbuf(be, x)
        by, _ = hbuf(be, y)
        assert be.ops.dispatch_linear_tile(be.device(), pipe, C.byref(bw), None, 0, C.byref(bx),
                                           C.byref(by), cols, rows, 0, 0, False)
        arrays[f"c{i}_meta"] = np.array([t, rows, cols], np.int64)
        arrays[f"c{i}_w"], arrays[f"c{i}_x"], arrays[f"c{i}_y"] = w, x, y
    # convention B with offsets and accumulate: two Q4_K column tiles of an 8 x 4096
    # tensor into y[4:12] starting from y = 3.0, x window at 256
    t, rows, half = V.Q4_K, 8, 2048
    w = V.synth_matrix(host, t, rows, 2 * half, SEED, 1100)
    x = V.synth_normal(host, 2 * half + 256, SEED, 2100)
    y = np.full(rows + 4, 3.0, np.float32)
    rb = V.row_bytes(t, half)
    pipe = be.ops.compile_linear_pipeline(be.device(), t, None, 0)
    bx, _ = hbuf(be, x)
    by, _ = hbuf(be, y)
    for k in range(2):
        tile = np.ascontiguousarray(w[:, k * rb:(k + 1) * rb])
        stage = be.alloc(tile.nbytes, True)
        priv = be.alloc(tile.nbytes)
        C.memmove(stage.contents.host_ptr, tile.ctypes.data, tile.nbytes)
        assert be.ops.dispatch_linear_tile(be.device(), pipe, priv, stage, tile.nbytes,
                                           C.byref(bx), C.byref(by), half, rows, 256 + k * half,
                                           4, k == 1)
        be.ops.free_buffer(stage)
        be.ops.free_buffer(priv)
    arrays["acc_w"], arrays["acc_x"], arrays["acc_y"] = w, x, y
    np.savez_compressed(os.path.join(HERE, "linear.npz"), **arrays)


def gen_prims(host):
    be = ref_backend()
    dev = be.device()
    arrays = {}

    def prim(kind, args):
        pipe = be.ops.compile_primitive_pipeline(dev, kind, None, 0)
        assert be.dispatch(pipe, args)

    keep = []
    # rms_norm dim 4096 and 384
    for n in (4096, 384):
        x = V.synth_normal(host, n, SEED, 3000 + n) * 2.0
        w = V.synth_normal(host, n, SEED, 3100 + n, 0.1, 1.0)
        out = np.zeros(n, np.float32)
        prim(V.OP_NORMALIZE, [V.VbsArg(0, x.ctypes.data, 0), V.VbsArg(0, w.ctypes.data, 0),
                              V.VbsArg(0, out.ctypes.data, 0), be.u32_arg(keep, n),
                              be.f32_arg(keep, 1e-5)])
        arrays[f"rms{n}_x"], arrays[f"rms{n}_w"], arrays[f"rms{n}_out"] = x, w, out
    # rope: 32 heads x 128, theta 1e4 and 5e5, several positions
    x0 = V.synth_normal(host, 32 * 128, SEED, 3200)
    for theta in (10000.0, 500000.0):
        for pos in (0, 7, 2047, 2175, 8191):
            x = x0.copy()
            prim(V.OP_ROTARY, [V.VbsArg(0, x.ctypes.data, 0), be.u32_arg(keep, pos),
                               be.u32_arg(keep, 128), be.u32_arg(keep, 32),
                               be.f32_arg(keep, theta)])
            arrays[f"rope_{int(theta)}_{pos}"] = x
    arrays["rope_x"] = x0
    # kv store with edge values (subnormal, ties, overflow, nan)
    kvd, max_ctx, layers = 1024, 24, 3
    k = V.synth_normal(host, kvd, SEED, 3300) * 1e-5
    v = V.synth_normal(host, kvd, SEED, 3301) * 3e4
    k[:10] = [6.1e-5, -3.05e-5, 2 ** -25, 2 ** -26, 65520.0, -1e9, np.nan, 0.0, 5.9604645e-08,
              8.940697e-08]
    kc = np.zeros(layers * max_ctx * kvd, np.uint16)
    vc = np.zeros_like(kc)
    prim(V.OP_CACHE, [V.VbsArg(0, k.ctypes.data, 0), V.VbsArg(0, v.ctypes.data, 0),
                      V.VbsArg(0, kc.ctypes.data, 0), V.VbsArg(0, vc.ctypes.data, 0),
                      be.u32_arg(keep, 17), be.u32_arg(keep, 2), be.u32_arg(keep, max_ctx),
                      be.u32_arg(keep, kvd)])
    base = (2 * max_ctx + 17) * kvd
    arrays["kv_k"], arrays["kv_v"] = k, v
    arrays["kv_kc"], arrays["kv_vc"] = kc[base:base + kvd], vc[base:base + kvd]
    # silu * up and add
    n = 11008
    g = V.synth_normal(host, n, SEED, 3400) * 3.0
    u = V.synth_normal(host, n, SEED, 3401)
    o = np.zeros(n, np.float32)
    prim(V.OP_ACTIVATION, [V.VbsArg(0, g.ctypes.data, 0), V.VbsArg(0, u.ctypes.data, 0),
                           V.VbsArg(0, o.ctypes.data, 0), be.u32_arg(keep, n)])
    arrays["silu_g"], arrays["silu_u"], arrays["silu_out"] = g, u, o
    a = V.synth_normal(host, 4096, SEED, 3500)
    b = V.synth_normal(host, 4096, SEED, 3501)
    o2 = np.zeros(4096, np.float32)
    prim(V.OP_ELEMENTWISE, [V.VbsArg(0, a.ctypes.data, 0), V.VbsArg(0, b.ctypes.data, 0),
                            V.VbsArg(0, o2.ctypes.data, 0), be.u32_arg(keep, 4096)])
    arrays["add_a"], arrays["add_b"], arrays["add_out"] = a, b, o2
    # attention: nq 8, nkv 2, hd 64, layer 1 of 2, max_ctx 320, seq 1, 64, 300
    nq, nkv, hd, mc = 8, 2, 64, 320
    kcache = V.synth_normal_f16(host, 2 * mc * nkv * hd, SEED, 3600)
    vcache = V.synth_normal_f16(host, 2 * mc * nkv * hd, SEED, 3601)
    q = V.synth_normal(host, nq * hd, SEED, 3602)
    arrays["att_kc"], arrays["att_vc"], arrays["att_q"] = kcache, vcache, q
    for seq in (1, 64, 300):
        out = np.zeros(nq * hd, np.float32)
        prim(V.OP_ATTENTION, [V.VbsArg(0, q.ctypes.data, 0), V.VbsArg(0, kcache.ctypes.data, 0),
                              V.VbsArg(0, vcache.ctypes.data, 0), V.VbsArg(0, out.ctypes.data, 0),
                              be.u32_arg(keep, seq), be.u32_arg(keep, 1), be.u32_arg(keep, mc),
                              be.u32_arg(keep, nq), be.u32_arg(keep, nkv), be.u32_arg(keep, hd),
                              be.f32_arg(keep, 1.0 / np.sqrt(np.float32(hd)))])
        arrays[f"att_out{seq}"] = out
    # embedding through the ops table (one token per dispatch)
    for t in TYPES:
        table = V.synth_matrix(host, t, 16, 512, SEED, 3700 + t)
        out = np.zeros(512, np.float32)
        pipe = be.ops.compile_embed_pipeline(dev, t, None, 0)
        assert be.dispatch(pipe, [V.VbsArg(0, table.ctypes.data, 0), be.u32_arg(keep, 11),
                                  V.VbsArg(0, out.ctypes.data, 0), be.u32_arg(keep, 512)])
        arrays[f"emb{t}_table"], arrays[f"emb{t}_out"] = table, out
    np.savez_compressed(os.path.join(HERE, "prims.npz"), **arrays)


TINY = dict(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
            max_ctx=64)


def gen_tiny(host):
    be = ref_backend()
    model = V.SynthModel(host, **TINY, seed=99)
    d = V.Decoder(host, be, model)
    toks, last = [], None
    tok = 1
    for pos in range(24):
        last = d.step(tok, pos)
        tok = int(np.argmax(last))
        toks.append(tok)
    d.close()
    with open(os.path.join(HERE, "tiny_model.json"), "w") as fh:
        json.dump({"config": TINY, "seed": 99, "start_token": 1, "tokens": toks,
                   "last_logits_f32_bits": [int(v) for v in last.view(np.uint32)]}, fh)


def write_provenance():
    """Where the fixtures were computed: the libm behind the reference's powf,
    cosf, sinf and expf (RoPE angles, softmax weights in prims.npz and
    tiny_model.json) and the compiler that built the reference sources."""
    import platform
    import subprocess
    cc = subprocess.run(["gcc", "--version"], capture_output=True, text=True).stdout.splitlines()
    info = {"libc": " ".join(platform.libc_ver()), "cc": cc[0] if cc else "",
            "machine": platform.machine(),
            "reference_build": "gcc -std=c11 -O3 -D_GNU_SOURCE (oracle/Makefile, ref target)"}
    with open(os.path.join(HERE, "provenance.json"), "w") as f:
        json.dump(info, f, indent=1)


if __name__ == "__main__":
    write_provenance()
    lib = ref_lib()
    host = V.load_host()
    gen_dequant(lib, host)
    gen_half(lib)
    gen_linear(host)
    gen_prims(host)
    gen_tiny(host)
    print("golden fixtures written to", HERE)
