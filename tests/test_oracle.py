"""Pinning the CPU oracle (oracle/vbs_oracle.c) before it is trusted as the
checker of the gfx950 kernels.

Three kinds of evidence, chosen so that a plausible slip (a dropped term, a
wrong shift or index, swapped operands, a different rounding) fails one:
  * golden vectors written by the reference's own code (tests/golden/, made by
    gen_golden.py from oracle/_ref) -- compared bit for bit;
  * the reference's known-answer blocks (src/main.c:452-516) and its
    self-test's unit-scale packers (src/vbs_backend_test.c:277-323);
  * closed forms and exhaustive checks (IEEE half conversion, pack/unpack
    round trips, linearity, integer-exact dots).
"""
import hashlib
import json
import math
import os
import struct

import numpy as np
import pytest

import vbs_gfx950 as V
from oracle_lib import REF_SO, Oracle, reference_cpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold_npz(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def f16bits(v):
    return struct.unpack("<H", struct.pack("<e", v))[0]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- half precision
def test_f16_to_f32_exhaustive_vs_ieee_and_golden(orc):
    h = np.arange(65536, dtype=np.uint16)
    # through a stored row (an F16 "row" of all 65536 halves): a float return
    # value would pass through a double and quiet signalling NaN payloads
    got = orc.dequant_row(V.F16, h.view(np.uint8), 65536)
    # IEEE binary16 -> binary32 is exact; numpy implements it. NaNs: the
    # reference keeps the payload bits (man << 13), numpy quiets them.
    ieee = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ieee)
    assert np.array_equal(bits(got)[~nan], bits(ieee)[~nan])
    exp = ((h[nan].astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | ((h[nan].astype(np.uint32) & 0x3FF) << 13)
    assert np.array_equal(bits(got)[nan], exp)
    meta = json.load(open(os.path.join(GOLD, "half.json")))
    assert hashlib.sha256(bits(got).astype("<u4").tobytes()).hexdigest() == meta["f16_to_f32_sha256"]


def test_f32_to_f16_closed_forms(orc):
    f = lambda v: orc._f32_to_f16(float(np.float32(v)))
    assert f(1.0) == 0x3C00 and f(-2.0) == 0xC000 and f(0.0) == 0 and f(-0.0) == 0x8000
    assert f(65504.0) == 0x7BFF and f(65520.0) == 0x7C00 and f(1e9) == 0x7C00
    assert f(float("inf")) == 0x7C00 and f(float("-inf")) == 0xFC00
    assert f(float("nan")) == 0x7C01  # NaN keeps only a nonzero-payload bit
    # normals round to nearest, ties to even: 1 + 2^-11 is a tie -> 1.0;
    # 1 + 3*2^-11 is a tie -> 1 + 2^-9 (even mantissa)
    assert f(1.0 + 2 ** -11) == 0x3C00 and f(1.0 + 3 * 2 ** -11) == 0x3C02
    # subnormals round half UP (not to even): 0.5 ulp (2^-25) -> 1 ulp;
    # 2.5 ulp -> 3 ulp; below 2^-25 -> 0
    ulp = 2.0 ** -24
    assert f(0.5 * ulp) == 0x0001 and f(2.5 * ulp) == 0x0003 and f(0.49 * ulp) == 0
    assert f(-2.5 * ulp) == 0x8003
    # the largest subnormal rounding up becomes the smallest normal
    assert f(1023.5 * ulp) == 0x0400
    # against IEEE (numpy) away from the subnormal ties
    rng = np.random.default_rng(3)
    for v in rng.standard_normal(20000).astype(np.float32) * 100:
        assert f(v) == f16bits(np.float16(v))


def test_f32_to_f16_exhaustive_digest_matches_reference(orc):
    """All 2^32 inputs: the oracle's converter hashes to the digest the
    reference's vbs_f32_to_f16 produced (tests/golden/half.json)."""
    meta = json.load(open(os.path.join(GOLD, "half.json")))
    d = orc._digest_f32_to_f16(orc.f16_fn, os.cpu_count() or 4)
    assert f"{d:016x}" == meta["f32_to_f16_digest"]
    for v, vb, want in meta["f32_to_f16_edges"]:
        assert orc._f32_to_f16(struct.unpack("<f", struct.pack("<I", vb))[0]) == want, v


# ---------------------------------------------------------------- block decoders
def test_known_answer_blocks(orc):
    """src/main.c:452-516 (the reference's --dequant checks)."""
    def deq(t, blk):
        out = np.zeros(256, np.float32)
        assert orc._dequant_block(t, blk.ctypes.data, out.ctypes.data) == V.GEOMETRY[t][0]
        return out
    b = np.zeros(18, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(orc._f32_to_f16(0.5)).tobytes(), np.uint8)
    for i in range(16):
        b[2 + i] = i | ((15 - i) << 4)
    y = deq(V.Q4_0, b)
    assert y[0] == 0.5 * (0 - 8) and y[16] == 0.5 * (15 - 8)
    b = np.zeros(34, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(orc._f32_to_f16(0.125)).tobytes(), np.uint8)
    for i in range(32):
        b[2 + i] = (i * 7 - 80) & 0xFF  # (uint8_t)(int8_t)(i*7-80), wrapping as in C
    y = deq(V.Q8_0, b)
    assert y[0] == 0.125 * -80 and y[31] == 0.125 * (((31 * 7 - 80) + 128) % 256 - 128)
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(orc._f32_to_f16(2.0)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(orc._f32_to_f16(1.0)).tobytes(), np.uint8)
    b[4], b[8], b[5], b[9], b[16] = 2, 1, 3, 0, 0x21
    y = deq(V.Q4_K, b)
    assert y[0] == 3.0 and y[32] == 12.0
    b = np.zeros(210, np.uint8)
    b[192], b[194], b[0], b[32] = 3, 1, 0x21, 0x05
    b[208:210] = np.frombuffer(np.uint16(orc._f32_to_f16(2.0)).tobytes(), np.uint8)
    y = deq(V.Q6_K, b)
    assert y[0] == -186.0 and y[32] == -54.0


@pytest.mark.parametrize("t", [V.Q4_0, V.Q4_1, V.Q8_0, V.Q4_K, V.Q6_K],
                         ids=lambda t: V.TYPE_NAMES[t])
def test_dequant_matches_reference_golden(orc, t):
    g = gold_npz("dequant_blocks.npz")
    blocks, want = g[f"t{t}_in"], g[f"t{t}_out"]
    e = V.GEOMETRY[t][0]
    for blk, w in zip(blocks, want):
        out = np.zeros(e, np.float32)
        blk = np.ascontiguousarray(blk)
        assert orc._dequant_block(t, blk.ctypes.data, out.ctypes.data) == e
        assert np.array_equal(bits(out), w)


def test_q4k_scale_min_pack_roundtrip_exhaustive(orc):
    """Every (scale, min) in 0..63 for every sub-block position survives the
    12-byte packing of the config-2 generator (the inverse of
    src/vbs_dequant.c:225-233): d = 1, dmin = 1 and nibble 1 in sub-block j
    decode to sc - m exactly; nibble 0 decodes to -m."""
    one = orc._f32_to_f16(1.0)
    for j in range(8):
        for sc in range(64):
            ms = np.arange(64)
            scs = np.full(8, 7)
            for m in (0, 17, 42, 63):
                mns = np.full(8, 5)
                scs[j], mns[j] = sc, m
                b = np.zeros(144, np.uint8)
                b[0:2] = np.frombuffer(np.uint16(one).tobytes(), np.uint8)
                b[2:4] = np.frombuffer(np.uint16(one).tobytes(), np.uint8)
                s = b[4:16]
                for k in range(4):
                    s[k] = scs[k] | ((scs[k + 4] >> 4) << 6)
                    s[k + 4] = mns[k] | ((mns[k + 4] >> 4) << 6)
                    s[k + 8] = (scs[k + 4] & 15) | ((mns[k + 4] & 15) << 4)
                g, hi = j >> 1, j & 1
                b[16 + 32 * g] = (1 << 4) if hi else 1  # element 32j gets nibble 1
                out = np.zeros(256, np.float32)
                orc._dequant_block(V.Q4_K, b.ctypes.data, out.ctypes.data)
                assert out[32 * j] == sc - m and out[32 * j + 1] == -m
            del ms


def test_q6k_unit_scale_roundtrip_exhaustive(orc):
    """src/vbs_backend_test.c:302-323 packs 6-bit values with unit scales;
    every (element, value) pair must decode to value - 32."""
    rng = np.random.default_rng(5)
    for rep in range(64):
        q = rng.integers(0, 64, 256) if rep else np.arange(256) % 64
        b = np.zeros(210, np.uint8)
        b[192:208] = 1
        b[208:210] = np.frombuffer(np.uint16(orc._f32_to_f16(1.0)).tobytes(), np.uint8)
        for e in range(256):
            h, qq, l = e >> 7, (e & 127) >> 5, e & 31
            qi = h * 64 + (qq & 1) * 32 + l
            b[qi] |= (q[e] & 15) << (4 if qq >= 2 else 0)
            b[128 + h * 32 + l] |= (q[e] >> 4) << (2 * qq)
        out = np.zeros(256, np.float32)
        orc._dequant_block(V.Q6_K, b.ctypes.data, out.ctypes.data)
        assert np.array_equal(out, (q - 32).astype(np.float32))


# ---------------------------------------------------------------- linear tile
def test_linear_matches_reference_golden_bit_exact(orc):
    g = gold_npz("linear.npz")
    i = 0
    while f"c{i}_meta" in g:
        t, rows, cols = (int(v) for v in g[f"c{i}_meta"])
        y = orc.linear(t, g[f"c{i}_w"], g[f"c{i}_x"], cols, rows, threads=1)
        assert np.array_equal(bits(y), bits(g[f"c{i}_y"])), (t, rows, cols)
        i += 1
    assert i == 9
    w, x, want = g["acc_w"], g["acc_x"], g["acc_y"]
    half, rows = 2048, 8
    rb = V.row_bytes(V.Q4_K, half)
    y = np.full(rows + 4, 3.0, np.float32)
    orc.linear(V.Q4_K, np.ascontiguousarray(w[:, :rb]), x, half, rows, y=y, col_off=256, row_off=4)
    orc.linear(V.Q4_K, np.ascontiguousarray(w[:, rb:]), x, half, rows, y=y, col_off=256 + half,
               row_off=4, accumulate=True)
    assert np.array_equal(bits(y), bits(want))


def test_linear_unit_scale_blocks_give_exact_integer_dots(orc, host):
    """Unit-scale Q4_K blocks (d=1, scales 1, mins 0; the self-test packer
    src/vbs_backend_test.c:280-300) make W an integer matrix: y = W @ x is
    exact for integer x."""
    rng = np.random.default_rng(9)
    rows, cols = 6, 512
    vals = rng.integers(0, 16, (rows, cols))
    w = np.zeros((rows, (cols // 256) * 144), np.uint8)
    one = orc._f32_to_f16(1.0)
    for r in range(rows):
        for b in range(cols // 256):
            blk = w[r, b * 144:(b + 1) * 144]
            blk[0:2] = np.frombuffer(np.uint16(one).tobytes(), np.uint8)
            blk[4:8] = 1
            blk[12:16] = 1
            for e in range(256):
                gg, ww = e >> 6, e & 63
                idx = 16 + gg * 32 + (ww & 31)
                blk[idx] |= vals[r, 256 * b + e] << (4 if ww >= 32 else 0)
    x = rng.integers(-50, 50, cols).astype(np.float32)
    y = orc.linear(V.Q4_K, w, x, cols, rows)
    assert np.array_equal(y, (vals @ x.astype(np.int64)).astype(np.float32))


def test_linear_is_linear_in_x(orc, host):
    t, rows, cols = V.Q6_K, 16, 1024
    w = V.synth_matrix(host, t, rows, cols, 1, 1)
    a, b = V.synth_normal(host, cols, 1, 2), V.synth_normal(host, cols, 1, 3)
    ya, yb = orc.linear(t, w, a, cols, rows), orc.linear(t, w, b, cols, rows)
    yab = orc.linear(t, w, (a + b).astype(np.float32), cols, rows)
    # a + b is rounded to f32 once; the tolerance covers that one rounding
    assert np.allclose(yab, ya + yb, rtol=1e-5, atol=1e-4)
    # and against a float64 dense product of the oracle's own dequantised rows
    dense = np.stack([orc.dequant_row(t, w[r], cols) for r in range(rows)]).astype(np.float64)
    assert np.array_equal(ya, (dense @ a.astype(np.float64)).astype(np.float32)) or \
        np.allclose(ya, dense @ a, rtol=1e-6, atol=1e-5)


def test_linear_threaded_is_bit_identical(orc, host):
    t, rows, cols = V.Q4_K, 300, 4096
    w = V.synth_matrix(host, t, rows, cols, 2, 1)
    x = V.synth_normal(host, cols, 2, 2)
    assert np.array_equal(bits(orc.linear(t, w, x, cols, rows, threads=1)),
                          bits(orc.linear(t, w, x, cols, rows, threads=7)))


# ---------------------------------------------------------------- primitives
def test_primitives_match_reference_golden(orc):
    g = gold_npz("prims.npz")
    for n in (4096, 384):
        assert np.array_equal(bits(orc.rms_norm(g[f"rms{n}_x"], g[f"rms{n}_w"], np.float32(1e-5))),
                              bits(g[f"rms{n}_out"]))
    for theta in (10000.0, 500000.0):
        for pos in (0, 7, 2047, 2175, 8191):
            got = orc.rope(g["rope_x"], pos, 128, 32, theta)
            assert np.array_equal(bits(got), bits(g[f"rope_{int(theta)}_{pos}"])), (theta, pos)
    kc = np.zeros(3 * 24 * 1024, np.uint16)
    vc = np.zeros_like(kc)
    orc.cache_store(g["kv_k"], g["kv_v"], kc, vc, 17, 2, 24, 1024)
    base = (2 * 24 + 17) * 1024
    assert np.array_equal(kc[base:base + 1024], g["kv_kc"])
    assert np.array_equal(vc[base:base + 1024], g["kv_vc"])
    assert np.array_equal(bits(orc.silu_mul(g["silu_g"], g["silu_u"])), bits(g["silu_out"]))
    assert np.array_equal(orc.add(g["add_a"], g["add_b"]), g["add_out"])
    for seq in (1, 64, 300):
        got = orc.attention(g["att_q"], g["att_kc"], g["att_vc"], seq, 1, 320, 8, 2, 64,
                            np.float32(1.0 / math.sqrt(64)))
        assert np.array_equal(bits(got), bits(g[f"att_out{seq}"])), seq
    for t in (V.Q4_0, V.Q4_1, V.Q8_0, V.Q4_K, V.Q6_K):
        got = orc.embed(t, g[f"emb{t}_table"], 11, 512)
        assert np.array_equal(bits(got), bits(g[f"emb{t}_out"]))


def test_primitive_closed_forms(orc, host):
    # rms_norm of a constant vector is w (up to one rounding of the scale)
    x = np.full(512, 3.0, np.float32)
    w = V.synth_normal(host, 512, 4, 1)
    assert np.allclose(orc.rms_norm(x, w, np.float32(0.0)), w, rtol=1e-6)
    # rope at position 0 is the identity; at any position it preserves pair norms
    v = V.synth_normal(host, 4 * 64, 4, 2)
    assert np.array_equal(orc.rope(v, 0, 64, 4, 10000.0), v)
    r = orc.rope(v, 1234, 64, 4, 10000.0)
    assert np.allclose(np.hypot(r[0::2], r[1::2]), np.hypot(v[0::2], v[1::2]), rtol=1e-5)
    # attention over one position returns that position's (f16) value row
    kc = V.synth_normal_f16(host, 16 * 2 * 32, 4, 3)
    vc = V.synth_normal_f16(host, 16 * 2 * 32, 4, 4)
    q = V.synth_normal(host, 4 * 32, 4, 5)
    out = orc.attention(q, kc, vc, 1, 0, 16, 4, 2, 32, np.float32(0.17))
    v0 = vc[:2 * 32].view(np.float16).astype(np.float32).reshape(2, 32)
    assert np.array_equal(out.reshape(4, 32), v0[[0, 0, 1, 1]])
    # silu(0) * u = 0; silu(g) -> g for large g
    g = np.array([0.0, 30.0, -30.0], np.float32)
    u = np.ones(3, np.float32)
    s = orc.silu_mul(g, u)
    assert s[0] == 0.0 and s[1] == 30.0 and abs(s[2]) < 1e-11


def test_tiny_model_decode_matches_reference_golden(orc, host):
    """F5: the oracle's forward pass reproduces the reference CPU backend's
    greedy tokens and final logits bit for bit."""
    from test_decode import TINY, full_cache
    meta = json.load(open(os.path.join(GOLD, "tiny_model.json")))
    assert meta["config"] == TINY
    model = V.SynthModel(host, **TINY, seed=meta["seed"])
    kc, vc = full_cache(model, None, None, 0)
    om = orc.model(model, kc, vc)
    tok, toks, lg = meta["start_token"], [], None
    for pos in range(len(meta["tokens"])):
        lg = orc.forward(om, tok, pos, TINY["vocab"], threads=4)
        tok = int(np.argmax(lg))
        toks.append(tok)
    assert toks == meta["tokens"]
    assert np.array_equal(bits(lg), np.array(meta["last_logits_f32_bits"], np.uint32))


@pytest.mark.skipif(not os.path.exists(REF_SO), reason="oracle/_ref not built here")
def test_oracle_against_reference_library_random_blocks(orc, host):
    """Where the reference's own library is present, compare fresh random
    blocks of every type directly (beyond the stored fixtures)."""
    ref = reference_cpu()
    rng = np.random.default_rng(11)
    for t in (V.Q4_0, V.Q4_1, V.Q8_0, V.Q4_K, V.Q6_K):
        e, nb = V.GEOMETRY[t]
        for _ in range(300):
            blk = rng.integers(0, 256, nb, dtype=np.uint8)
            a, b = np.zeros(e, np.float32), np.zeros(e, np.float32)
            ref.vbs_dequant_block(t, blk.ctypes.data, a.ctypes.data)
            orc._dequant_block(t, blk.ctypes.data, b.ctypes.data)
            assert np.array_equal(bits(a), bits(b))
    # the converters on random bit patterns
    for u in rng.integers(0, 2 ** 32, 50000, dtype=np.uint64):
        f = struct.unpack("<f", struct.pack("<I", int(u)))[0]
        assert ref.vbs_f32_to_f16(f) == orc._f32_to_f16(f)


@pytest.mark.skipif(not os.path.exists(REF_SO), reason="oracle/_ref not built here")
def test_lns8_rows_against_reference_embedding(orc):
    """LNS8 (value = 2^q * f32 scale) lives in the reference's host math, not in
    vbs_dequant_block, so it is pinned through the reference CPU backend's
    EMBEDDING op (vbs_host_embed_row -> vbs_host_dequant_row,
    src/vbs_host_math.h:111-121): random codes (including those whose power
    overflows to inf) and random scales, bit for bit."""
    import ctypes as C
    ref = V.Backend(C.CDLL(REF_SO), "g_vbs_cpu_backend")
    assert ref.init()
    rng = np.random.default_rng(40)
    dim, rows = 256, 24
    blocks = rng.integers(0, 256, (rows, dim // 32, 36), dtype=np.uint8)
    scales = (rng.standard_normal((rows, dim // 32)) * 2.0 ** rng.integers(-140, -100, (rows, dim // 32)))
    blocks[:, :, 32:36] = scales.astype(np.float32).view(np.uint8).reshape(rows, dim // 32, 4)
    table = np.ascontiguousarray(blocks.reshape(rows, -1))
    pipe = ref.ops.compile_embed_pipeline(ref.device(), V.LNS8, None, 0)
    assert pipe
    tb = ref.upload(table)
    out_buf = ref.alloc(dim * 4)
    for tok in range(rows):
        keep = []
        args = [V.Backend.buf_arg(tb), V.Backend.u32_arg(keep, tok), V.Backend.buf_arg(out_buf),
                V.Backend.u32_arg(keep, dim)]
        assert ref.dispatch(pipe, args)
        want = ref.download(out_buf, (dim,), np.float32)
        got = np.zeros(dim, np.float32)
        assert orc._dequant_row(V.LNS8, np.ascontiguousarray(table[tok]).ctypes.data, dim,
                                got.ctypes.data)
        assert np.array_equal(bits(got), bits(want)), tok
