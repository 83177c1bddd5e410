"""gfx950 kernels vs the CPU oracle, through the C ABI of libvbs_gfx950.so.

Bars (north star): dequantised values and the gather bit-exact; matvec
relative L2 error <= 1e-5 against the oracle's double-accumulated
vbs_host_linear_tile restatement, over the vector and per row (lin_err); RoPE, KV store and add bit-exact; RMSNorm
within 1e-6 relative; SiLU*up 1e-5 and attention 1e-4 (the reference
self-test's tolerances, src/vbs_backend_test.c:540, 798).
"""
import math

import numpy as np
import pytest

import vbs_gfx950 as V

pytestmark = pytest.mark.gpu

SEED = 20260101
TYPES = [V.Q4_0, V.Q4_1, V.Q8_0, V.Q4_K, V.Q6_K, V.F16, V.F32]
LIN_TOL = 1e-5


class Mem:
    """Device allocations freed at the end of a test."""

    def __init__(self, dev):
        self.dev, self.ptrs = dev, []

    def up(self, a):
        p = self.dev.upload(a)
        self.ptrs.append(p)
        return p

    def zeros(self, n, dtype=np.float32):
        return self.up(np.zeros(n, dtype))

    def close(self):
        for p in self.ptrs:
            self.dev.free(p)


@pytest.fixture
def mem(dev):
    m = Mem(dev)
    yield m
    m.close()


def rel_l2(got, want):
    want = want.astype(np.float64)
    return float(np.linalg.norm(got.astype(np.float64) - want) / max(np.linalg.norm(want), 1e-30))


def lin_err(got, want):
    """The matvec bar, over the whole vector and per row: the larger of the
    relative L2 error and max_r |got_r - want_r| / (|want_r| + rms(want)),
    so that one row off by more than 1e-5 of its own size (or, for a row
    near zero, of the vector's rms) fails however many rows are right."""
    g, w = got.astype(np.float64), want.astype(np.float64)
    rms = max(float(np.sqrt(np.mean(w * w))), 1e-30)
    per_row = float(np.max(np.abs(g - w) / (np.abs(w) + rms))) if w.size else 0.0
    return max(rel_l2(got, want), per_row)


def synth_x(host, n, stream=7):
    return V.synth_normal(host, n, SEED, stream)


@pytest.mark.parametrize("t", TYPES + [V.LNS8], ids=lambda t: V.TYPE_NAMES[t])
def test_dequant_rows_bit_exact(dev, host, oracle, mem, t):
    rows, cols = 48, 4096
    if t == V.LNS8:
        # codes U{0..255} (inf above 127 is part of the format) and a finite scale
        rng = np.random.default_rng(SEED)
        w = rng.integers(0, 256, size=(rows, cols // 32, 36), dtype=np.uint8)
        w[:, :, 32:36] = np.frombuffer(np.float32(1.0 / 256).tobytes(), np.uint8)
        w = w.reshape(rows, -1)
    else:
        w = V.synth_matrix(host, t, rows, cols, SEED, 11)
    pw, out = mem.up(w), mem.zeros(rows * cols)
    dev.dequant_rows(t, pw, 0, rows, cols, out)
    got = dev.download(out, (rows, cols), np.float32)
    want = np.stack([oracle.dequant_row(t, w[r], cols) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", TYPES, ids=lambda t: V.TYPE_NAMES[t])
@pytest.mark.parametrize("rows,cols", [(16, 4096), (16, 11008), (200, 512), (1, 256)])
def test_linear_parity(dev, host, oracle, mem, t, rows, cols):
    w = V.synth_matrix(host, t, rows, cols, SEED, 21)
    x = synth_x(host, cols)
    pw, px, py = mem.up(w), mem.up(x), mem.zeros(rows)
    dev.linear(t, pw, px, py, cols, rows)
    got = dev.download(py, rows, np.float32)
    want = oracle.linear(t, w, x, cols, rows)
    assert lin_err(got, want) <= LIN_TOL


@pytest.mark.parametrize("t,rows,cols", [(V.Q4_K, 4096, 11008), (V.Q4_K, 11008, 4096),
                                         (V.Q6_K, 4096, 11008), (V.Q8_0, 11008, 4096),
                                         (V.Q4_0, 4096, 4096), (V.Q6_K, 32000, 4096)],
                         ids=["q4k_4096x11008", "q4k_11008x4096", "q6k_4096x11008",
                              "q80_11008x4096", "q40_4096x4096", "q6k_32000x4096_head"])
def test_linear_full_size(dev, host, oracle, mem, t, rows, cols):
    w = V.synth_matrix(host, t, rows, cols, SEED, 31)
    x = synth_x(host, cols)
    pw, px, py = mem.up(w), mem.up(x), mem.zeros(rows)
    dev.linear(t, pw, px, py, cols, rows)
    got = dev.download(py, rows, np.float32)
    want = oracle.linear(t, w, x, cols, rows, threads=16)
    assert lin_err(got, want) <= LIN_TOL


@pytest.mark.parametrize("t,rows,cols", [(V.Q4_K, 28672, 8192), (V.Q6_K, 8192, 28672),
                                         (V.Q4_K, 11008, 4096), (V.Q8_0, 4096, 11008)],
                         ids=["q4k_28672x8192", "q6k_8192x28672", "q4k_11008x4096",
                              "q80_4096x11008"])
def test_linear_full_size_properties(dev, host, oracle, mem, t, rows, cols):
    """Size-independent properties over every row of the full matrices, where
    the oracle checks a sample of rows. x travels as three balanced digit
    planes of rint(x 2^(22-e)) per 32-element sub-block, so scaling x by a
    power of two leaves every digit unchanged and scales every row value
    exactly. Negating x negates each integer dot, but the digits of -X are not
    the negated digits of X (they range over -128..127), and the two low
    planes are added in int32 before one conversion to float: that sum stays
    below 2^24, hence exact, only for Q4_K's 32 x 15-bounded groups, so the
    negation is exact for Q4_K and within a few ulps otherwise. A row's value
    depends only on its own bytes, so reversing the rows reverses y exactly.
    The sampled rows match the oracle."""
    w = V.synth_matrix(host, t, rows, cols, SEED, 41)
    x = synth_x(host, cols, stream=42)
    pw, pr = mem.up(w), mem.up(np.ascontiguousarray(w[::-1]))
    ys = {}
    for name, xv, wp in (("x", x, pw), ("4x", 4.0 * x, pw), ("-x", -x, pw), ("rev", x, pr)):
        px, py = mem.up(xv.astype(np.float32)), mem.zeros(rows)
        dev.linear(t, wp, px, py, cols, rows)
        ys[name] = dev.download(py, rows, np.float32)
    y = ys["x"]
    assert np.all(np.isfinite(y))
    assert np.array_equal(ys["4x"], 4.0 * y)
    if t == V.Q4_K:
        assert np.array_equal(ys["-x"].view(np.uint32), (-y).view(np.uint32))
    else:
        assert rel_l2(-ys["-x"], y) <= 1e-6
    assert np.array_equal(ys["rev"].view(np.uint32), y[::-1].view(np.uint32))
    sample = np.r_[0:96, rows // 2 - 48:rows // 2 + 48, rows - 96:rows]
    want = oracle.linear(t, w[sample], x, cols, len(sample), threads=16)
    assert lin_err(y[sample], want) <= LIN_TOL


@pytest.mark.parametrize("rows,cols", [(8192, 8192), (9000, 6144)], ids=["8192x8192", "9000x6144"])
@pytest.mark.parametrize("accumulate", [False, True], ids=["store", "acc"])
def test_q4k_two_tile_plan(dev, host, oracle, mem, rows, cols, accumulate):
    """Q4_K rows of 17-32 blocks with two or more 16-row tiles per CU and
    fewer than 1024 tiles take two tiles per workgroup, the block's x
    operands serving both (the 70B O projection, 512 tiles). 9000 rows end in
    a workgroup whose second tile lies past the matrix. Every row against the
    oracle, store and accumulate."""
    w = V.synth_matrix(host, V.Q4_K, rows, cols, SEED, 61)
    x = synth_x(host, cols, stream=62)
    y0 = synth_x(host, rows, 63)
    pw, px, py = mem.up(w), mem.up(x), mem.up(y0)
    dev.linear(V.Q4_K, pw, px, py, cols, rows, accumulate=accumulate)
    got = dev.download(py, rows, np.float32)
    want = oracle.linear(V.Q4_K, w, x, cols, rows, y=y0.copy() if accumulate else None,
                         accumulate=accumulate, threads=16)
    assert lin_err(got, want) <= LIN_TOL


@pytest.mark.parametrize("t,rows,cols", [(V.Q4_K, 4096, 4096), (V.Q4_K, 1024, 4096),
                                         (V.Q4_K, 11008, 4096), (V.Q4_K, 4096, 11008),
                                         (V.Q6_K, 4096, 4096), (V.Q6_K, 4096, 11008)],
                         ids=["q4k_4096x4096", "q4k_1024x4096", "q4k_11008x4096",
                              "q4k_4096x11008", "q6k_4096x4096", "q6k_4096x11008"])
@pytest.mark.parametrize("join", ["norm", "rope", "norm_rope", "acc", "silu", "cache"])
def test_linear_fused_equals_ops_one_by_one(dev, host, mem, t, rows, cols, join):
    """vbs_gfx950_linear_fused with each neighbour it takes (the RMSNorm
    before, the RoPE, residual add, SiLU gate or f16 K/V store after) writes
    the same bits, to every buffer, as the device library's ops issued one by
    one: the matvec, the normalised x, the rotated rows, the accumulator, the
    hidden vector and both cache rows. The shapes cover the LDS-DMA Q4_K
    kernel (16-block rows), the matrix-core fallback (1024 rows, 43-block
    rows) and the Q6_K ring kernel (the add after a 43-block Q6_K row)."""
    hd, pos, theta, eps = 128, 2175, 500000.0, 1e-5
    layer, max_ctx = 1, 2200
    w = V.synth_matrix(host, t, rows, cols, SEED, 131)
    x = synth_x(host, cols, 132) * 1.7
    nw = synth_x(host, cols, 133)
    acc0 = synth_x(host, rows, 134)
    gate = synth_x(host, rows, 135) * 3.0
    krow = synth_x(host, rows, 136) * 40.0
    pw, px, pnw, pg, pk = mem.up(w), mem.up(x), mem.up(nw), mem.up(gate), mem.up(krow)
    norm = join in ("norm", "norm_rope")
    cache_elems = 2 * max_ctx * rows

    def buffers():
        return dict(y=mem.zeros(rows), xn=mem.zeros(cols), acc=mem.up(acc0), hid=mem.zeros(rows),
                    kc=mem.zeros(cache_elems, np.uint16), vc=mem.zeros(cache_elems, np.uint16))

    ref, fus = buffers(), buffers()
    # the ops one by one
    xin = px
    if norm:
        dev.rms_norm(px, pnw, ref["xn"], cols, eps)
        xin = ref["xn"]
    dev.linear(t, pw, xin, ref["y"], cols, rows)
    if join in ("rope", "norm_rope"):
        dev.rope(ref["y"], pos, hd, rows // hd, theta)
    elif join == "acc":
        dev.add(ref["acc"], ref["y"], ref["acc"], rows)
    elif join == "silu":
        dev.silu_mul(pg, ref["y"], ref["hid"], rows)
    elif join == "cache":
        dev.cache_store(pk, ref["y"], ref["kc"], ref["vc"], pos, layer, max_ctx, rows)
    # one launch
    j = {}
    if norm:
        j.update(norm_w=pnw, norm_eps=eps, x_normed=fus["xn"])
    if join in ("rope", "norm_rope"):
        j.update(rope=1, pos=pos, head_dim=hd, theta=theta)
    elif join == "acc":
        j.update(acc=fus["acc"])
    elif join == "silu":
        j.update(gate=pg, hidden=fus["hid"])
    elif join == "cache":
        j.update(k_row=pk, kc=fus["kc"], vc=fus["vc"], kv_off=(layer * max_ctx + pos) * rows)
    assert dev.linear_fused(t, pw, px, fus["y"], cols, rows, **j)
    for name, n, dt in (("y", rows, np.float32), ("xn", cols, np.float32),
                        ("acc", rows, np.float32), ("hid", rows, np.float32),
                        ("kc", cache_elems, np.uint16), ("vc", cache_elems, np.uint16)):
        a = dev.download(ref[name], n, dt)
        b = dev.download(fus[name], n, dt)
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), name


@pytest.mark.parametrize("t,q_rows,kv_rows,cols", [
    (V.Q4_K, 4096, 1024, 4096), (V.Q4_K, 8192, 1024, 8192), (V.Q4_K, 256, 128, 512),
    (V.Q6_K, 4096, 1024, 4096), (V.Q4_K, 4096, 4096, 4096)],
    ids=["q4k_7b", "q4k_70b", "q4k_small", "q6k_7b", "q4k_mha"])
@pytest.mark.parametrize("norm", [True, False], ids=["norm", "plain"])
def test_qkv_fused_equals_ops_one_by_one(dev, host, mem, t, q_rows, kv_rows, cols, norm):
    """vbs_gfx950_qkv_fused (the shim's grouped NORMALIZE, q, ROTARY, k,
    ROTARY, v, CACHE) writes the same bits to the normalised x, q, k, v and
    both caches as the device library's ops issued one by one. The shapes
    take the LDS-DMA kernel (16-block rows, 6144 or more rows), the
    matrix-core kernel's ranged and tiled plans, and Q6_K."""
    hd, pos, theta, eps, layer, max_ctx = 128, 1999, 10000.0, 1e-5, 2, 2048
    wq = V.synth_matrix(host, t, q_rows, cols, SEED, 151)
    wk = V.synth_matrix(host, t, kv_rows, cols, SEED, 152)
    wv = V.synth_matrix(host, t, kv_rows, cols, SEED, 153)
    x, nw = synth_x(host, cols, 154) * 2.0, synth_x(host, cols, 155)
    pq, pk, pv, px, pnw = mem.up(wq), mem.up(wk), mem.up(wv), mem.up(x), mem.up(nw)
    cache = 3 * max_ctx * kv_rows

    def buffers():
        return dict(xn=mem.zeros(cols), q=mem.zeros(q_rows), k=mem.zeros(kv_rows),
                    v=mem.zeros(kv_rows), kc=mem.zeros(cache, np.uint16),
                    vc=mem.zeros(cache, np.uint16))

    ref, fus = buffers(), buffers()
    xin = px
    if norm:
        dev.rms_norm(px, pnw, ref["xn"], cols, eps)
        xin = ref["xn"]
    dev.linear(t, pq, xin, ref["q"], cols, q_rows)
    dev.rope(ref["q"], pos, hd, q_rows // hd, theta)
    dev.linear(t, pk, xin, ref["k"], cols, kv_rows)
    dev.rope(ref["k"], pos, hd, kv_rows // hd, theta)
    dev.linear(t, pv, xin, ref["v"], cols, kv_rows)
    dev.cache_store(ref["k"], ref["v"], ref["kc"], ref["vc"], pos, layer, max_ctx, kv_rows)
    assert dev.qkv_fused(t, pq, pk, pv, px, cols, q_rows, kv_rows, pnw if norm else 0, eps,
                         fus["xn"] if norm else 0, fus["q"], fus["k"], fus["v"], pos, hd, theta,
                         fus["kc"], fus["vc"], layer, max_ctx)
    for name, n, dt in (("xn", cols, np.float32), ("q", q_rows, np.float32),
                        ("k", kv_rows, np.float32), ("v", kv_rows, np.float32),
                        ("kc", cache, np.uint16), ("vc", cache, np.uint16)):
        a = dev.download(ref[name], n, dt)
        b = dev.download(fus[name], n, dt)
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), name


@pytest.mark.parametrize("t,rows,cols", [(V.Q4_K, 11008, 4096), (V.Q4_K, 28672, 8192),
                                         (V.Q4_K, 512, 256), (V.Q6_K, 11008, 4096)],
                         ids=["q4k_7b", "q4k_70b", "q4k_small", "q6k_7b"])
@pytest.mark.parametrize("norm", [True, False], ids=["norm", "plain"])
def test_gate_up_fused_equals_ops_one_by_one(dev, host, mem, t, rows, cols, norm):
    """vbs_gfx950_gate_up_fused (the shim's grouped NORMALIZE, gate, up,
    ACTIVATION) writes the same bits to the normalised x, gate, up and the
    hidden vector as the ops issued one by one."""
    eps = 1e-5
    wg = V.synth_matrix(host, t, rows, cols, SEED, 161)
    wu = V.synth_matrix(host, t, rows, cols, SEED, 162)
    x, nw = synth_x(host, cols, 163) * 2.0, synth_x(host, cols, 164)
    pg, pu, px, pnw = mem.up(wg), mem.up(wu), mem.up(x), mem.up(nw)

    def buffers():
        return dict(xn=mem.zeros(cols), gate=mem.zeros(rows), up=mem.zeros(rows),
                    hid=mem.zeros(rows))

    ref, fus = buffers(), buffers()
    xin = px
    if norm:
        dev.rms_norm(px, pnw, ref["xn"], cols, eps)
        xin = ref["xn"]
    dev.linear(t, pg, xin, ref["gate"], cols, rows)
    dev.linear(t, pu, xin, ref["up"], cols, rows)
    dev.silu_mul(ref["gate"], ref["up"], ref["hid"], rows)
    assert dev.gate_up_fused(t, pg, pu, px, cols, rows, pnw if norm else 0, eps,
                             fus["xn"] if norm else 0, fus["gate"], fus["up"], fus["hid"])
    for name, n in (("xn", cols), ("gate", rows), ("up", rows), ("hid", rows)):
        a = dev.download(ref[name], n, np.float32)
        b = dev.download(fus[name], n, np.float32)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name


def test_linear_fused_declines_and_rejects(dev, host, mem):
    """Combinations no fused kernel takes come back as 2 (nothing launched,
    y untouched); half-given neighbours are errors."""
    rows, cols = 4096, 4096
    w = V.synth_matrix(host, V.Q4_K, rows, cols, SEED, 141)
    pw, px, py = mem.up(w), mem.up(synth_x(host, cols, 142)), mem.up(np.full(rows, 7.0, np.float32))
    pa, pn = mem.zeros(rows), mem.up(synth_x(host, cols, 143))
    xn = mem.zeros(cols)
    declined = [dict(), dict(acc=pa, rope=1, pos=0, head_dim=128, theta=1e4),
                dict(norm_w=pn, x_normed=xn, acc=pa), dict(gate=pa, hidden=pa, acc=pa),
                dict(rope=1, pos=0, head_dim=96, theta=1e4)]
    for j in declined:
        assert not dev.linear_fused(V.Q4_K, pw, px, py, cols, rows, **j), j
    qw = mem.up(V.synth_matrix(host, V.Q8_0, rows, cols, SEED, 144))
    assert not dev.linear_fused(V.Q8_0, qw, px, py, cols, rows, acc=pa)
    assert np.all(dev.download(py, rows, np.float32) == 7.0)
    for j in (dict(norm_w=pn), dict(gate=pa), dict(k_row=pa, kc=pa)):
        with pytest.raises(V.GpuError):
            dev.linear_fused(V.Q4_K, pw, px, py, cols, rows, **j)


@pytest.mark.parametrize("t", [V.Q4_K, V.Q6_K, V.Q8_0, V.Q4_0], ids=lambda t: V.TYPE_NAMES[t])
def test_linear_activation_edge_cases(dev, host, oracle, mem, t):
    """x with all-zero sub-blocks, 1e4 outliers, subnormal-scale blocks and
    huge blocks: the result must stay within the same relative L2 bar."""
    rows, cols = 64, 4096
    w = V.synth_matrix(host, t, rows, cols, SEED, 23)
    x = synth_x(host, cols, 24)
    x[0:32] = 0.0                      # an all-zero sub-block
    x[40] = 1.0e4                      # an outlier in an otherwise N(0,1) sub-block
    x[64:96] *= 1e-40                  # subnormal-scale sub-block
    x[96:128] *= 1e30                  # huge sub-block
    x[200] = -0.0
    pw, px, py = mem.up(w), mem.up(x), mem.zeros(rows)
    dev.linear(t, pw, px, py, cols, rows)
    got = dev.download(py, rows, np.float32)
    want = oracle.linear(t, w, x, cols, rows)
    assert lin_err(got, want) <= LIN_TOL


@pytest.mark.parametrize("t", [V.Q4_K, V.Q6_K, V.Q4_0, V.Q4_1, V.Q8_0],
                         ids=lambda t: V.TYPE_NAMES[t])
@pytest.mark.parametrize("rows,cols", [(1, 256), (3, 768), (37, 4352), (700, 8192), (64, 16640),
                                       (5, 28672), (19, 11008), (1100, 4096)])
def test_kquant_odd_shapes(dev, host, oracle, mem, t, rows, cols):
    """Row counts that leave streams and waves partly idle, several waves per
    row (cols > 4096), 65 and 112 blocks of 256 per row, misaligned x
    (col_off 3) and y (row_off 5) windows; for Q6_K and the 32-element block
    types (units of 144, 160, 272 bytes) also rows at every 2-byte offset and
    a last unit ending off a 16-byte boundary; four tiles per workgroup
    (1100 rows)."""
    w = V.synth_matrix(host, t, rows, cols, SEED, 25)
    x = synth_x(host, cols + 3, 26)
    pw, px = mem.up(w), mem.up(x)
    py = mem.up(np.full(rows + 5, -2.0, np.float32))
    dev.linear(t, pw, px, py, cols, rows, col_off=3, row_off=5, accumulate=True)
    got = dev.download(py, rows + 5, np.float32)
    want = np.full(rows + 5, -2.0, np.float32)
    oracle.linear(t, w, x, cols, rows, y=want, col_off=3, row_off=5, accumulate=True)
    assert np.array_equal(got[:5], want[:5])
    assert lin_err(got[5:], want[5:]) <= LIN_TOL


@pytest.mark.parametrize("t", [V.Q6_K, V.Q4_0, V.Q4_1, V.Q8_0], ids=lambda t: V.TYPE_NAMES[t])
@pytest.mark.parametrize("rows,cols", [(3, 768), (37, 4352), (4096, 11008)])
@pytest.mark.parametrize("off", [2, 6, 14])
def test_kquant_matrix_base_off_16_bytes(dev, host, oracle, mem, t, rows, cols, off):
    """A matrix whose first byte is only 2-byte aligned (these types' blocks
    are, so a matrix may start anywhere even): the matrix-core kernels read it
    as 16-byte chunks counted from the address rounded down to 16, never
    before that granule or past the matrix's last one. The batched kernel
    (Q6_K) reads it the same way."""
    w = V.synth_matrix(host, t, rows, cols, SEED, 27)
    x = synth_x(host, cols, 28)
    base = dev.alloc(w.nbytes + 32)
    mem.ptrs.append(base)
    pw = base + off
    dev.write(pw, w)
    px, py = mem.up(x), mem.zeros(rows)
    dev.linear(t, pw, px, py, cols, rows)
    got = dev.download(py, rows, np.float32)
    sample = np.unique(np.r_[0:min(rows, 48), max(rows - 48, 0):rows])
    want = oracle.linear(t, w[sample], x, cols, len(sample), threads=16)
    assert lin_err(got[sample], want) <= LIN_TOL
    if t == V.Q6_K:
        batch = 5
        xb = np.stack([synth_x(host, cols, 29 + b) for b in range(batch)])
        pxb, pyb = mem.up(xb), mem.zeros(batch * rows)
        dev.linear_batch(t, pw, pxb, cols, pyb, rows, cols, rows, batch)
        gotb = dev.download(pyb, (batch, rows), np.float32)
        for b in range(batch):
            wantb = oracle.linear(t, w[sample], xb[b], cols, len(sample), threads=16)
            assert lin_err(gotb[b][sample], wantb) <= LIN_TOL


@pytest.mark.parametrize("rows,cols,off", [(4096, 11008, 0), (3000, 8448, 0), (2100, 12288, 0),
                                          (3001, 11008, 10), (8192, 28672, 0), (4100, 28672, 0),
                                          (5000, 25088, 0)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_q6k_ring_kernel_shapes(dev, host, oracle, mem, rows, cols, off, accumulate):
    """Q6_K rows of 33-48 blocks over 2049-4096 rows and of 97-112 blocks
    over 4097-8192 rows take the LDS-DMA ring kernel: full row ranges (16 and
    32 rows per workgroup), short ones (12, 9, 17 and 20), 33, 48, 98 and 112
    blocks, and a matrix starting 10 bytes past a 16-byte boundary whose last
    block still ends inside its last aligned chunk; every row against the
    oracle."""
    w = V.synth_matrix(host, V.Q6_K, rows, cols, SEED, 31)
    x = synth_x(host, cols, 32)
    base = dev.alloc(w.nbytes + 32)
    mem.ptrs.append(base)
    pw = base + off
    dev.write(pw, w)
    y0 = synth_x(host, rows, 33)
    px, py = mem.up(x), mem.up(y0)
    dev.linear(V.Q6_K, pw, px, py, cols, rows, accumulate=accumulate)
    got = dev.download(py, rows, np.float32)
    want = oracle.linear(V.Q6_K, w, x, cols, rows, y=y0.copy() if accumulate else None,
                         accumulate=accumulate, threads=16)
    assert lin_err(got, want) <= LIN_TOL


def test_linear_offsets_accumulate(dev, host, oracle, mem):
    """Two column tiles into one output window: offsets index x and y, the
    second tile accumulates (src/vbs_backend_test.c:888-948)."""
    t, rows, cols, half = V.Q4_K, 64, 4096, 2048
    w = V.synth_matrix(host, t, rows, cols, SEED, 41)
    x = synth_x(host, cols + 512)
    rb = V.row_bytes(t, half)
    tiles = [np.ascontiguousarray(w[:, i * rb:(i + 1) * rb]) for i in range(2)]
    py = mem.up(np.full(rows + 8, 7.0, np.float32))
    px = mem.up(x)
    for i, tile in enumerate(tiles):
        dev.linear(t, mem.up(tile), px, py, half, rows, col_off=256 + i * half, row_off=8,
                   accumulate=(i == 1))
    got = dev.download(py, rows + 8, np.float32)
    want = np.full(rows + 8, 7.0, np.float32)
    oracle.linear(t, tiles[0], x, half, rows, y=want, col_off=256, row_off=8)
    oracle.linear(t, tiles[1], x, half, rows, y=want, col_off=256 + half, row_off=8,
                  accumulate=True)
    assert np.array_equal(got[:8], want[:8])  # untouched head
    assert lin_err(got[8:], want[8:]) <= LIN_TOL


@pytest.mark.parametrize("t", [V.Q4_K, V.Q6_K, V.Q8_0], ids=lambda t: V.TYPE_NAMES[t])
@pytest.mark.parametrize("batch", [1, 3, 8])
def test_linear_batch_matches_single(dev, host, oracle, mem, t, batch):
    rows, cols = 96, 4096
    w = V.synth_matrix(host, t, rows, cols, SEED, 51)
    X = np.stack([synth_x(host, cols, 60 + b) for b in range(batch)])
    pw, px, py = mem.up(w), mem.up(X), mem.zeros(batch * rows)
    dev.linear_batch(t, pw, px, cols, py, rows, cols, rows, batch)
    got = dev.download(py, (batch, rows), np.float32)
    for b in range(batch):
        assert lin_err(got[b], oracle.linear(t, w, X[b], cols, rows)) <= LIN_TOL


@pytest.mark.parametrize("t", TYPES, ids=lambda t: V.TYPE_NAMES[t])
def test_embed_gather_bit_exact(dev, host, oracle, mem, t):
    vocab, dim = 1000, 4096
    table = V.synth_matrix(host, t, vocab, dim, SEED, 61)
    pt, out = mem.up(table), mem.zeros(dim)
    ids = [0, 1, 999, 517, 64]
    for tok in ids:
        dev.embed(t, pt, tok, out, dim)
        got = dev.download(out, dim, np.float32)
        want = oracle.embed(t, table, tok, dim)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q6k_gather_64_tokens(dev, host, oracle, mem):
    """Config 3: 64 random ids from a 32000-row Q6_K table, batched gather."""
    vocab, dim = 32000, 4096
    table = V.synth_matrix(host, V.Q6_K, vocab, dim, SEED, 62)
    ids = np.random.default_rng(SEED).integers(0, vocab, 64).astype(np.uint32)
    pt, pid, out = mem.up(table), mem.up(ids), mem.zeros(64 * dim)
    dev.dequant_rows(V.Q6_K, pt, pid, 64, dim, out)
    got = dev.download(out, (64, dim), np.float32)
    for i, tok in enumerate(ids):
        want = oracle.embed(V.Q6_K, table, int(tok), dim)
        assert np.array_equal(got[i].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n", [384, 4096, 8192, 1000])
def test_rms_norm(dev, host, oracle, mem, n):
    x = synth_x(host, n, 71) * 2.0
    w = synth_x(host, n, 72)
    px, pw, po = mem.up(x), mem.up(w), mem.zeros(n)
    dev.rms_norm(px, pw, po, n, 1e-5)
    got = dev.download(po, n, np.float32)
    want = oracle.rms_norm(x, w, 1e-5)
    assert np.max(np.abs(got - want) / (np.abs(want) + 1e-30)) <= 1e-6


@pytest.mark.parametrize("pos", [0, 7, 2047, 2175, 8191])
@pytest.mark.parametrize("theta", [10000.0, 500000.0])
def test_rope_bit_exact(dev, host, oracle, mem, pos, theta):
    nh, hd = 32, 128
    x = synth_x(host, nh * hd, 81)
    px = mem.up(x)
    dev.rope(px, pos, hd, nh, theta)
    got = dev.download(px, nh * hd, np.float32)
    want = oracle.rope(x, pos, hd, nh, theta)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_cache_store_bit_exact(dev, host, oracle, mem):
    layers, max_ctx, kvd = 3, 40, 1024
    # include subnormal, tie, overflow and NaN inputs
    k = synth_x(host, kvd, 91) * 1e-5
    v = synth_x(host, kvd, 92) * 3e4
    k[:8] = [6.1e-5, -3.05e-5, 2 ** -25, 2 ** -26, 65520.0, -1e9, np.nan, 0.0]
    kc = np.zeros(layers * max_ctx * kvd, np.uint16)
    vc = np.zeros_like(kc)
    pk, pv, pkc, pvc = mem.up(k), mem.up(v), mem.up(kc), mem.up(vc)
    dev.cache_store(pk, pv, pkc, pvc, 17, 2, max_ctx, kvd)
    gk = dev.download(pkc, kc.size, np.uint16)
    gv = dev.download(pvc, vc.size, np.uint16)
    oracle.cache_store(k, v, kc, vc, 17, 2, max_ctx, kvd)
    assert np.array_equal(gk, kc) and np.array_equal(gv, vc)


@pytest.mark.parametrize("n", [777, 11008, 28672])
def test_silu_mul(dev, host, oracle, mem, n):
    g = synth_x(host, n, 101) * 3.0
    u = synth_x(host, n, 102)
    pg, pu, po = mem.up(g), mem.up(u), mem.zeros(n)
    dev.silu_mul(pg, pu, po, n)
    got = dev.download(po, n, np.float32)
    want = oracle.silu_mul(g, u)
    assert np.all(np.abs(got - want) <= 1e-5 + 1e-5 * np.abs(want))


def test_add_in_place(dev, host, oracle, mem):
    n = 4096
    a, b = synth_x(host, n, 111), synth_x(host, n, 112)
    pa, pb = mem.up(a), mem.up(b)
    dev.add(pa, pb, pa, n)
    got = dev.download(pa, n, np.float32)
    assert np.array_equal(got, oracle.add(a, b))


@pytest.mark.parametrize("nqh,nkh,hd,seq,max_ctx,layer", [
    (4, 2, 32, 6, 16, 1),          # the reference self-test case
    (32, 8, 128, 64, 2176, 0),
    (32, 8, 128, 2049, 2176, 3),
    (64, 8, 128, 1000, 1024, 1),
    (8, 8, 64, 130, 200, 0),
    (64, 8, 128, 8192, 8200, 0),   # 70B shape at the config-5 context
    (16, 1, 256, 300, 512, 0),     # group 16, head_dim 256 (LDS above 64 KiB)
    (4, 4, 128, 1, 8, 2),          # one position
    (3, 1, 64, 65, 70, 0),         # group 3; last chunk holds one position
    (6, 2, 96, 100, 128, 0),       # head_dim 96: generic two-kernel path
    (16, 8, 128, 33, 64, 1),       # group 2; the chunk's second tile holds one position
    (8, 1, 128, 300, 512, 0),      # one kv head of eight q heads: many short chunks
    (32, 4, 128, 5000, 5000, 0),   # group 8 over four kv heads, chunks of several tiles
    (24, 8, 128, 257, 300, 2),     # group 3
])
def test_attention(dev, host, oracle, mem, nqh, nkh, hd, seq, max_ctx, layer):
    layers = layer + 1
    kvd = nkh * hd
    kc = V.synth_normal_f16(host, layers * max_ctx * kvd, SEED, 121)
    vc = V.synth_normal_f16(host, layers * max_ctx * kvd, SEED, 122)
    q = synth_x(host, nqh * hd, 123)
    scale = 1.0 / math.sqrt(hd)
    pq, pkc, pvc, po = mem.up(q), mem.up(kc), mem.up(vc), mem.zeros(nqh * hd)
    dev.attention(pq, pkc, pvc, po, seq, layer, max_ctx, nqh, nkh, hd, np.float32(scale))
    got = dev.download(po, nqh * hd, np.float32)
    want = oracle.attention(q, kc, vc, seq, layer, max_ctx, nqh, nkh, hd, np.float32(scale))
    assert np.all(np.abs(got - want) <= 1e-4 + 1e-4 * np.abs(want))


def _linear_draws(n=24, seed=SEED + 5):
    """Seeded shapes across the launch plans: every type, rows from 1 to
    12288, columns from one block to 16384 in the type's block size."""
    rng = np.random.default_rng(seed)
    block = {V.Q4_0: 32, V.Q4_1: 32, V.Q8_0: 32, V.Q4_K: 256, V.Q6_K: 256, V.F16: 32, V.F32: 32}
    out = []
    for i in range(n):
        t = TYPES[i % len(TYPES)]
        rows = int(rng.choice([1, 15, 16, 17, 100, 1000, 2049, 4096, 4097, 11008, 12288]))
        cols = int(block[t] * rng.integers(1, 16384 // block[t] + 1))
        out.append((t, rows, cols))
    return out


@pytest.mark.parametrize("t,rows,cols", _linear_draws(),
                         ids=[f"{V.TYPE_NAMES[t]}-{r}x{c}" for t, r, c in _linear_draws()])
def test_linear_random_shapes(dev, host, oracle, mem, t, rows, cols):
    """Seeded random shapes against the oracle under the matvec bar, so a
    plan chosen by shape (k_mvl, k_mvr, k_mvf and its tile counts, the
    32-element block kernels, the VALU fallbacks) is checked away from the
    shapes the other tests name."""
    w = V.synth_matrix(host, t, rows, cols, SEED, 31)
    x = synth_x(host, cols, 32)
    pw, px, py = mem.up(w), mem.up(x), mem.zeros(rows)
    dev.linear(t, pw, px, py, cols, rows)
    got = dev.download(py, rows, np.float32)
    want = oracle.linear(t, w, x, cols, rows)
    assert lin_err(got, want) <= LIN_TOL, (V.TYPE_NAMES[t], rows, cols)


def _attention_draws(n=12, seed=SEED + 6):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        nkh = int(rng.choice([1, 2, 4, 8]))
        group = int(rng.choice([1, 2, 3, 4, 8]))
        hd = int(rng.choice([32, 64, 96, 128]))
        seq = int(rng.integers(1, 3001))
        max_ctx = seq + int(rng.integers(0, 100))
        out.append((nkh * group, nkh, hd, seq, max_ctx, int(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("nqh,nkh,hd,seq,max_ctx,layer", _attention_draws())
def test_attention_random_shapes(dev, host, oracle, mem, nqh, nkh, hd, seq, max_ctx, layer):
    """Seeded random head counts, groups, head sizes (the matrix-core, VALU
    and generic chunk kernels), sequence lengths and layers against the
    oracle, at the attention tolerance."""
    kvd = nkh * hd
    kc = V.synth_normal_f16(host, (layer + 1) * max_ctx * kvd, SEED, 141)
    vc = V.synth_normal_f16(host, (layer + 1) * max_ctx * kvd, SEED, 142)
    q = synth_x(host, nqh * hd, 143)
    scale = np.float32(1.0 / math.sqrt(hd))
    pq, pkc, pvc, po = mem.up(q), mem.up(kc), mem.up(vc), mem.zeros(nqh * hd)
    dev.attention(pq, pkc, pvc, po, seq, layer, max_ctx, nqh, nkh, hd, scale)
    got = dev.download(po, nqh * hd, np.float32)
    want = oracle.attention(q, kc, vc, seq, layer, max_ctx, nqh, nkh, hd, scale)
    assert np.all(np.abs(got - want) <= 1e-4 + 1e-4 * np.abs(want))


@pytest.mark.parametrize("qscale", [1e-6, 1e4])
def test_attention_q_magnitude(dev, host, oracle, mem, qscale):
    """q far from unit scale (the matrix-core kernel rescales each head's q
    before splitting it into f16 halves); scores stay moderate by a matching
    softmax scale."""
    nqh, nkh, hd, seq, max_ctx = 32, 8, 128, 700, 768
    kvd = nkh * hd
    kc = V.synth_normal_f16(host, max_ctx * kvd, SEED, 131)
    vc = V.synth_normal_f16(host, max_ctx * kvd, SEED, 132)
    q = synth_x(host, nqh * hd, 133) * np.float32(qscale)
    scale = np.float32(1.0 / (math.sqrt(hd) * qscale))
    pq, pkc, pvc, po = mem.up(q), mem.up(kc), mem.up(vc), mem.zeros(nqh * hd)
    dev.attention(pq, pkc, pvc, po, seq, 0, max_ctx, nqh, nkh, hd, scale)
    got = dev.download(po, nqh * hd, np.float32)
    want = oracle.attention(q, kc, vc, seq, 0, max_ctx, nqh, nkh, hd, scale)
    assert np.all(np.abs(got - want) <= 1e-4 + 1e-4 * np.abs(want))


def test_rejections(dev, mem):
    """Unsupported types and malformed shapes fail with a reason, not a fault."""
    import ctypes
    p = mem.zeros(1024)
    assert dev._linear(V.Q8_K, p, p, p, 256, 1, 0, 0, 0) == 0
    assert "no gfx950 kernel" in dev.error()
    assert dev._linear(V.Q4_K, p, p, p, 100, 1, 0, 0, 0) == 0
    assert dev._attention(p, p, p, p, 4, 0, 2, 4, 2, 32, ctypes.c_float(1.0)) == 0
    assert dev._linear_supported(V.Q5_K) == 0
