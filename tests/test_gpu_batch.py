"""Batched (skinny) K-quant matvec on the gfx950 f16 matrix cores vs the oracle.

The reference has no batched matvec (its decode loops tokens one by one,
src/vbs_specializer.c:353-357), so the oracle of vbs_gfx950_linear_batch is
`batch` independent vbs_host_linear_tile calls (src/vbs_host_math.h:223-267):
every vector must meet the single matvec's bar, relative L2 <= 1e-5.
"""
import ctypes

import numpy as np
import pytest

import vbs_gfx950 as V
from test_gpu_kernels import LIN_TOL, SEED, Mem, lin_err, mem, rel_l2, synth_x  # noqa: F401 (mem: fixture)

pytestmark = pytest.mark.gpu

KQ = [V.Q4_K, V.Q6_K]


def run_batch(dev, mem, t, w, X, rows, cols, xs=None, ys=None):
    """Y = W X^T through the C ABI; X rows padded to stride xs, Y rows at
    stride ys pre-filled with -3 (so untouched entries are visible)."""
    batch = X.shape[0]
    xs, ys = xs or cols, ys or rows
    Xp = np.zeros((batch, xs), np.float32)
    Xp[:, :cols] = X
    pw, px = mem.up(w), mem.up(Xp)
    py = mem.up(np.full(batch * ys, -3.0, np.float32))
    dev.linear_batch(t, pw, px, xs, py, ys, cols, rows, batch)
    return dev.download(py, (batch, ys), np.float32)


def vectors(host, batch, cols, stream):
    return np.stack([synth_x(host, cols, stream + b) for b in range(batch)])


@pytest.mark.parametrize("t", KQ, ids=lambda t: V.TYPE_NAMES[t])
@pytest.mark.parametrize("batch", [1, 2, 5, 8, 11, 16])
@pytest.mark.parametrize("rows,cols", [(1, 256), (37, 4352), (700, 8192), (19, 11008),
                                       (96, 28672), (1030, 4096)])
def test_batch_parity(dev, host, oracle, mem, t, batch, rows, cols):
    """Row counts that leave tiles, waves and workgroups partly idle, one to
    eight blocks per wave, one and two launches of eight vectors."""
    w = V.synth_matrix(host, t, rows, cols, SEED, 71)
    X = vectors(host, batch, cols, 80)
    Y = run_batch(dev, mem, t, w, X, rows, cols)
    for b in range(batch):
        assert lin_err(Y[b], oracle.linear(t, w, X[b], cols, rows)) <= LIN_TOL, b


@pytest.mark.parametrize("t", KQ, ids=lambda t: V.TYPE_NAMES[t])
def test_batch_strides(dev, host, oracle, mem, t):
    """x and y strides wider than the row; entries past `rows` untouched."""
    rows, cols, batch = 300, 4096, 6
    w = V.synth_matrix(host, t, rows, cols, SEED, 72)
    X = vectors(host, batch, cols, 90)
    Y = run_batch(dev, mem, t, w, X, rows, cols, xs=cols + 40, ys=rows + 13)
    assert np.all(Y[:, rows:] == -3.0)
    for b in range(batch):
        assert lin_err(Y[b, :rows], oracle.linear(t, w, X[b], cols, rows)) <= LIN_TOL


@pytest.mark.parametrize("t", KQ, ids=lambda t: V.TYPE_NAMES[t])
def test_batch_activation_edge_cases(dev, host, oracle, mem, t):
    """Per-vector scaling: an all-zero vector, a vector of 1e-30 scale, one of
    1e30 scale, outliers, zero and subnormal-scale sub-blocks; every vector
    meets the bar on its own."""
    rows, cols = 128, 4096
    w = V.synth_matrix(host, t, rows, cols, SEED, 73)
    X = vectors(host, 8, cols, 100)
    X[0] = 0.0
    X[1] *= 1e-30
    X[2] *= 1e30
    X[3, 40] = 1.0e4
    X[4, 0:32] = 0.0
    X[4, 64:96] *= 1e-40
    X[5, 96:128] *= 1e30
    X[6, 7] = -0.0
    Y = run_batch(dev, mem, t, w, X, rows, cols)
    assert np.all(Y[0] == 0.0)
    for b in range(1, 8):
        want = oracle.linear(t, w, X[b], cols, rows)
        assert np.all(np.isfinite(Y[b])), b
        assert lin_err(Y[b], want) <= LIN_TOL, b


@pytest.mark.parametrize("t", KQ, ids=lambda t: V.TYPE_NAMES[t])
def test_batch_non_finite_vector(dev, host, oracle, mem, t):
    """A vector holding inf or NaN gives NaN rows (as the batch-1 matrix-core
    kernel does for such a sub-block); the other vectors are unaffected."""
    rows, cols = 64, 4096
    w = V.synth_matrix(host, t, rows, cols, SEED, 74)
    X = vectors(host, 4, cols, 110)
    X[1, 300] = np.inf
    X[2, 5] = np.nan
    Y = run_batch(dev, mem, t, w, X, rows, cols)
    assert np.all(np.isnan(Y[1])) and np.all(np.isnan(Y[2]))
    for b in (0, 3):
        assert lin_err(Y[b], oracle.linear(t, w, X[b], cols, rows)) <= LIN_TOL


@pytest.mark.parametrize("t,rows,cols", [(V.Q4_K, 28672, 8192), (V.Q6_K, 8192, 28672),
                                         (V.Q6_K, 32000, 8192)],
                         ids=["q4k_70b_gate", "q6k_70b_down", "q6k_70b_head"])
def test_batch_70b_shapes(dev, host, oracle, mem, t, rows, cols):
    """The Llama-70B layer shapes at batch 8, the oracle on the first and last
    192 rows (the packed rows are sliced out of the full matrix)."""
    w = V.synth_matrix(host, t, rows, cols, SEED, 75)
    X = vectors(host, 8, cols, 120)
    Y = run_batch(dev, mem, t, w, X, rows, cols)
    k = 192
    for lo in (0, rows - k):
        ws = np.ascontiguousarray(w[lo:lo + k])
        for b in range(8):
            assert lin_err(Y[b, lo:lo + k], oracle.linear(t, ws, X[b], cols, k)) <= LIN_TOL, (lo, b)


@pytest.mark.parametrize("rows,cols", [(4096, 11008), (3000, 8448), (4100, 28672), (5000, 25088)])
@pytest.mark.parametrize("batch", [3, 8, 11])
def test_batch_q6k_ring_shapes(dev, host, oracle, mem, rows, cols, batch):
    """Q6_K rows of 33-48 blocks over 2049-4096 rows and of 97-112 blocks
    over 4097-8192 rows take the batched LDS-DMA ring kernel: whole and short
    row ranges per workgroup, 33-112 blocks, one and two launches of eight
    vectors; every row of every vector against the oracle."""
    w = V.synth_matrix(host, V.Q6_K, rows, cols, SEED, 77)
    X = vectors(host, batch, cols, 130)
    Y = run_batch(dev, mem, V.Q6_K, w, X, rows, cols)
    for b in range(batch):
        assert lin_err(Y[b], oracle.linear(V.Q6_K, w, X[b], cols, rows, threads=16)) <= LIN_TOL, b


@pytest.mark.parametrize("rows", [11008, 22016])
@pytest.mark.parametrize("batch", [5, 8])
def test_batch_7b_gate_shape(dev, host, oracle, mem, batch, rows):
    """Q4_K 11008x4096 and 22016x4096 (the Llama-7B gate, and gate/up as one
    launch): 688 and 1376 tiles of 16-block rows, three tiles per workgroup
    (the last workgroup partly idle), every row against the oracle."""
    cols = 4096
    w = V.synth_matrix(host, V.Q4_K, rows, cols, SEED, 77)
    X = vectors(host, batch, cols, 130)
    Y = run_batch(dev, mem, V.Q4_K, w, X, rows, cols)
    for b in range(batch):
        assert lin_err(Y[b], oracle.linear(V.Q4_K, w, X[b], cols, rows)) <= LIN_TOL, b


def test_batch_ranged_qkv_every_row(dev, host, oracle, mem):
    """The 70B Q/K/V shape at batch 5 takes the ranged plan (an even range of
    42 rows of one matrix per workgroup, 246 workgroups, the last range of
    each matrix shorter): every row of every matrix against the oracle, per
    vector, and entries past each matrix's rows untouched."""
    shapes, cols, batch, pad = [8192, 1024, 1024], 8192, 5, 7
    ws = [V.synth_matrix(host, V.Q4_K, r, cols, SEED, 160 + m) for m, r in enumerate(shapes)]
    X = vectors(host, batch, cols, 170)
    px = mem.up(X)
    pws = [mem.up(w) for w in ws]
    pys = [mem.up(np.full(batch * (r + pad), -3.0, np.float32)) for r in shapes]
    dev.linear_batch_multi(V.Q4_K, pws, shapes, px, cols, pys, [r + pad for r in shapes], cols, batch)
    for m, (w, r) in enumerate(zip(ws, shapes)):
        Y = dev.download(pys[m], (batch, r + pad), np.float32)
        assert np.all(Y[:, r:] == -3.0), m
        for b in range(batch):
            want = oracle.linear(V.Q4_K, w, X[b], cols, r, threads=16)
            assert lin_err(Y[b, :r], want) <= LIN_TOL, (m, b)
            # a row of a wrong range would stand out even inside the L2 norm
            assert np.max(np.abs(Y[b, :r] - want)) <= 1e-4 * (np.max(np.abs(want)) + 1.0), (m, b)


@pytest.mark.parametrize("t,shapes,cols", [
    (V.Q4_K, [8192, 1024, 1024], 8192), (V.Q4_K, [4096, 1024, 1024], 4096),
    (V.Q4_K, [28672, 28672], 8192), (V.Q6_K, [4096, 1000, 13], 4096), (V.Q4_K, [37], 512)],
    ids=["q4k_70b_qkv", "q4k_7b_qkv", "q4k_70b_gate_up", "q6k_ragged", "q4k_one"])
@pytest.mark.parametrize("batch", [5, 8, 11])
def test_batch_multi_matrix_launch(dev, host, oracle, mem, t, shapes, cols, batch):
    """vbs_gfx950_linear_batch_multi: Q/K/V (or gate/up) of one layer over the
    same vectors in one launch. Workgroups of several tiles span the
    boundaries between the matrices (70B Q/K/V: 640 tiles, three per
    workgroup, the last one partly idle). The first and last 64 rows of every
    matrix (so the rows on both sides of each boundary, and the last
    workgroup's) against the oracle, per vector; entries past each matrix's
    rows untouched."""
    ws = [V.synth_matrix(host, t, r, cols, SEED, 140 + m) for m, r in enumerate(shapes)]
    X = vectors(host, batch, cols, 150)
    px = mem.up(X)
    pad = 7
    pws = [mem.up(w) for w in ws]
    pys = [mem.up(np.full(batch * (r + pad), -3.0, np.float32)) for r in shapes]
    dev.linear_batch_multi(t, pws, shapes, px, cols, pys, [r + pad for r in shapes], cols, batch)
    for m, (w, r) in enumerate(zip(ws, shapes)):
        Y = dev.download(pys[m], (batch, r + pad), np.float32)
        assert np.all(Y[:, r:] == -3.0), m
        spans = sorted({(0, min(64, r)), (max(0, r - 64), r)})
        for lo, hi in spans:
            wsl = np.ascontiguousarray(w[lo:hi])
            for b in range(batch):
                want = oracle.linear(t, wsl, X[b], cols, hi - lo)
                assert lin_err(Y[b, lo:hi], want) <= LIN_TOL, (m, lo, b)


def test_scratch_growth_keeps_captured_graphs(dev, host, oracle, mem):
    """The batched matvec keeps its prepared x in the library's scratch. A
    graph captured from the library's stream holds the scratch address of the
    capture, so a later call that grows the scratch (a long attention: its
    per-chunk partials live there too) must leave that memory valid: every
    replay still meets the oracle. A call under capture that would need more
    scratch fails with a reason and launches nothing (growing allocates)."""
    hip, stream = V.Hip(), dev.stream()
    t, rows, cols, batch = V.Q4_K, 96, 4096, 4
    w = V.synth_matrix(host, t, rows, cols, SEED, 78)
    X = vectors(host, batch, cols, 140)
    pw, px, py = mem.up(w), mem.up(X), mem.zeros(batch * rows)
    want = [oracle.linear(t, w, X[b], cols, rows) for b in range(batch)]
    nqh, nkh, hd = 8, 1, 128
    pq, po = mem.up(synth_x(host, nqh * hd, 141)), mem.zeros(nqh * hd)

    # zero keys and values for the long attentions below, allocated before any capture
    caches = {seq: (mem.zeros(seq * hd, np.uint16), mem.zeros(seq * hd, np.uint16))
              for seq in (520_000, 1_100_000)}

    def attention(seq):
        """Attention over `seq` zero keys and values: per-chunk partials of
        8 x seq/64 x 130 floats (32 MiB at 520,000 positions)."""
        kc, vc = caches[seq]
        return dev._attention(pq, kc, vc, po, seq, 0, seq, nqh, nkh, hd, ctypes.c_float(0.088))

    dev.linear_batch(t, pw, px, cols, py, rows, cols, rows, batch)  # sizes the scratch
    graph = hip.capture(stream, lambda: dev.linear_batch(t, pw, px, cols, py, rows, cols, rows,
                                                         batch))
    try:
        for rep in range(3):
            dev.write(py, np.zeros(batch * rows, np.float32))
            if rep == 1:  # grows the scratch well past anything the other tests use
                assert attention(520_000) == 1, dev.error()
                assert np.all(dev.download(po, nqh * hd, np.float32) == 0.0)
            hip.launch(graph, stream)
            Y = dev.download(py, (batch, rows), np.float32)
            for b in range(batch):
                assert lin_err(Y[b], want[b]) <= LIN_TOL, (rep, b)
    finally:
        hip.destroy(graph)
    rc = []
    failed = hip.capture(stream, lambda: rc.append(attention(1_100_000)))
    hip.destroy(failed)
    assert rc == [0] and "capturing" in dev.error(), dev.error()
    # the stream works on after the refused call
    dev.linear_batch(t, pw, px, cols, py, rows, cols, rows, batch)
    Y = dev.download(py, (batch, rows), np.float32)
    assert lin_err(Y[0], want[0]) <= LIN_TOL
