"""GPU parity of the hot-kernel table adapter: vbs_gfx950_quantize_q8 and
vbs_gfx950_hot_matvec against the oracle (src/vbs_cpu.c:166-182,
src/hotkernels/vbs_hot_ref_impl.h:49-129), bit for bit, and the host-pointer
module lib/libvbs_hot_gfx950.so against the reference's own built-in table,
also when reached through the reference's loader and timed dispatch wrappers
(src/vbs_hotpath.c:78-109, 153-177).
"""
import ctypes as C
import os

import numpy as np
import pytest

import vbs_gfx950 as V
from oracle_lib import (REF_CPU_SO, REF_HOT_SO, Oracle, cpu_model_logits, reference_cpu_model,
                        reference_hot)

pytestmark = pytest.mark.gpu

HOT_TYPES = [V.Q8_0, V.Q4_0, V.Q4_1, V.F32, V.F16]
IDS = [V.TYPE_NAMES[t] for t in HOT_TYPES]


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def edge_activations(host, cols, seed):
    x = V.synth_normal(host, cols, seed, 2).copy()
    b = x.reshape(-1, 32)
    n = b.shape[0]
    if n > 8:
        b[1] = 0.0
        b[3] = 0.0
        b[3][[0, 5, 9]] = [127.0, 2.5, -0.5]
        b[4] *= np.float32(1e-7)
        b[5] *= np.float32(1e-9)
        b[7] = np.float32(-3.0)
    return x


def dev_quantize(dev, x):
    cols = x.size
    nb = cols // 32
    px = dev.upload(x)
    pq, pd, ps = dev.alloc(max(cols, 4)), dev.alloc(max(nb * 4, 4)), dev.alloc(max(nb * 4, 4))
    try:
        dev.quantize_q8(px, cols, pq, pd, ps)
        return (dev.download(pq, cols, np.int8), dev.download(pd, nb, np.float32),
                dev.download(ps, nb, np.float32))
    finally:
        for p in (px, pq, pd, ps):
            dev.free(p)


@pytest.mark.parametrize("cols", [32, 4096, 11008, 28672])
def test_quantize_q8_bit_exact(dev, host, orc, cols):
    x = edge_activations(host, cols, 40 + cols % 97)
    got = dev_quantize(dev, x)
    want = orc.quantize_q8(x)
    assert np.array_equal(got[0], want[0])
    assert same_bits(got[1], want[1]) and same_bits(got[2], want[2])


def test_quantize_q8_rejects_ragged_cols(dev):
    p = dev.alloc(4096)
    try:
        with pytest.raises(V.GpuError, match="multiple of 32"):
            dev.quantize_q8(p, 40, p, p, p)
    finally:
        dev.free(p)


def dev_hot(dev, t, w, rows, cols, xq, qd, qs, x):
    pw = dev.upload(w)
    act = dev.upload(xq if t in (V.Q8_0, V.Q4_0, V.Q4_1) else x)
    pd = dev.upload(qd) if qd is not None and qd.size else 0
    ps = dev.upload(qs) if qs is not None and qs.size else 0
    py = dev.alloc(max(rows * 4, 4))
    try:
        dev.hot_matvec(t, pw, rows, cols, act, pd, ps, py)
        return dev.download(py, rows, np.float32)
    finally:
        for p in (pw, act, pd, ps, py):
            if p:
                dev.free(p)


@pytest.mark.parametrize("t", HOT_TYPES, ids=IDS)
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (33, 11008), (5, 28672), (7, 32), (3, 96)])
def test_hot_matvec_bit_exact(dev, host, orc, t, rows, cols):
    w = V.synth_matrix(host, t, rows, cols, 60 + t, 1)
    x = edge_activations(host, cols, 61 + t)
    xq, qd, qs = orc.quantize_q8(x)
    got = dev_hot(dev, t, w, rows, cols, xq, qd, qs, x)
    want = orc.hot_matvec(t, w, rows, cols, xq, qd, qs, x)
    assert same_bits(got, want), (t, rows, cols, np.flatnonzero(got != want)[:5])


@pytest.mark.parametrize("t", [V.F32, V.F16], ids=["F32", "F16"])
def test_hot_matvec_ragged_float_rows(dev, host, orc, t):
    rows, cols = 9, 1000  # F32 / F16 rows need not be whole blocks
    w = V.synth_matrix(host, t, rows, cols, 70, 1)
    x = V.synth_normal(host, cols, 71, 2)
    got = dev_hot(dev, t, w, rows, cols, None, None, None, x)
    assert same_bits(got, orc.hot_matvec(t, w, rows, cols, x=x))


def test_hot_matvec_refuses_types_outside_the_table(dev):
    p = dev.alloc(4096)
    try:
        with pytest.raises(V.GpuError, match="not in the hot-kernel table"):
            dev.hot_matvec(V.Q4_K, p, 1, 256, p, p, p, p)
    finally:
        dev.free(p)


@pytest.fixture(scope="module")
def hot_module(dev):
    return V.HotModule()


@pytest.mark.parametrize("t", HOT_TYPES, ids=IDS)
def test_module_equals_reference_builtin(dev, host, orc, hot_module, t):
    rows, cols = 300, 4096
    w = V.synth_matrix(host, t, rows, cols, 80 + t, 1)
    x = V.synth_normal(host, cols, 81 + t, 2)
    xq, qd, qs = orc.quantize_q8(x)
    got = hot_module.matvec(t, w, rows, cols, xq=xq, qd=qd, qsum=qs, x=x)
    assert hot_module.last_error() == "ok"
    assert same_bits(got, orc.hot_matvec(t, w, rows, cols, xq, qd, qs, x))
    ref = reference_hot()
    if ref is not None:
        tb = ref.vbs_hot_builtin().contents
        want = np.empty(rows, np.float32)
        if t == V.Q4_1:
            tb.matvec_q4_1(w.ctypes.data, rows, cols, xq.ctypes.data, qd.ctypes.data,
                           qs.ctypes.data, want.ctypes.data)
        elif t in (V.Q8_0, V.Q4_0):
            fn = tb.matvec_q8_0 if t == V.Q8_0 else tb.matvec_q4_0
            fn(w.ctypes.data, rows, cols, xq.ctypes.data, qd.ctypes.data, want.ctypes.data)
        else:
            fn = tb.matvec_f32 if t == V.F32 else tb.matvec_f16
            fn(w.ctypes.data, rows, cols, x.ctypes.data, want.ctypes.data)
        assert same_bits(got, want)


def test_module_ragged_quant_cols_ignore_the_tail(dev, host, orc, hot_module):
    """cols = 100: the reference reads cols/32 = 3 blocks and ignores the tail."""
    rows, cols = 4, 100
    w = V.synth_matrix(host, V.Q8_0, rows, 96, 90, 1)
    x = V.synth_normal(host, 128, 91, 2)
    xq, qd, qs = orc.quantize_q8(x)
    got = hot_module.matvec(V.Q8_0, w, rows, cols, xq=xq, qd=qd)
    assert same_bits(got, orc.hot_matvec(V.Q8_0, w, rows, 96, xq, qd))


@pytest.mark.skipif(not os.path.exists(REF_HOT_SO), reason="oracle/_ref hot table not built")
def test_through_the_reference_loader_and_wrappers(dev, host, orc):
    """vbs_hot_load(module) then the reference's own timed dispatch wrappers
    (what vbs_cpu.c calls) give the built-in table's bits."""
    ref = reference_hot()
    err = C.create_string_buffer(256)
    assert ref.vbs_hot_load(V.HOT_LIB.encode(), err, 256), err.value
    try:
        assert ref.vbs_hot_current_name() == b"gfx950-hip"
        rows, cols = 512, 11008
        for t in (V.Q8_0, V.Q4_0, V.Q4_1):
            w = V.synth_matrix(host, t, rows, cols, 95 + t, 1)
            x = V.synth_normal(host, cols, 96 + t, 2)
            xq, qd, qs = orc.quantize_q8(x)
            got = np.empty(rows, np.float32)
            want = np.empty(rows, np.float32)
            tb = ref.vbs_hot_builtin().contents
            if t == V.Q4_1:
                ref.vbs_hot_matvec_q4_1(w.ctypes.data, rows, cols, xq.ctypes.data, qd.ctypes.data,
                                        qs.ctypes.data, got.ctypes.data)
                tb.matvec_q4_1(w.ctypes.data, rows, cols, xq.ctypes.data, qd.ctypes.data,
                               qs.ctypes.data, want.ctypes.data)
            else:
                name = "q8_0" if t == V.Q8_0 else "q4_0"
                getattr(ref, "vbs_hot_matvec_" + name)(w.ctypes.data, rows, cols, xq.ctypes.data,
                                                       qd.ctypes.data, got.ctypes.data)
                getattr(tb, "matvec_" + name)(w.ctypes.data, rows, cols, xq.ctypes.data,
                                              qd.ctypes.data, want.ctypes.data)
            assert same_bits(got, want), V.TYPE_NAMES[t]
    finally:
        assert ref.vbs_hot_rollback(err, 256), err.value


@pytest.mark.skipif(not os.path.exists(REF_CPU_SO), reason="oracle/_ref CPU model not built")
@pytest.mark.parametrize("mix", [None, {"q": V.Q8_0, "k": V.Q4_0, "v": V.Q4_1, "o": V.F16,
                                        "gate": V.Q4_0, "up": V.Q8_0, "down": V.Q4_1,
                                        "embd": V.Q8_0, "head": V.F32}],
                         ids=["q4_k_m", "every_table_type"])
def test_reference_cpu_model_on_the_module(dev, host, tmp_path, mix):
    """The reference's own CPU model (src/vbs_cpu.c) with its hot table
    swapped for lib/libvbs_hot_gfx950.so by its own loader: every step's
    logits equal the built-in table's bit for bit."""
    model = V.SynthModel(host, n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2,
                         head_dim=64, vocab=512, max_ctx=64, seed=33, mix=mix)
    path = tmp_path / "tiny.gguf"
    V.write_gguf(host, str(path), model, context_length=2176)
    lib = reference_cpu_model()
    tokens = [1, 17, 300, 5, 42, 7]
    want = cpu_model_logits(lib, path, tokens)
    err = C.create_string_buffer(256)
    assert lib.vbs_hot_load(V.HOT_LIB.encode(), err, 256), err.value
    try:
        assert lib.vbs_hot_current_name() == b"gfx950-hip"
        got = cpu_model_logits(lib, path, tokens)
    finally:
        assert lib.vbs_hot_rollback(err, 256), err.value
    for step, (a, b) in enumerate(zip(got, want)):
        assert same_bits(a, b), step


def test_module_accepts_host_arrays_at_odd_addresses(dev, host, orc, hot_module):
    """The table passes host pointers with no alignment promise (blocks are
    2-byte fields at any address); the module stages them byte for byte."""
    rows, cols = 37, 4096
    w = V.synth_matrix(host, V.Q4_0, rows, cols, 97, 1)
    x = V.synth_normal(host, cols, 98, 2)
    xq, qd, _ = orc.quantize_q8(x)
    raw = np.empty(w.nbytes + 1, np.uint8)
    wo = raw[1:].reshape(w.shape)
    wo[...] = w
    xr = np.empty(cols + 3, np.int8)
    xo = xr[3:]
    xo[...] = xq
    got = hot_module.matvec(V.Q4_0, wo, rows, cols, xq=xo, qd=qd)
    assert same_bits(got, orc.hot_matvec(V.Q4_0, w, rows, cols, xq, qd))
