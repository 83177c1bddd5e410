"""CPU side of the hot-kernel table adapter (the reference's vbs_hotpath.h ABI v1).

Pins the oracle's restatement of the table (src/hotkernels/vbs_hot_ref_impl.h:
49-129) and of the CPU model's activation quantiser (src/vbs_cpu.c:74-93,
166-182):

* the table against the reference's own built-in kernels, compiled from
  src/vbs_hotpath.c into oracle/_ref (bit for bit, every type);
* the table on unit-scale blocks, where y is an exact integer dot;
* the round-to-nearest-even f16 conversion against numpy's IEEE
  float32 -> float16 conversion (every exponent, random and boundary
  significands), and its non-finite rule (NaN and inf -> inf);
* the quantiser against an independent numpy formulation (IEEE f32 division
  and products, half-away-from-zero rounding done in float64, numpy's f16),
  with ties, all-zero, subnormal-scale and overflowing-scale blocks.

Also that lib/libvbs_hot_gfx950.so passes the reference's own module loader
(vbs_hot_load, src/vbs_hotpath.c:78-109) and reports a failed call as NaN
rows plus a reason, without touching a GPU.
"""
import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

import vbs_gfx950 as V
from oracle_lib import REF_HOT_SO, Oracle, reference_hot

HOT_TYPES = [V.Q8_0, V.Q4_0, V.Q4_1, V.F32, V.F16]


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def hot_inputs(host, t, rows, cols, seed):
    """Packed weights of type t plus activations as the CPU model forms them."""
    w = V.synth_matrix(host, t, rows, cols, seed, 1)
    x = V.synth_normal(host, cols, seed, 2)
    return w, x


def np_f16_rne(v):
    with np.errstate(over="ignore"):
        return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def np_quantize_q8(x):
    """Independent numpy form of src/vbs_cpu.c:166-182."""
    xb = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(xb).max(axis=1).astype(np.float32)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (xb * inv[:, None]).astype(np.float32).astype(np.float64)
    q = np.sign(v) * np.floor(np.abs(v) + 0.5)
    q = np.clip(q, -127, 127).astype(np.int64)
    qd = np_f16_rne(d).view(np.float16).astype(np.float32)
    s = (q.sum(axis=1).astype(np.float32) * d).astype(np.float32)
    qs = np_f16_rne(s).view(np.float16).astype(np.float32)
    return q.astype(np.int8).ravel(), qd, qs


def test_f16_rne_matches_ieee_conversion(orc):
    rng = np.random.default_rng(5)
    exps = np.arange(0, 255, dtype=np.uint32)
    mant = rng.integers(0, 1 << 23, size=(exps.size, 64), dtype=np.uint32)
    edge = np.array([0, 1, 0xFFF, 0x1000, 0x1001, 0x2000, 0x3000, 0x7FFFFF, 0x7FE000, 0x7FF000,
                     0x400000, 0x401000, 0x7FFFFF - 0xFFF], np.uint32)
    mant = np.concatenate([mant, np.broadcast_to(edge, (exps.size, edge.size))], axis=1)
    bits = (exps[:, None] << 23) | mant
    bits = np.concatenate([bits.ravel(), bits.ravel() | 0x80000000])
    f = bits.view(np.float32)
    got = np.array([orc._f32_to_f16_rne(float(v)) for v in f], np.uint16)
    want = np_f16_rne(f)
    assert np.array_equal(got, want)
    for v, h in [(np.inf, 0x7C00), (-np.inf, 0xFC00), (np.nan, 0x7C00), (65519.0, 0x7BFF),
                 (65520.0, 0x7C00), (2.0 ** -25, 0), (2.0 ** -25 * 1.5, 1), (2.0 ** -24, 1)]:
        assert orc._f32_to_f16_rne(float(v)) == h, v


def test_quantize_q8_matches_independent_form(host, orc):
    x = V.synth_normal(host, 32 * 64, 9, 3).copy()
    blocks = x.reshape(-1, 32)
    blocks[1] = 0.0                                      # d == 0: all zero
    blocks[2] = np.arange(32, dtype=np.float32) - 15.5   # amax 16.5
    blocks[3] = 0.0
    blocks[3][[0, 5, 9]] = [127.0, 2.5, -0.5]            # d == 1: exact ties
    blocks[4] *= np.float32(1e-7)                        # subnormal f16 scale
    blocks[5] *= np.float32(1e-9)                        # scale flushes to zero
    blocks[6] *= np.float32(1e8)                         # f16 scale overflows to inf
    blocks[7] = np.float32(-3.0)                         # constant block
    xq, qd, qs = orc.quantize_q8(x)
    wq, wd, ws = np_quantize_q8(x)
    assert np.array_equal(xq, wq)
    assert np.array_equal(qd.view(np.uint32), wd.view(np.uint32))
    assert np.array_equal(qs.view(np.uint32), ws.view(np.uint32))
    assert xq[3 * 32 + 5] == 3 and xq[3 * 32 + 9] == -1   # half away from zero
    assert np.all(xq[32:64] == 0) and qd[1] == 0 and qs[1] == 0
    assert np.isinf(qd[6])


def test_hot_matvec_unit_scales_give_integer_dots(orc):
    rng = np.random.default_rng(3)
    rows, cols = 5, 96
    nb = cols // 32
    xq = rng.integers(-127, 128, cols).astype(np.int8)
    qd = np.ones(nb, np.float32)
    # Q8_0 with d = 1.0
    q8 = rng.integers(-128, 128, (rows, nb, 32)).astype(np.int8)
    blk = np.zeros((rows, nb, 34), np.uint8)
    blk[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[:, :, 2:] = q8.view(np.uint8)
    y = orc.hot_matvec(V.Q8_0, blk, rows, cols, xq, qd)
    want = (q8.reshape(rows, cols).astype(np.int64) * xq.astype(np.int64)).sum(axis=1)
    assert np.array_equal(y, want.astype(np.float32))
    # Q4_0 with d = 1.0: (nib - 8) * x, low nibbles are elements 0..15
    nib = rng.integers(0, 16, (rows, nb, 32)).astype(np.uint8)
    b4 = np.zeros((rows, nb, 18), np.uint8)
    b4[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    b4[:, :, 2:] = nib[:, :, :16] | (nib[:, :, 16:] << 4)
    y = orc.hot_matvec(V.Q4_0, b4, rows, cols, xq, qd)
    want = ((nib.reshape(rows, cols).astype(np.int64) - 8) * xq.astype(np.int64)).sum(axis=1)
    assert np.array_equal(y, want.astype(np.float32))
    # Q4_1 with d = 1, m = 0.5, qsum = 2: every block adds 1.0 after its dot
    b41 = np.zeros((rows, nb, 20), np.uint8)
    b41[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    b41[:, :, 2:4] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    b41[:, :, 4:] = nib[:, :, :16] | (nib[:, :, 16:] << 4)
    y = orc.hot_matvec(V.Q4_1, b41, rows, cols, xq, qd, np.full(nb, 2.0, np.float32))
    want = (nib.reshape(rows, cols).astype(np.int64) * xq.astype(np.int64)).sum(axis=1) + nb
    assert np.array_equal(y, want.astype(np.float32))


@pytest.mark.skipif(not os.path.exists(REF_HOT_SO), reason="oracle/_ref hot table not built")
@pytest.mark.parametrize("t", HOT_TYPES, ids=[V.TYPE_NAMES[t] for t in HOT_TYPES])
@pytest.mark.parametrize("rows,cols", [(48, 4096), (7, 11008), (3, 32)])
def test_oracle_hot_table_equals_reference_builtin(host, orc, t, rows, cols):
    ref = reference_hot()
    w, x = hot_inputs(host, t, rows, cols, 17 + t)
    xq, qd, qs = orc.quantize_q8(x)
    got = orc.hot_matvec(t, w, rows, cols, xq, qd, qs, x)
    want = np.empty(rows, np.float32)
    tb = ref.vbs_hot_builtin().contents
    if t == V.Q4_1:
        tb.matvec_q4_1(w.ctypes.data, rows, cols, xq.ctypes.data, qd.ctypes.data, qs.ctypes.data,
                       want.ctypes.data)
    elif t in (V.Q8_0, V.Q4_0):
        fn = tb.matvec_q8_0 if t == V.Q8_0 else tb.matvec_q4_0
        fn(w.ctypes.data, rows, cols, xq.ctypes.data, qd.ctypes.data, want.ctypes.data)
    else:
        fn = tb.matvec_f32 if t == V.F32 else tb.matvec_f16
        fn(w.ctypes.data, rows, cols, x.ctypes.data, want.ctypes.data)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_module_exports_the_v1_table():
    m = V.HotModule()
    assert m.abi_version() == 1
    tb = m.table
    assert tb.abi_version == 1 and tb.name == b"gfx950-hip"
    for f in ("matvec_q8_0", "matvec_q4_0", "matvec_q4_1", "matvec_f32", "matvec_f16"):
        assert getattr(tb, f)


@pytest.mark.skipif(not os.path.exists(REF_HOT_SO), reason="oracle/_ref hot table not built")
def test_reference_loader_accepts_the_module():
    ref = reference_hot()
    err = C.create_string_buffer(256)
    assert ref.vbs_hot_load(V.HOT_LIB.encode(), err, 256), err.value
    assert ref.vbs_hot_current_name() == b"gfx950-hip"
    assert ref.vbs_hot_current_path() == V.HOT_LIB.encode()
    assert ref.vbs_hot_has_rollback()
    assert ref.vbs_hot_rollback(err, 256)
    assert ref.vbs_hot_current_name() == b"builtin-ref"


def test_failed_call_gives_nan_rows_and_a_reason(tmp_path):
    """No device library: every row NaN, the reason kept (run in a child so
    the module's one-shot probe does not stick to this process)."""
    code = (
        "import sys, numpy as np; sys.path.insert(0, %r); import vbs_gfx950 as V\n"
        "m = V.HotModule()\n"
        "y = m.matvec(V.F32, np.ones((3, 64), np.float32), 3, 64, x=np.ones(64, np.float32))\n"
        "assert np.all(np.isnan(y)), y\n"
        "assert 'not found' in m.last_error(), m.last_error()\n"
        "print('ok')\n" % os.path.dirname(V.__file__))
    env = dict(os.environ, VBS_GFX950_LIB=str(tmp_path / "absent.so"))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr


def test_module_exports_every_declared_symbol():
    import re
    hdr = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                            "include", "vbs_hot_abi.h")).read()
    declared = sorted(set(re.findall(r"\b(vbs_hot_\w+)\s*\(", hdr)))
    assert declared == ["vbs_hot_abi_version", "vbs_hot_gfx950_last_error", "vbs_hot_kernels"]
    lib = C.CDLL(V.HOT_LIB)
    for name in declared:
        assert hasattr(lib, name), name


@pytest.mark.skipif(not os.path.isdir("/root/reference/include"),
                    reason="reference headers not mounted")
def test_table_layout_matches_reference_header(tmp_path):
    """sizeof/offsetof of vbs_hot_kernels_t and the ABI version agree between
    include/vbs_hot_abi.h and the reference's include/vbs_hotpath.h."""
    probe = r'''
#include <stdio.h>
#include <stddef.h>
#include HDR
int main(void) {
  printf("%d %zu %zu %zu %zu %zu\n", VBS_HOT_ABI_VERSION, sizeof(vbs_hot_kernels_t),
         offsetof(vbs_hot_kernels_t, name), offsetof(vbs_hot_kernels_t, matvec_q8_0),
         offsetof(vbs_hot_kernels_t, matvec_q4_1), offsetof(vbs_hot_kernels_t, matvec_f16));
  return 0;
}
'''
    src = tmp_path / "probe.c"
    src.write_text(probe)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    outs = []
    for hdr, inc in (('"vbs_hot_abi.h"', os.path.join(root, "include")),
                     ('"vbs_hotpath.h"', "/root/reference/include")):
        exe = tmp_path / f"probe{len(outs)}"
        subprocess.run(["gcc", "-std=c11", f"-DHDR={hdr}", "-I" + inc, str(src), "-o", str(exe)],
                       check=True)
        outs.append(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout)
    assert outs[0] == outs[1]
