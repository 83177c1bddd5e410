"""vbs_gfx950_attention_noalloc: the attention entry point that allocates
nothing (its partial results live in a fixed device array of the library).
It has no counterpart in the reference; it must give exactly what
vbs_gfx950_attention gives (same kernels), and both meet the attention bar
against the oracle of vbs_host_attention (src/vbs_host_math.h:170-209):
|got - want| <= 1e-4 + 1e-4 |want|.
"""
import ctypes
import math

import numpy as np
import pytest

import vbs_gfx950 as V
from test_gpu_kernels import SEED, Mem, mem, synth_x  # noqa: F401 (mem: fixture)

pytestmark = pytest.mark.gpu


def _case(host, mem, nqh, nkh, hd, seq, max_ctx, layer, stream):
    kvd = nkh * hd
    n = (layer + 1) * max_ctx * kvd
    kc = V.synth_normal_f16(host, n, SEED, stream)
    vc = V.synth_normal_f16(host, n, SEED, stream + 1)
    q = synth_x(host, nqh * hd, stream + 2)
    return q, kc, vc, [mem.up(q), mem.up(kc), mem.up(vc), mem.zeros(nqh * hd), mem.zeros(nqh * hd)]


def test_noalloc_matches_attention_twice(dev, host, oracle, mem):
    """Two calls in a row, the second smaller: a 70B-shaped layer at 8192
    positions (4.3 MB of partials), then a 7B-shaped one at 2049 positions;
    each equals the allocating entry point bit for bit and meets the bar."""
    for nqh, nkh, hd, seq, max_ctx, layer, st in ((64, 8, 128, 8192, 8192, 0, 150),
                                                  (32, 8, 128, 2049, 2176, 1, 160)):
        q, kc, vc, (pq, pkc, pvc, pa, pb) = _case(host, mem, nqh, nkh, hd, seq, max_ctx, layer, st)
        scale = ctypes.c_float(1.0 / math.sqrt(hd))
        dev.attention(pq, pkc, pvc, pa, seq, layer, max_ctx, nqh, nkh, hd, scale.value)
        assert dev._attention_noalloc(pq, pkc, pvc, pb, seq, layer, max_ctx, nqh, nkh, hd,
                                      scale) == 1, dev.error()
        a = dev.download(pa, nqh * hd, np.float32)
        b = dev.download(pb, nqh * hd, np.float32)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (nqh, seq)
        want = oracle.attention(q, kc, vc, seq, layer, max_ctx, nqh, nkh, hd, np.float32(scale.value))
        assert np.all(np.abs(b - want) <= 1e-4 + 1e-4 * np.abs(want)), (nqh, seq)


def test_noalloc_refuses_beyond_its_scratch(dev, mem):
    """Partials larger than the fixed array: refused with a reason, nothing
    launched, and the library keeps working."""
    p = mem.zeros(64 * 128)
    kv = mem.zeros(16384 * 8 * 128, np.uint16)  # sized for the shape, though nothing runs
    rc = dev._attention_noalloc(p, kv, kv, p, 16384, 0, 16384, 64, 8, 128, ctypes.c_float(0.1))
    assert rc == 0 and "exceed" in dev.error(), dev.error()
