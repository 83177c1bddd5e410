"""The reference's special f16 cases on the device.

The reference converts halves exactly, subnormals and the payloads of Inf/NaN
included (vbs_f16_to_f32, src/vbs_dequant.c:21-44), and rounds floats to
halves with its own rules: round-to-nearest-even for normals, half-up for
subnormals, flush below 2^-25, overflow to +-inf, NaN to 0x7C01
(vbs_f32_to_f16, src/vbs_dequant.c:46-74). The oracle is pinned to both over
every input on the CPU (tests/test_oracle.py); these tests hold the device
decoders to the same inputs:

* every one of the 65,536 halves as an F16 row, through the batched gather
  and the one-token EMBEDDING op, against the SHA-256 of the reference's own
  table (tests/golden/half.json) and the oracle, bit for bit;
* the golden blocks of every block type (tests/golden/dequant_blocks.npz,
  made by the reference's dequantiser: synthetic, random-byte and edge blocks
  with subnormal, maximal, negative-zero-adjacent and NaN scales), through
  the gather, against the stored reference outputs bit for bit;
* the KV store on every float whose biased exponent lies in 101..143 (both
  signs): the whole span from below the flush threshold through the half
  subnormals and normals to overflow, against the oracle bit for bit.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import vbs_gfx950 as V
from test_gpu_kernels import Mem, mem  # noqa: F401 (mem: fixture)

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_f16_row_of_every_half(dev, oracle, mem):
    halves = np.arange(65536, dtype=np.uint16)
    want_sha = json.load(open(os.path.join(GOLDEN, "half.json")))["f16_to_f32_sha256"]
    pw, out, emb = mem.up(halves), mem.zeros(65536), mem.zeros(65536)
    dev.dequant_rows(V.F16, pw, 0, 1, 65536, out)
    dev.embed(V.F16, pw, 0, emb, 65536)
    want = oracle.dequant_row(V.F16, halves.view(np.uint8), 65536).view(np.uint32)
    for p in (out, emb):
        got = dev.download(p, 65536, np.uint32)
        assert hashlib.sha256(got.astype("<u4").tobytes()).hexdigest() == want_sha
        assert np.array_equal(got, want)


@pytest.mark.parametrize("t", [V.Q4_0, V.Q4_1, V.Q8_0, V.Q4_K, V.Q6_K],
                         ids=lambda t: V.TYPE_NAMES[t])
def test_golden_blocks_on_device(dev, mem, t):
    """Each golden block is one row of a matrix one block wide; the gather
    of all rows and single-token gathers of the edge blocks (the last rows)
    must reproduce the reference's stored output words."""
    g = np.load(os.path.join(GOLDEN, "dequant_blocks.npz"))
    blocks, want = g[f"t{t}_in"], g[f"t{t}_out"]
    n, e = want.shape
    pw, out = mem.up(np.ascontiguousarray(blocks)), mem.zeros(n * e)
    dev.dequant_rows(t, pw, 0, n, e, out)
    got = dev.download(out, (n, e), np.uint32)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"blocks {bad.tolist()} differ"
    one = mem.zeros(e)
    for r in range(n - 10, n):
        dev.embed(t, pw, r, one, e)
        assert np.array_equal(dev.download(one, e, np.uint32), want[r]), r


def test_kv_store_exponents_101_to_143(dev, oracle, mem):
    """k holds the 2^23 positive floats of one biased exponent and v the
    negative ones; one store per exponent from 101 (below 2^-25, flushed)
    through 112-113 (half subnormal to normal) to 143 (2^16, past the half
    maximum 65504)."""
    kvd = 1 << 23
    mant = np.arange(kvd, dtype=np.uint32)
    pk, pv = mem.zeros(kvd), mem.zeros(kvd)
    pkc, pvc = mem.zeros(kvd, np.uint16), mem.zeros(kvd, np.uint16)
    kc = np.zeros(kvd, np.uint16)
    vc = np.zeros(kvd, np.uint16)
    for ex in range(101, 144):
        k = (mant | np.uint32(ex << 23)).view(np.float32)
        v = (mant | np.uint32((ex << 23) | 0x80000000)).view(np.float32)
        dev.write(pk, k)
        dev.write(pv, v)
        dev.cache_store(pk, pv, pkc, pvc, 0, 0, 1, kvd)
        oracle.cache_store(k, v, kc, vc, 0, 0, 1, kvd)
        gk = dev.download(pkc, kvd, np.uint16)
        gv = dev.download(pvc, kvd, np.uint16)
        assert np.array_equal(gk, kc), (ex, int(np.nonzero(gk != kc)[0][0]))
        assert np.array_equal(gv, vc), (ex, int(np.nonzero(gv != vc)[0][0]))
