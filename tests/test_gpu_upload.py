"""Host -> device copies: large pageable sources go through the runtime's
pinned double-buffered staging (vbs_gfx950_copy_h2d), pinned sources straight
to the DMA engine; every byte must arrive, for sizes that are not multiples of
the staging chunk and for sources at odd addresses."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,offset", [(16 << 20, 0), ((100 << 20) + 12345, 3),
                                           ((64 << 20) + 1, 1), ((32 << 20) - 7, 0)])
def test_pageable_upload_round_trip(dev, nbytes, offset):
    rng = np.random.default_rng(nbytes % 1000)
    buf = rng.integers(0, 256, nbytes + offset, dtype=np.uint8)
    src = buf[offset:]
    p = dev.alloc(nbytes)
    try:
        dev.check(dev._copy_h2d(p, src.ctypes.data, nbytes), "copy_h2d")
        back = dev.download(p, nbytes, np.uint8)
        assert np.array_equal(back, src)
        # a second upload into the same buffer (the staging buffers are reused)
        src2 = src[::-1].copy()
        dev.write(p, src2)
        assert np.array_equal(dev.download(p, nbytes, np.uint8), src2)
    finally:
        dev.free(p)


def test_pinned_upload_round_trip(dev):
    n = (48 << 20) + 5
    h = dev._host_alloc(n)
    assert h
    p = dev.alloc(n)
    try:
        src = np.random.default_rng(7).integers(0, 256, n, dtype=np.uint8)
        C.memmove(h, src.ctypes.data, n)
        dev.check(dev._copy_h2d(p, h, n), "copy_h2d")
        assert np.array_equal(dev.download(p, n, np.uint8), src)
    finally:
        dev.free(p)
        dev._host_free(h)


def test_upload_is_ordered_after_earlier_kernels(dev, host):
    """A staged upload into a buffer a queued kernel still reads must wait
    for it: y = W x, then overwrite x with a large upload, then read y."""
    import vbs_gfx950 as V
    rows, cols = 4096, 4096
    w = V.synth_matrix(host, V.Q4_K, rows, cols, 5, 1)
    x = V.synth_normal(host, cols, 5, 2)
    big = np.zeros((20 << 20) // 4, np.float32)
    big[:cols] = x
    pw, px, py = dev.upload(w), dev.upload(big), dev.alloc(rows * 4)
    try:
        dev.linear(V.Q4_K, pw, px, py, cols, rows)
        first = dev.download(py, rows, np.float32)
        dev.linear(V.Q4_K, pw, px, py, cols, rows)
        dev.write(px, np.ones_like(big))
        again = dev.download(py, rows, np.float32)
        assert np.array_equal(first.view(np.uint32), again.view(np.uint32))
    finally:
        for p in (pw, px, py):
            dev.free(p)


@pytest.mark.parametrize("variant", [0, 1, 2], ids=["dma_1wg", "dma_2wg", "reg"])
@pytest.mark.parametrize("nbytes", [16, 1008, 65536, 65536 + 48, 3 * 65536 - 16, 25362432])
def test_checksum_matches_host(dev, nbytes, variant):
    """vbs_gfx950_checksum (and its read-floor variants: two workgroups per
    CU, register loads) over regions that end inside a 1 KB run, a workgroup
    span and exactly on one: the XOR of the partial words equals the host's
    XOR of the same 32-bit words, and one flipped bit changes it."""
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    p = dev.upload(host)
    try:
        assert dev.checksum(p, nbytes, variant) == int(np.bitwise_xor.reduce(host))
        flipped = host.copy()
        flipped[-1] ^= 1 << 7
        dev.write(p, flipped)
        assert dev.checksum(p, nbytes, variant) == int(np.bitwise_xor.reduce(host)) ^ (1 << 7)
    finally:
        dev.free(p)
