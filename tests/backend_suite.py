"""The reference's backend self-test (src/vbs_backend_test.c:456-963),
restated as a reusable check list that drives any vbs_backend_ops_t table
through the ops table only, with reference values from the CPU oracle.

Checks and tolerances follow the reference: 1 MiB copy round trip; add n=1000
(1e-6); silu*up n=777 (1e-5); rms_norm dim 384 (1e-5); rope theta 1e4 and 5e5
at pos 7 (1e-5); embedding of all seven types, token 3, dim 256 (1e-4, F16
1e-3); KV store at layer 1 / pos 5 then GQA attention nqh 4 / nkh 2 / hd 32 /
seq 6 (1e-4); linear 8x256 for F32, F16, Q8_0, Q4_0, Q4_1, Q4_K, Q6_K, LNS8 in
both calling conventions (F32 1e-4, others 2e-3); two F32 column tiles with
offsets and accumulate (1e-4); Q8_K linear refused.
"""
import ctypes as C
import math

import numpy as np

import vbs_gfx950 as V


def close(got, want, tol):
    d = np.abs(got.astype(np.float64) - want)
    return bool(np.all(d <= tol + tol * np.abs(want))), float(d.max() if d.size else 0.0)


def lns8_blocks(rng, n_blocks):
    b = np.zeros((n_blocks, 36), np.uint8)
    b[:, :32] = rng.integers(100, 128, (n_blocks, 32))  # 2^code stays finite
    b[:, 32:36] = np.frombuffer(np.float32(2.0 ** -118).tobytes(), np.uint8)
    return b.reshape(-1)


def packed(host, t, rows, cols, seed, stream, rng):
    if t == V.LNS8:
        return lns8_blocks(rng, rows * cols // 32).reshape(rows, -1)
    return V.synth_matrix(host, t, rows, cols, seed, stream)


def run_suite(be: V.Backend, orc, host, seed=12345):
    rng = np.random.default_rng(seed)
    res = []
    dev = be.device()
    keep = []

    def buf(a):
        return be.upload(np.ascontiguousarray(a))

    def get(b, n, dt=np.float32):
        return be.download(b, n, dt)

    def prim(kind):
        return be.ops.compile_primitive_pipeline(dev, kind, None, 0)

    def A(b):
        return V.Backend.buf_arg(b)

    # alloc/copy round trip
    src = (np.arange(1 << 20, dtype=np.uint64) * 2654435761 >> 24).astype(np.uint8)
    b = buf(src)
    res.append(("copy 1 MiB", np.array_equal(get(b, src.size, np.uint8), src), 0))
    be.ops.free_buffer(b)

    # add
    n = 1000
    a_, b_ = rng.uniform(-1, 1, n).astype(np.float32), rng.uniform(-1, 1, n).astype(np.float32)
    ba, bb, bo = buf(a_), buf(b_), buf(np.zeros(n, np.float32))
    ok = be.dispatch(prim(V.OP_ELEMENTWISE), [A(ba), A(bb), A(bo), be.u32_arg(keep, n)], 4, 256)
    be.ops.synchronize_device(dev)
    res.append(("add n=1000", ok and close(get(bo, n), orc.add(a_, b_), 1e-6)[0], 0))

    # silu
    n = 777
    g_, u_ = (rng.uniform(-1, 1, n) * 3).astype(np.float32), rng.uniform(-1, 1, n).astype(np.float32)
    bg, bu, bo = buf(g_), buf(u_), buf(np.zeros(n, np.float32))
    ok = be.dispatch(prim(V.OP_ACTIVATION), [A(bg), A(bu), A(bo), be.u32_arg(keep, n)], 4, 256)
    res.append(("silu_mul n=777", ok and close(get(bo, n), orc.silu_mul(g_, u_), 1e-5)[0], 0))

    # rms_norm
    n = 384
    x_, w_ = (rng.uniform(-1, 1, n) * 2).astype(np.float32), rng.uniform(-1, 1, n).astype(np.float32)
    bx, bw, bo = buf(x_), buf(w_), buf(np.zeros(n, np.float32))
    ok = be.dispatch(prim(V.OP_NORMALIZE), [A(bx), A(bw), A(bo), be.u32_arg(keep, n),
                                            be.f32_arg(keep, 1e-5)], 2, 256)
    res.append(("rms_norm dim=384", ok and close(get(bo, n), orc.rms_norm(x_, w_, np.float32(1e-5)), 1e-5)[0], 0))

    # rope, two thetas
    for theta in (10000.0, 500000.0):
        x_ = rng.uniform(-1, 1, 4 * 64).astype(np.float32)
        bx = buf(x_)
        ok = be.dispatch(prim(V.OP_ROTARY), [A(bx), be.u32_arg(keep, 7), be.u32_arg(keep, 64),
                                             be.u32_arg(keep, 4), be.f32_arg(keep, theta)], 1, 256)
        res.append((f"rope theta={theta:.0f}", ok and close(get(bx, 256), orc.rope(x_, 7, 64, 4, theta), 1e-5)[0], 0))

    # embedding, all seven types
    for t, tol in ((V.F32, 1e-6), (V.F16, 1e-3), (V.Q8_0, 1e-4), (V.Q4_0, 1e-4),
                   (V.Q4_1, 1e-4), (V.Q4_K, 1e-4), (V.Q6_K, 1e-4)):
        table = packed(host, t, 8, 256, seed, 40 + t, rng)
        bt, bo = buf(table), buf(np.zeros(256, np.float32))
        pipe = be.ops.compile_embed_pipeline(dev, t, None, 0)
        ok = bool(pipe) and be.dispatch(pipe, [A(bt), be.u32_arg(keep, 3), A(bo), be.u32_arg(keep, 256)], 1, 256)
        want = orc.embed(t, table, 3, 256)
        res.append((f"embed {V.TYPE_NAMES[t]}", ok and close(get(bo, 256), want, tol)[0], 0))

    # kv store at layer 1 pos 5, then positions 0..4, then attention over 6
    L, mc, nkh, hd, nqh = 2, 16, 2, 32, 4
    kvd = nkh * hd
    kc_h = np.zeros(L * mc * kvd, np.uint16)
    vc_h = np.zeros_like(kc_h)
    bkc, bvc = buf(kc_h), buf(vc_h)
    ok = True
    for pos in (5, 0, 1, 2, 3, 4):
        k_, v_ = rng.uniform(-1, 1, kvd).astype(np.float32), rng.uniform(-1, 1, kvd).astype(np.float32)
        bk, bv = buf(k_), buf(v_)
        ok &= be.dispatch(prim(V.OP_CACHE), [A(bk), A(bv), A(bkc), A(bvc), be.u32_arg(keep, pos),
                                             be.u32_arg(keep, 1), be.u32_arg(keep, mc),
                                             be.u32_arg(keep, kvd)], 1, 256)
        orc.cache_store(k_, v_, kc_h, vc_h, pos, 1, mc, kvd)
    gk, gv = get(bkc, kc_h.size, np.uint16), get(bvc, vc_h.size, np.uint16)
    res.append(("kv_cache_store layer=1 pos=0..5", ok and np.array_equal(gk, kc_h) and np.array_equal(gv, vc_h), 0))
    q_ = rng.uniform(-1, 1, nqh * hd).astype(np.float32)
    bq, bo = buf(q_), buf(np.zeros(nqh * hd, np.float32))
    scale = np.float32(1.0 / math.sqrt(hd))
    ok = be.dispatch(prim(V.OP_ATTENTION), [A(bq), A(bkc), A(bvc), A(bo), be.u32_arg(keep, 6),
                                            be.u32_arg(keep, 1), be.u32_arg(keep, mc),
                                            be.u32_arg(keep, nqh), be.u32_arg(keep, nkh),
                                            be.u32_arg(keep, hd), be.f32_arg(keep, scale)], nqh, 32)
    want = orc.attention(q_, kc_h, vc_h, 6, 1, mc, nqh, nkh, hd, scale)
    res.append(("attention_gqa nqh=4 nkh=2 hd=32 seq=6", ok and close(get(bo, nqh * hd), want, 1e-4)[0], 0))

    # linear tiles, both calling conventions
    rows, cols = 8, 256
    for t, tol in ((V.F32, 1e-4), (V.F16, 2e-3), (V.Q8_0, 2e-3), (V.Q4_0, 2e-3), (V.Q4_1, 2e-3),
                   (V.Q4_K, 2e-3), (V.Q6_K, 2e-3), (V.LNS8, 2e-3)):
        w = packed(host, t, rows, cols, seed, 60 + t, rng)
        x_ = rng.uniform(-1, 1, cols).astype(np.float32)
        want = orc.linear(t, w, x_, cols, rows)
        pipe = be.ops.compile_linear_pipeline(dev, t, None, 0)
        bw, bx, by = buf(w), buf(x_), buf(np.zeros(rows, np.float32))
        ok = bool(pipe) and be.ops.dispatch_linear_tile(dev, pipe, bw, None, 0, bx, by, cols, rows,
                                                        0, 0, False)
        be.ops.synchronize_device(dev)
        res.append((f"linear {V.TYPE_NAMES[t]} resident", ok and close(get(by, rows), want, tol)[0], 0))
        stage, priv = be.alloc(w.nbytes, False), be.alloc(w.nbytes, False)
        C.memmove(stage.contents.host_ptr, np.ascontiguousarray(w).ctypes.data, w.nbytes)
        by2 = buf(np.zeros(rows, np.float32))
        ok = bool(pipe) and be.ops.dispatch_linear_tile(dev, pipe, priv, stage, w.nbytes, bx, by2,
                                                        cols, rows, 0, 0, False)
        res.append((f"linear {V.TYPE_NAMES[t]} staged", ok and close(get(by2, rows), want, tol)[0], 0))
        for bb_ in (stage, priv, bw, bx, by, by2):
            be.ops.free_buffer(bb_)

    # offsets + accumulate: two F32 column tiles
    rows, cols, half = 4, 256, 128
    mat = rng.uniform(-1, 1, (rows, cols)).astype(np.float32)
    x_ = rng.uniform(-1, 1, cols).astype(np.float32)
    want = (mat.astype(np.float64) @ x_.astype(np.float64)).astype(np.float32)
    pipe = be.ops.compile_linear_pipeline(dev, V.F32, None, 0)
    bx, by = buf(x_), buf(np.zeros(rows, np.float32))
    ok = True
    for tile in range(2):
        tm = np.ascontiguousarray(mat[:, tile * half:(tile + 1) * half])
        stage, priv = be.alloc(tm.nbytes, True), be.alloc(tm.nbytes)
        C.memmove(stage.contents.host_ptr, tm.ctypes.data, tm.nbytes)
        ok &= be.ops.dispatch_linear_tile(dev, pipe, priv, stage, tm.nbytes, bx, by, half, rows,
                                          tile * half, 0, tile == 1)
        be.ops.free_buffer(stage)
        be.ops.free_buffer(priv)
    be.ops.synchronize_device(dev)
    res.append(("linear F32 offsets+accumulate 2 tiles", ok and close(get(by, rows), want, 1e-4)[0], 0))

    # refusal
    err = C.create_string_buffer(256)
    p = be.ops.compile_linear_pipeline(dev, V.Q8_K, err, 256)
    res.append(("linear Q8_K refused", not p and len(err.value) > 0, 0))
    return res


def bind_linear_batch(be: V.Backend):
    """vbs_hip_dispatch_linear_batch / vbs_hip_linear_batch_version of the
    shim (include/vbs_hip_batch.h)."""
    lib = be.lib
    lib.vbs_hip_linear_batch_version.restype = C.c_uint32
    f = lib.vbs_hip_dispatch_linear_batch
    f.restype = C.c_bool
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p,
                  C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]
    return f


def run_linear_batch(be: V.Backend, orc, host, shapes, batches, seed=777):
    """The batched extension through the shim against `batch` independent
    oracle linear tiles (src/vbs_host_math.h:223-267): (name, ok) pairs,
    including the argument refusals."""
    fn = bind_linear_batch(be)
    res = [("linear batch version", be.lib.vbs_hip_linear_batch_version() == 1)]
    dev = be.device()
    for t, rows, cols in shapes:
        pipe = be.ops.compile_linear_pipeline(dev, t, None, 0)
        w = V.synth_matrix(host, t, rows, cols, seed, 5)
        bw = be.upload(w)
        for batch in batches:
            xs, ys = cols + 32, rows + 7  # strides beyond the shape
            x = np.zeros(batch * xs, np.float32)
            for b in range(batch):
                x[b * xs:b * xs + cols] = V.synth_normal(host, cols, seed + b, 6)
            bx, by = be.upload(x), be.upload(np.full(batch * ys, -1.0, np.float32))
            ok = fn(dev, pipe, bw, bx, xs, by, ys, cols, rows, batch)
            y = be.download(by, batch * ys, np.float32) if ok else None
            good = bool(ok)
            for b in range(batch if ok else 0):
                want = orc.linear(t, w, x[b * xs:b * xs + cols], cols, rows)
                got = y[b * ys:b * ys + rows]
                rel = np.linalg.norm(got.astype(np.float64) - want) / max(
                    np.linalg.norm(want.astype(np.float64)), 1e-30)
                good &= bool(rel <= 1e-5) and bool(np.all(y[b * ys + rows:(b + 1) * ys] == -1.0))
            res.append((f"linear batch {V.TYPE_NAMES[t]} {rows}x{cols} b{batch}", good))
            be.ops.free_buffer(bx)
            be.ops.free_buffer(by)
        # refusals: nothing launched, a reason left
        bx = be.upload(np.zeros(cols * 17, np.float32))
        by = be.upload(np.zeros(rows * 17, np.float32))
        for name, args in [("batch 0", (cols, rows, 0)), ("batch 17", (cols, rows, 17)),
                           ("x stride", (cols - 1, rows, 2)), ("y stride", (cols, rows - 1, 2))]:
            xs_, ys_, b_ = args
            res.append((f"linear batch refuses {name}",
                        not fn(dev, pipe, bw, bx, xs_, by, ys_, cols, rows, b_)
                        and "linear batch" in be.last_error()))
        small = be.upload(np.zeros(cols, np.float32))
        res.append(("linear batch refuses a short x",
                    not fn(dev, pipe, bw, small, cols, by, rows, cols, rows, 2)))
        for b_ in (bw, bx, by, small):
            be.ops.free_buffer(b_)
    return res
