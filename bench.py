#!/usr/bin/env python3
"""Benchmark of the gfx950 quantized decode hot path (one MI355X).

Metric: Q4_K matvec HBM GB/s (% of peak); decode tokens/sec
at 7B Q4_K_M, 1 GPU.

A step is one pass of the Llama-7B layer matvec set at batch 1 (config 2):
Q, K, V, O 4096x4096, gate and up 11008x4096, down 4096x11008, all Q4_K,
f32 activations. Weights are synthetic (host/vbs_synth.c, the config-2
distributions) and resident in HBM before timing starts; NCOPY distinct copies
of the layer set rotate so the 256 MB Infinity Cache cannot serve re-reads.
`value` is algorithmic bytes (packed W + 4*cols + 4*rows per matvec) per
second over the timed steps.

Each step is one HIP graph of its seven launches (captured from the library's
stream), so the timed region measures the kernels rather than the host's
per-call launch cost.

roofline: the dominant kernel is the Q4_K matvec at 11008x4096 / 4096x11008;
its average duration is the elapsed time between two HIP events on the
library's stream around `roof_reps` replays of a graph holding those launches
for every weight copy, divided by the number of launches (inter-kernel gaps
included, so it is an upper bound on the kernel time rocprof reports).

cpu_baseline: the reference's own CPU backend (oracle/_ref, compiled from the
reference sources) -- or, where that file is absent, the oracle restatement --
runs dispatch_linear_tile over the same layer set, single-threaded as the
reference is, for a bounded number of passes. Its `beside` entries time the
reference CPU path on the host copies of the other GPU entries (configs 1 and
3, the hot-table call).

Also reported: configs 1-3 on the GPU; the CPU hot-kernel table
(vbs_hotpath.h ABI v1) as a device kernel and as the host-pointer module;
decode tokens/sec of the synthetic 7B Q4_K_M model (config 4:
32 layers, KV prefilled to 2048, greedy from position 2048) through the graph
decoder (vbs_gfx950_decoder_*), and through the g_vbs_hip_backend ops table
with one dispatch per bridge call. The decode entry's `checked` block comes
from the CPU leg, after every GPU timing: the decoded tokens against the
reference CPU backend's 128 for the same model and start
(tests/golden/decode_7b_greedy.npz) and the first four against the oracle's
forward pass run on the host; beside it, the decode entry's `cpu_baseline` is
the same decode on the host: one full token of the reference CPU backend on one thread (driven
through its ops table in the bridge's order) and, as `all_cores`, the
oracle's forward pass on every core.

roofline.ceiling.read_floor.variants: the same 25 MB read with two
workgroups per CU and with register loads instead of LDS DMA, timed like the
matvec, to show how tight the read floor is.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "verum-bespoke-singularity_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
import vbs_gfx950 as V  # noqa: E402
from vbs_gfx950 import Hip  # noqa: E402

PEAK_HBM_GBS = 8000.0
H, FF = 4096, 11008
LAYER_SET = [("q", H, H), ("k", H, H), ("v", H, H), ("o", H, H),
             ("gate", FF, H), ("up", FF, H), ("down", H, FF)]  # (name, rows, cols)
SEED = 424242
# Config 4's synthetic model seed: the one the reference CPU backend's 128
# greedy tokens in tests/golden/decode_7b_greedy.npz were decoded with.
DECODE_SEED = 7
DECODE_FIXTURE = os.path.join(ROOT, "tests", "golden", "decode_7b_greedy.npz")

# HBM bytes per launch of the dominant kernel (11008x4096 Q4_K, k_mvl) from
# two rocprofv3 --pmc passes over this program (FETCH_SIZE, WRITE_SIZE in KiB
# per dispatch), each scaled by what the counter reads for a 256 MiB device
# copy in the same run: FETCH_SIZE x (262144 / 131092.9) + WRITE_SIZE x 1.0000
# (profiles/q4k_matvec_7b_layer_set.md).
TRAFFIC_BYTES = round((12479.5 * 262144 / 131092.9 + 50.0) * 1024)


def algo_bytes(t, rows, cols):
    return V.row_bytes(t, cols) * rows + 4 * cols + 4 * rows


def cpu_hot_q8_0_s(w, xq, qd, rows, cols, max_seconds=1.0):
    """Seconds per call of the reference's built-in hot-table matvec_q8_0
    (src/vbs_hotpath.c compiled into oracle/_ref), or None if not built."""
    from oracle_lib import REF_HOT_SO, reference_hot
    if not os.path.exists(REF_HOT_SO):
        return None
    tb = reference_hot().vbs_hot_builtin().contents
    y = np.empty(rows, np.float32)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < max_seconds:
        tb.matvec_q8_0(w.ctypes.data, rows, cols, xq.ctypes.data, qd.ctypes.data, y.ctypes.data)
        n += 1
    return (time.perf_counter() - t0) / n


def cpu_beside(work):
    """The reference CPU path on the host copies of the other GPU entries
    (single-threaded, as the reference is)."""
    out = {}
    for name, job in work.items():
        if job[0] == "linear":
            _, t, w, rows, cols, b, budget = job
            sec, kind = cpu_linear_s(t, w, rows, cols, max_seconds=budget)
        else:
            _, w, xq, qd, rows, cols, b, budget = job
            sec, kind = cpu_hot_q8_0_s(w, xq, qd, rows, cols, budget), "reference"
            if sec is None:
                continue
        out[name] = {"ms_per_matvec": round(1e3 * sec, 3), "GB_per_s": round(b / sec / 1e9, 4),
                     "kind": kind, "cores": 1}
    return out


def cpu_baseline(host, weights, xs, min_seconds=10.0, beside=None):
    """Single-threaded reference CPU linear over the layer set: whole passes
    until at least min_seconds of CPU work (a bounded sample, ~10-12 s)."""
    from oracle_lib import REF_SO, Oracle
    kind, passes, t_total, nbytes = "port", 0, 0.0, 0
    ys = [np.zeros(r, np.float32) for _, r, _ in LAYER_SET]
    if os.path.exists(REF_SO):
        kind = "reference"
        lib = C.CDLL(REF_SO)
        ref = V.Backend(lib, "g_vbs_cpu_backend")
        ref.init()
        pipe = ref.ops.compile_linear_pipeline(ref.device(), V.Q4_K, None, 0)
        bufs = []
        for (_, r, c), w, x, y in zip(LAYER_SET, weights, xs, ys):
            mk = lambda a: V.VbsBuffer(a.ctypes.data, a.ctypes.data, a.nbytes, ref.device())
            bufs.append((mk(w), mk(x), mk(y), r, c))

        def one(i):
            bw, bx, by, r, c = bufs[i]
            ok = ref.ops.dispatch_linear_tile(ref.device(), pipe, C.byref(bw), None, 0,
                                              C.byref(bx), C.byref(by), c, r, 0, 0, False)
            assert ok
    else:
        orc = Oracle()

        def one(i):
            _, r, c = LAYER_SET[i]
            orc.linear(V.Q4_K, weights[i], xs[i], c, r, y=ys[i], threads=1)
    t0 = time.perf_counter()
    while True:
        for i in range(len(LAYER_SET)):
            one(i)
        passes += 1
        t_total = time.perf_counter() - t0
        if t_total >= min_seconds:
            break
    nbytes = passes * sum(algo_bytes(V.Q4_K, r, c) for _, r, c in LAYER_SET)
    cpu = host_cpu_model()
    # beside it: the oracle's row-parallel restatement on every host core
    # (bit-identical outputs to the single-threaded path, tested)
    orc_all = Oracle()
    ncores = min(16, os.cpu_count() or 1)
    ys_all = [np.zeros(r, np.float32) for _, r, _ in LAYER_SET]
    p_all, t0 = 0, time.perf_counter()
    while True:
        for i, (_, r, c) in enumerate(LAYER_SET):
            orc_all.linear(V.Q4_K, weights[i], xs[i], c, r, y=ys_all[i], threads=ncores)
        p_all += 1
        t_all = time.perf_counter() - t0
        if t_all >= 2.0 or p_all >= 256:
            break
    all_cores = {"value": round(p_all * sum(algo_bytes(V.Q4_K, r, c) for _, r, c in LAYER_SET)
                                / t_all / 1e9, 4), "unit": "GB/s", "cores": ncores,
                 "kind": "port", "sample": f"{p_all} pass(es) of the same layer set in "
                                           f"{t_all:.1f} s, oracle row-parallel linear"}
    return {"value": round(nbytes / t_total / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
            "all_cores": all_cores, "beside": cpu_beside(beside or {}),
            "sample": f"{passes} pass(es) of the Q4_K 7B layer matvec set "
                      f"({len(LAYER_SET)} matvecs, {nbytes / passes / 1e6:.1f} MB each pass) in "
                      f"{t_total:.1f} s, single thread, dispatch_linear_tile of the "
                      f"{'reference CPU backend' if kind == 'reference' else 'oracle port'}; "
                      f"host: {cpu}, nproc {os.cpu_count()}"}


def bench_matvec(dev, host, steps, warmup, ncopy, roof_reps):
    t = V.Q4_K
    weights_host = [V.synth_matrix(host, t, r, c, SEED, 10 + i) for i, (_, r, c) in enumerate(LAYER_SET)]
    xs_host = [V.synth_normal(host, c, SEED, 30 + i) for i, (_, _, c) in enumerate(LAYER_SET)]
    # NCOPY distinct resident copies of the layer set (different bytes per copy)
    copies = []
    for k in range(ncopy):
        set_k = []
        for i, (_, r, c) in enumerate(LAYER_SET):
            w = weights_host[i] if k == 0 else V.synth_matrix(host, t, r, c, SEED + k, 10 + i)
            set_k.append(dev.upload(w))
        copies.append(set_k)
    px = [dev.upload(x) for x in xs_host]
    py = [dev.upload(np.zeros(r, np.float32)) for _, r, _ in LAYER_SET]
    stream = dev.stream()
    hip = Hip()
    big = [i for i, (_, r, c) in enumerate(LAYER_SET) if r * c == H * FF]

    def enqueue(k, which):
        for i in which:
            _, r, c = LAYER_SET[i]
            dev.linear(t, copies[k][i], px[i], py[i], c, r)

    # one graph per copy: the seven launches of a step, replayed per step
    step_graphs = [hip.capture(stream, lambda k=k: enqueue(k, range(len(LAYER_SET))))
                   for k in range(ncopy)]
    for s in range(warmup):
        hip.launch(step_graphs[s % ncopy], stream)
    dev.sync()
    # timed region: exactly K steps, synchronised on both sides
    e0, e1 = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(e0, stream)
    for s in range(steps):
        hip.launch(step_graphs[s % ncopy], stream)
    hip.record(e1, stream)
    dev.sync()
    wall = time.perf_counter() - t0
    gpu_ms = hip.elapsed_ms(e0, e1)
    # dominant kernel: the three 11008-wide matvecs of every copy back to back,
    # replayed roof_reps times between two events on the same stream
    big_graph = hip.capture(stream, lambda: [enqueue(k, big) for k in range(ncopy)])
    hip.launch(big_graph, stream)
    dev.sync()
    evs = [hip.event() for _ in range(roof_reps + 1)]
    hip.record(evs[0], stream)
    for i in range(roof_reps):
        hip.launch(big_graph, stream)
        hip.record(evs[i + 1], stream)
    dev.sync()
    per_launch = ncopy * len(big)
    big_ms = hip.elapsed_ms(evs[0], evs[-1]) / (roof_reps * per_launch)
    rep_ms = sorted(hip.elapsed_ms(evs[i], evs[i + 1]) / per_launch for i in range(roof_reps))
    ceiling = bench_ceiling(dev, hip, stream, [copies[k][i] for k in range(ncopy) for i in big],
                            algo_bytes(t, FF, H) - 4 * (FF + H), roof_reps)
    # a replay of copy 0's step graph against the same launches issued eagerly
    hip.launch(step_graphs[0], stream)
    y_graph = [dev.download(py[i], (r,), np.float32) for i, (_, r, _) in enumerate(LAYER_SET)]
    for g in step_graphs + [big_graph]:
        hip.destroy(g)
    enqueue(0, range(len(LAYER_SET)))
    y_eager = [dev.download(py[i], (r,), np.float32) for i, (_, r, _) in enumerate(LAYER_SET)]
    replay_equal = all(np.array_equal(a.view(np.uint32), b.view(np.uint32))
                       for a, b in zip(y_graph, y_eager))
    step_bytes = sum(algo_bytes(t, r, c) for _, r, c in LAYER_SET)
    res = {"step_bytes": step_bytes, "wall_s": wall, "gpu_ms": gpu_ms,
           "big_bytes": algo_bytes(t, FF, H), "avg_big_ms": big_ms, "rep_big_ms": rep_ms,
           "replay_equals_eager": replay_equal, "ceiling": ceiling,
           "weights_host": weights_host, "xs_host": xs_host}
    for k_ in copies:
        for p in k_:
            dev.free(p)
    for p in px + py:
        dev.free(p)
    return res


def bench_ceiling(dev, hip, stream, regions, region_bytes, reps):
    """What a launch of this size can reach on this part, measured the way the
    roofline is (graph replays between HIP events on the library's stream):
    vbs_gfx950_checksum reading the same weight regions the dominant matvec
    reads (every byte once, nothing else: the read floor), the same over
    1 GiB (the streaming rate), a 16-byte checksum (the cost of one launch
    back to back), and device-to-device copies of 25.4 MB and 1 GiB."""
    n_part = int(dev._checksum_partials(1 << 30))
    part = dev.alloc(4 * n_part)

    def per_launch_us(enqueue, launches, rep):
        g = hip.capture(stream, enqueue)
        hip.launch(g, stream)
        dev.sync()
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, stream)
        for _ in range(rep):
            hip.launch(g, stream)
        hip.record(e1, stream)
        dev.sync()
        hip.destroy(g)
        return hip.elapsed_ms(e0, e1) * 1e3 / (rep * launches)

    out = {}
    read_us = per_launch_us(lambda: [dev.check(dev._checksum(r, region_bytes, part), "checksum")
                                     for r in regions], len(regions), reps)
    # the same read in two other shapes: is the floor tight?
    variants = {}
    for v, name in ((1, "two_8wave_workgroups_per_cu_lds_dma"),
                    (2, "one_16wave_workgroup_per_cu_register_loads")):
        us = per_launch_us(lambda: [dev.check(dev._checksum_variant(r, region_bytes, part, v),
                                              "checksum") for r in regions], len(regions), reps)
        variants[name] = {"us_per_launch": round(us, 3),
                          "frac": round(region_bytes / us / 1e3 / PEAK_HBM_GBS, 4)}
    gib = 1 << 30
    big = dev.alloc(gib)
    try:
        stream_us = per_launch_us(lambda: [dev.check(dev._checksum(big, gib, part), "checksum")
                                           for _ in range(2)], 2, 4)
        one_us = per_launch_us(lambda: [dev.check(dev._checksum(big, 16, part), "checksum")
                                        for _ in range(100)], 100, 4)
        dst = dev.alloc(region_bytes)
        try:
            cp_us = per_launch_us(lambda: [dev.check(dev._copy_d2d(dst, r, region_bytes), "copy")
                                           for r in regions], len(regions), 8)
        finally:
            dev.free(dst)
        half = gib // 2
        cpg_us = per_launch_us(lambda: [dev.check(dev._copy_d2d(big + half, big, half), "copy")
                                        for _ in range(2)], 2, 4)
    finally:
        dev.free(big)
        dev.free(part)
    gbs = lambda b, us: round(b / us / 1e3, 1)
    out = {"read_floor": {"us_per_launch": round(read_us, 3),
                          "GB_per_s": gbs(region_bytes, read_us),
                          "frac": round(region_bytes / read_us / 1e3 / PEAK_HBM_GBS, 4),
                          "bytes": region_bytes,
                          "kernel": "vbs_gfx950_checksum over the same weight copies",
                          "variants": variants},
           "stream_1GiB_GB_per_s": gbs(gib, stream_us),
           "launch_floor_us": round(one_us, 3),
           "copy_d2d_GB_per_s": {"25.4MB_read_plus_write": gbs(2 * region_bytes, cp_us),
                                 "512MiB_read_plus_write": gbs(2 * half, cpg_us)}}
    return out


def gpu_matvec_us(dev, host, t, rows, cols, rotate_bytes=400e6, reps=3):
    """Average µs per batch-1 vbs_gfx950_linear launch of a (t, rows, cols)
    matrix: distinct resident copies (>= rotate_bytes together) replayed in
    one HIP graph, HIP events on the library's stream."""
    hip, stream = Hip(), dev.stream()
    w0 = V.synth_matrix(host, t, rows, cols, SEED, 400)
    ncopy = max(2, int(rotate_bytes // w0.nbytes) + 1)
    ws = [dev.upload(w0 if k == 0 else V.synth_matrix(host, t, rows, cols, SEED + k, 400))
          for k in range(ncopy)]
    x = dev.upload(V.synth_normal(host, cols, SEED, 401))
    y = dev.upload(np.zeros(rows, np.float32))
    per = 4
    g = hip.capture(stream, lambda: [dev.linear(t, ws[i % ncopy], x, y, cols, rows)
                                     for i in range(per * ncopy)])
    hip.launch(g, stream)
    dev.sync()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    for _ in range(reps):
        hip.launch(g, stream)
    hip.record(e1, stream)
    dev.sync()
    us = hip.elapsed_ms(e0, e1) * 1e3 / (reps * per * ncopy)
    hip.destroy(g)
    for p in ws + [x, y]:
        dev.free(p)
    return us, w0


def cpu_linear_s(t, w, rows, cols, max_seconds=2.0):
    """Seconds per single-threaded reference CPU matvec (oracle/_ref's
    dispatch_linear_tile; the oracle restatement when it is not built)."""
    from oracle_lib import REF_SO, Oracle
    x = np.ones(cols, np.float32)
    y = np.zeros(rows, np.float32)
    if os.path.exists(REF_SO):
        ref = V.Backend(C.CDLL(REF_SO), "g_vbs_cpu_backend")
        ref.init()
        pipe = ref.ops.compile_linear_pipeline(ref.device(), t, None, 0)
        mk = lambda a: V.VbsBuffer(a.ctypes.data, a.ctypes.data, a.nbytes, ref.device())
        bw, bx, by = mk(w), mk(x), mk(y)
        one = lambda: ref.ops.dispatch_linear_tile(ref.device(), pipe, C.byref(bw), None, 0,
                                                   C.byref(bx), C.byref(by), cols, rows, 0, 0,
                                                   False)
        kind = "reference"
    else:
        orc = Oracle()
        one = lambda: orc.linear(t, w, x, cols, rows, y=y, threads=1)
        kind = "port"
    n, t0 = 0, time.perf_counter()
    while True:
        one()
        n += 1
        if time.perf_counter() - t0 >= max_seconds * 0.5:
            break
    return (time.perf_counter() - t0) / n, kind


def bench_configs(dev, host, cpu_work=None):
    """The other benchmark configurations at batch 1 on the GPU: config 1 Q4_0
    4096x4096; config 2's Q8_0 repetition of the 7B layer set; config 3's
    Q6_K 32000x4096 head and the 64-id Q6_K embedding gather. The host copies
    of configs 1 and 3 go into `cpu_work` for the CPU baseline leg."""
    out = {}
    us, w = gpu_matvec_us(dev, host, V.Q4_0, 4096, 4096)
    b = algo_bytes(V.Q4_0, 4096, 4096)
    c1 = {"workload": "Q4_0 4096x4096 matvec, batch 1 (config 1)", "us_per_matvec": round(us, 3),
          "GB_per_s": round(b / us / 1e3, 1), "roofline_frac": round(b / us / 1e3 / PEAK_HBM_GBS, 4)}
    if cpu_work is not None:
        cpu_work["config1_q4_0"] = ("linear", V.Q4_0, w, 4096, 4096, b, 2.0)
    out["config1_q4_0"] = c1
    tot_us, tot_b, per = 0.0, 0, {}
    for name, r, c in LAYER_SET:
        key = f"{r}x{c}"
        if key not in per:
            per[key] = gpu_matvec_us(dev, host, V.Q8_0, r, c)[0]
        tot_us += per[key]
        tot_b += algo_bytes(V.Q8_0, r, c)
    out["config2_q8_0_layer_set"] = {
        "workload": "Llama-7B layer matvec set in Q8_0, batch 1 (config 2)",
        "us_per_set": round(tot_us, 2), "GB_per_s": round(tot_b / tot_us / 1e3, 1),
        "roofline_frac": round(tot_b / tot_us / 1e3 / PEAK_HBM_GBS, 4),
        "us_per_shape": {k: round(v, 2) for k, v in per.items()}}
    us, w = gpu_matvec_us(dev, host, V.Q6_K, 32000, 4096)
    b = algo_bytes(V.Q6_K, 32000, 4096)
    c3 = {"workload": "Q6_K 32000x4096 output head, batch 1 (config 3)", "us_per_matvec": round(us, 3),
          "GB_per_s": round(b / us / 1e3, 1), "roofline_frac": round(b / us / 1e3 / PEAK_HBM_GBS, 4)}
    if cpu_work is not None:
        cpu_work["config3_q6_k_head"] = ("linear", V.Q6_K, w, 32000, 4096, b, 1.0)
    # 64 random ids gathered from the same table in one launch
    hip, stream = Hip(), dev.stream()
    table = dev.upload(w)
    rng = np.random.default_rng(SEED)
    ids = dev.upload(rng.integers(0, 32000, 64).astype(np.uint32))
    outp = dev.upload(np.zeros(64 * 4096, np.float32))
    g = hip.capture(stream, lambda: [dev.dequant_rows(V.Q6_K, table, ids, 64, 4096, outp)
                                     for _ in range(50)])
    hip.launch(g, stream)
    dev.sync()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    for _ in range(4):
        hip.launch(g, stream)
    hip.record(e1, stream)
    dev.sync()
    gus = hip.elapsed_ms(e0, e1) * 1e3 / 200
    hip.destroy(g)
    for p in (table, ids, outp):
        dev.free(p)
    gb = 64 * V.row_bytes(V.Q6_K, 4096) + 64 * 4096 * 4
    c3["gather_64_ids_us"] = round(gus, 3)
    c3["gather_GB_per_s"] = round(gb / gus / 1e3, 1)
    out["config3_q6_k_head"] = c3
    return out


def bench_hot_table(dev, host, cpu_work=None, rows=4096, cols=4096):
    """The CPU hot-kernel table (the reference's vbs_hotpath.h ABI v1) on the
    device: Q8_0 rows x cols (the CPU model's Q8_0 weights, Q8 activations).
    Reports the device kernel on resident buffers (distinct copies rotated,
    one graph, HIP events) and the host-pointer module call as the
    reference's CPU model would make it (weights over PCIe every call); the
    same call goes into `cpu_work` for the reference's built-in CPU kernel."""
    hip, stream = Hip(), dev.stream()
    w0 = V.synth_matrix(host, V.Q8_0, rows, cols, SEED, 500)
    # the Q8 activations the CPU model hands over, made by vbs_gfx950_quantize_q8
    px = dev.upload(V.synth_normal(host, cols, SEED, 501))
    pq, pd, ps = dev.alloc(cols), dev.alloc(cols // 8), dev.alloc(cols // 8)
    dev.quantize_q8(px, cols, pq, pd, ps)
    xq, qd = dev.download(pq, cols, np.int8), dev.download(pd, cols // 32, np.float32)
    for p in (px, ps):
        dev.free(p)
    ncopy = max(2, int(400e6 // w0.nbytes) + 1)
    ws = [dev.upload(w0 if k == 0 else V.synth_matrix(host, V.Q8_0, rows, cols, SEED + k, 500))
          for k in range(ncopy)]
    py = dev.alloc(rows * 4)
    per = 4
    g = hip.capture(stream, lambda: [dev.hot_matvec(V.Q8_0, ws[i % ncopy], rows, cols, pq, pd, 0,
                                                    py) for i in range(per * ncopy)])
    hip.launch(g, stream)
    dev.sync()
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    for _ in range(3):
        hip.launch(g, stream)
    hip.record(e1, stream)
    dev.sync()
    us = hip.elapsed_ms(e0, e1) * 1e3 / (3 * per * ncopy)
    hip.destroy(g)
    for p in ws + [pq, pd, py]:
        dev.free(p)
    b = rows * V.row_bytes(V.Q8_0, cols) + cols + 4 * (cols // 32) + 4 * rows
    out = {"workload": f"hot-table matvec_q8_0 {rows}x{cols} (Q8 activations)",
           "device_us_per_matvec": round(us, 3), "device_GB_per_s": round(b / us / 1e3, 1),
           "device_roofline_frac": round(b / us / 1e3 / PEAK_HBM_GBS, 4)}
    mod = V.HotModule()
    mod.matvec(V.Q8_0, w0, rows, cols, xq=xq, qd=qd)
    n, t0 = 0, time.perf_counter()
    while n < 20:
        mod.matvec(V.Q8_0, w0, rows, cols, xq=xq, qd=qd)
        n += 1
    sec = (time.perf_counter() - t0) / n
    out["module_ms_per_call_pcie_inclusive"] = round(1e3 * sec, 3)
    out["module_GB_per_s_pcie_inclusive"] = round(b / sec / 1e9, 2)
    if cpu_work is not None:
        cpu_work["hot_table_q8_0"] = ("hot_q8_0", w0, xq, qd, rows, cols, b, 1.0)
    return out


def bench_weight_streaming(dev, host, upload_mib=1024, window_mib=64, passes=3):
    """Weight residency and streaming: copy_to_device of pageable host memory
    (how the fabric registers a model) and of pinned memory, and the 7B
    Q4_K layer set streamed through g_vbs_hip_backend's convention B the way
    the slice executor does it (src/vbs_slice_executor.c:42-107): two shared
    stage windows and two private device windows, each tile copied into a
    stage window's host_ptr, then dispatch_linear_tile(priv, stage, ...)."""
    out = {}
    n = upload_mib << 20
    src = np.ones(n, np.uint8)
    p = dev.alloc(n)
    dev.write(p, src)
    t0 = time.perf_counter()
    for _ in range(passes):
        dev.write(p, src)
    out["upload_pageable_GB_per_s"] = round(passes * n / (time.perf_counter() - t0) / 1e9, 2)
    h = dev._host_alloc(n)
    if h:
        C.memmove(h, src.ctypes.data, n)
        dev.check(dev._copy_h2d(p, h, n), "copy_h2d")
        t0 = time.perf_counter()
        for _ in range(passes):
            dev.check(dev._copy_h2d(p, h, n), "copy_h2d")
        out["upload_pinned_GB_per_s"] = round(passes * n / (time.perf_counter() - t0) / 1e9, 2)
        dev._host_free(h)
    dev.free(p)
    del src
    be = V.gfx950_backend()
    if not be.init():
        raise V.GpuError(f"shim init: {be.last_error()}")
    d = be.device()
    win = window_mib << 20
    stage = [be.alloc(win, True) for _ in range(2)]
    priv = [be.alloc(win, False) for _ in range(2)]
    pipe = be.ops.compile_linear_pipeline(d, V.Q4_K, None, 0)
    mats = [(V.synth_matrix(host, V.Q4_K, r, c, SEED, 600 + i), r, c)
            for i, (_, r, c) in enumerate(LAYER_SET)]
    xb = be.upload(V.synth_normal(host, FF, SEED, 601))
    yb = be.upload(np.zeros(FF, np.float32))

    def one_pass():
        turn = 0
        for w, r, c in mats:
            rb = w.shape[1]
            rows_per = max(1, win // rb)
            for rs in range(0, r, rows_per):
                rc = min(rows_per, r - rs)
                slot = turn & 1
                turn += 1
                C.memmove(stage[slot].contents.host_ptr, w[rs:rs + rc].ctypes.data, rc * rb)
                ok = be.ops.dispatch_linear_tile(d, pipe, priv[slot], stage[slot], rc * rb, xb,
                                                 yb, c, rc, 0, rs, False)
                if not ok:
                    raise V.GpuError(f"staged tile: {be.last_error()}")
        be.ops.synchronize_device(d)

    one_pass()
    t0 = time.perf_counter()
    for _ in range(passes):
        one_pass()
    sec = (time.perf_counter() - t0) / passes
    wbytes = sum(w.nbytes for w, _, _ in mats)
    out["staged_layer_set_ms"] = round(1e3 * sec, 3)
    out["staged_layer_set_GB_per_s"] = round(wbytes / sec / 1e9, 2)
    out["staged_window_MiB"] = window_mib
    out["workload"] = ("copy_to_device of %d MiB (pageable, pinned); Q4_K 7B layer set (%.1f MB) "
                       "streamed through convention B in %d MiB windows" %
                       (upload_mib, wbytes / 1e6, window_mib))
    for b in stage + priv + [xb, yb]:
        be.ops.free_buffer(b)
    return out


# Llama-70B layer matvec set (config 5) in the Q4_K_M mix: Q, K, V, O, gate, up, down
LAYER_SET_70B = [("q", V.Q4_K, 8192, 8192), ("k", V.Q4_K, 1024, 8192), ("v", V.Q4_K, 1024, 8192),
                 ("o", V.Q4_K, 8192, 8192), ("gate", V.Q4_K, 28672, 8192),
                 ("up", V.Q4_K, 28672, 8192), ("down", V.Q6_K, 8192, 28672)]


def bench_batch8_70b(dev, host, steps=20, batch=8, ncopy=2):
    """Config 5 at batch 8: the 70B layer matvec set through
    vbs_gfx950_linear_batch_multi as the batched decoder groups it (Q/K/V over
    one prepared x and one launch, O, gate/up over one prepared x, down: four
    preparations and four f16 matrix-core launches), one HIP graph per step,
    `ncopy` resident copies (1.08 GB) rotated so the Infinity Cache cannot
    serve the weights; beside it the same vectors as `batch` batch-1 matvec
    launches each."""
    hip, stream = Hip(), dev.stream()
    copies = [[dev.upload(V.synth_matrix(host, t, r, c, SEED + k, 200 + i))
               for i, (_, t, r, c) in enumerate(LAYER_SET_70B)] for k in range(ncopy)]
    px = {c: dev.upload(np.stack([V.synth_normal(host, c, SEED, 300 + b) for b in range(batch)]))
          for c in {c for _, _, _, c in LAYER_SET_70B}}
    py = [dev.upload(np.zeros(batch * r, np.float32)) for _, _, r, _ in LAYER_SET_70B]

    def step(k, batched):
        if batched:  # Q/K/V and gate/up over one prepared x each, as the batched decoder runs them
            for group in ((0, 1, 2), (3,), (4, 5), (6,)):
                t, c = LAYER_SET_70B[group[0]][1], LAYER_SET_70B[group[0]][3]
                rows = [LAYER_SET_70B[i][2] for i in group]
                dev.linear_batch_multi(t, [copies[k][i] for i in group], rows, px[c], c,
                                       [py[i] for i in group], rows, c, batch)
            return
        for i, (_, t, r, c) in enumerate(LAYER_SET_70B):
            for b in range(batch):
                dev.linear(t, copies[k][i], px[c] + 4 * b * c, py[i] + 4 * b * r, c, r)

    out = {}
    for batched in (True, False):
        step(0, batched)  # sizes the runtime scratch before capture
        dev.sync()
        graphs = [hip.capture(stream, lambda k=k: step(k, batched)) for k in range(ncopy)]
        for s in range(2 * ncopy):
            hip.launch(graphs[s % ncopy], stream)
        e0, e1 = hip.event(), hip.event()
        hip.record(e0, stream)
        for s in range(steps):
            hip.launch(graphs[s % ncopy], stream)
        hip.record(e1, stream)
        dev.sync()
        ms = hip.elapsed_ms(e0, e1) / steps
        for g in graphs:
            hip.destroy(g)
        out["batched" if batched else "batch1_x8"] = ms
    wbytes = sum(V.row_bytes(t, c) * r for _, t, r, c in LAYER_SET_70B)
    for k_ in copies:
        for p in k_:
            dev.free(p)
    for p in list(px.values()) + py:
        dev.free(p)
    return {"workload": "Llama-70B layer matvec set (Q4_K_M mix), batch 8 (config 5)",
            "batch": batch, "weight_bytes_per_step": wbytes, "weight_copies": ncopy,
            "launches": "Q/K/V, O, gate/up, down: each one x preparation + one matrix-core launch",
            "ms_per_step": round(out["batched"], 4),
            "weight_GB_per_s": round(wbytes / (out["batched"] * 1e-3) / 1e9, 1),
            "roofline_frac": round(wbytes / (out["batched"] * 1e-3) / (PEAK_HBM_GBS * 1e9), 4),
            "vector_matvecs_per_s": round(batch * len(LAYER_SET_70B) / (out["batched"] * 1e-3)),
            "batch1_x8_ms_per_step": round(out["batch1_x8"], 4),
            "speedup_vs_batch1_x8": round(out["batch1_x8"] / out["batched"], 2),
            "path": "vbs_gfx950_linear_batch_multi: k_xprep_b + one f16-MFMA launch per matrix group (k_mvbr4 Q4_K, k_mvbr6 Q6_K)"}


GEO_7B = dict(hidden=4096, ffn=11008, n_heads=32, n_kv_heads=8, head_dim=128, vocab=32000)
GEO_70B = dict(hidden=8192, ffn=28672, n_heads=64, n_kv_heads=8, head_dim=128, vocab=32000)


def bench_decode(dev, host, n_tokens, path="both", geo=GEO_7B, n_layers=32, ctx=2048,
                 n_dispatch_tokens=16, batch=0, batch_tokens=16, seed=SEED):
    """Greedy decode of a Q4_K_M synthetic Llama model (config 4: 7B, 32 layers,
    ctx 2048; config 5: 70B, 80 layers, ctx 8192) from position `ctx` with the
    KV cache prefilled N(0,1): the graph decoder (one graph launch per token)
    and, for comparison, the per-dispatch ops-table path."""
    n_dispatch_tokens = min(n_dispatch_tokens, n_tokens)
    t_build = time.perf_counter()
    steps = max(n_tokens, batch_tokens if batch else 0)  # the cache covers both runs
    model = V.SynthModel(host, n_layers=n_layers, **geo, max_ctx=ctx + steps + 1, seed=seed)
    kc, vc = model.kv_prefill(host, ctx)
    be = V.gfx950_backend()
    if not be.init():
        raise RuntimeError(be.last_error())
    d = V.Decoder(host, be, model)
    d.load_kv(kc, vc, ctx)
    t_build = time.perf_counter() - t_build
    # per-dispatch path (src/vbs_specializer.c order through the ops table)
    d.greedy(1, ctx, min(2, n_tokens))
    t0 = time.perf_counter()
    dtoks, dmargins = d.greedy(1, ctx, n_dispatch_tokens)
    dt_dispatch = time.perf_counter() - t0
    dispatches = d.dispatch_count()
    dispatch = {"tokens_per_s": round(n_dispatch_tokens / dt_dispatch, 2),
                "dispatches_per_token": dispatches,
                "path": "g_vbs_hip_backend ops table, one dispatch per bridge call"}
    if path == "dispatch":
        d.close()
        return {"dispatch_path": dispatch, "first_tokens": [int(x) for x in dtoks[:8]],
                "min_margin": float(np.min(dmargins))}
    # graph decoder over the same device weights and cache
    eager = path == "eager"
    g = V.GraphDecoder(dev, d, max_steps=n_tokens)
    g.greedy(1, ctx, min(2, n_tokens), eager)
    dev.sync()
    t0 = time.perf_counter()
    toks, margins = g.greedy(1, ctx, n_tokens, eager)
    dt = time.perf_counter() - t0
    g.close()
    batched = None
    if batch:
        batched = bench_batch_decode(dev, d, model, kc, vc, ctx, batch, batch_tokens, eager)
    del kc, vc
    d.close()
    wbytes = model.weight_bytes() - model.tok_embd.nbytes
    kvd = model.cfg["n_kv_heads"] * model.cfg["head_dim"]
    kv_bytes = sum(n_layers * (ctx + i + 1) * kvd * 2 * 2 for i in range(n_tokens)) / n_tokens
    return {"tokens_per_s": round(n_tokens / dt, 2), "ms_per_token": round(1e3 * dt / n_tokens, 3),
            "n_tokens": n_tokens, "context": ctx, "n_layers": n_layers,
            "hidden": geo["hidden"], "ffn": geo["ffn"], "heads": [geo["n_heads"], geo["n_kv_heads"]],
            "model_build_upload_s": round(t_build, 1),
            "bytes_per_token": int(wbytes + kv_bytes),
            "roofline_frac": round((wbytes + kv_bytes) / (dt / n_tokens) / (PEAK_HBM_GBS * 1e9), 4),
            "path": ("vbs_gfx950_decoder kernels launched one by one" if eager else
                     "vbs_gfx950_decoder: one HIP graph launch per token"),
            "dispatch_path": dispatch,
            "paths_agree": bool(np.array_equal(toks[:n_dispatch_tokens], dtoks)),
            "first_tokens": [int(x) for x in toks[:8]],
            "min_margin": float(np.min(margins)),
            "_tokens": toks, "_margins": margins,
            **({"batch_decode": batched} if batched else {})}


def host_cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            return next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        return ""


def decode_vs_checkers(host, toks, margins, n_oracle=4, ctx=2048):
    """Checker and CPU-baseline leg of the config-4 decode (graph decoder,
    seed DECODE_SEED, token 1 at position `ctx`): its tokens and top-1 minus
    top-2 margins against the reference CPU backend's 128 (the fixture), its
    first `n_oracle` tokens against the oracle's forward pass, run here on the
    host's cores over a fresh copy of the same synthetic model; and beside the
    GPU rate, the same decode on the CPU: one full token of the reference's
    own CPU backend (oracle/_ref, single-threaded as the reference is) driven
    through its ops table by host/vbs_decode.c in the bridge's order, and the
    oracle's forward pass on every host core (`cpu_baseline`)."""
    from oracle_lib import REF_SO, Oracle
    out = {}
    if os.path.exists(DECODE_FIXTURE):
        fx = np.load(DECODE_FIXTURE)
        n = min(len(toks), len(fx["tokens"]))
        want_m = fx["top2"][:n, 0].astype(np.float64) - fx["top2"][:n, 1]
        out["reference_tokens_compared"] = n
        out["reference_tokens_equal"] = bool(np.array_equal(toks[:n], fx["tokens"][:n]))
        out["max_abs_margin_diff"] = float(np.abs(np.asarray(margins[:n]) - want_m).max())
    t0 = time.perf_counter()
    model = V.SynthModel(host, n_layers=32, **GEO_7B, max_ctx=ctx + n_oracle + 1,
                         seed=DECODE_SEED)
    kc_p, vc_p = model.kv_prefill(host, ctx)
    ref_leg = None
    if os.path.exists(REF_SO):
        ref = V.Backend(C.CDLL(REF_SO), "g_vbs_cpu_backend")
        ref.init()
        d = V.Decoder(host, ref, model)
        d.load_kv(kc_p, vc_p, ctx)
        t1 = time.perf_counter()
        lg = d.step(1, ctx)
        ref_leg = (time.perf_counter() - t1, int(np.argmax(lg)))
        d.close()
    kvd = GEO_7B["n_kv_heads"] * GEO_7B["head_dim"]
    shape = (32, ctx + n_oracle + 1, kvd)
    kc, vc = np.zeros(shape, np.uint16), np.zeros(shape, np.uint16)
    kc[:, :ctx], vc[:, :ctx] = kc_p.reshape(32, ctx, kvd), vc_p.reshape(32, ctx, kvd)
    del kc_p, vc_p
    orc = Oracle()
    om = orc.model(model, kc, vc)
    threads, tok, want, t_fwd = min(16, os.cpu_count() or 1), 1, [], 0.0
    for i in range(n_oracle):
        t1 = time.perf_counter()
        lg = orc.forward(om, tok, ctx + i, GEO_7B["vocab"], threads)
        t_fwd += time.perf_counter() - t1
        tok = int(np.argmax(lg))
        want.append(tok)
    out["oracle_tokens_compared"] = n_oracle
    out["oracle_agree"] = bool(np.array_equal(np.asarray(toks[:n_oracle]), want))
    out["oracle_s"] = round(time.perf_counter() - t0, 1)
    cpu = host_cpu_model()
    all_cores = {"tokens_per_s": round(n_oracle / t_fwd, 4), "unit": "tokens/s",
                 "cores": threads, "kind": "port", "cpu": cpu,
                 "sample": f"{n_oracle} greedy tokens from position {ctx} of the same model, "
                           f"the oracle's forward pass row-parallel on {threads} threads "
                           f"({t_fwd:.1f} s of forward passes; model build excluded)"}
    if ref_leg is not None:
        sec, ref_tok = ref_leg
        out["cpu_baseline"] = {
            "tokens_per_s": round(1.0 / sec, 5), "unit": "tokens/s", "cores": 1,
            "kind": "reference", "cpu": cpu, "nproc": os.cpu_count(),
            "first_token_equal": ref_tok == int(toks[0]),
            "sample": f"1 full token (token 1 at position {ctx}, 32 layers, lm_head) of the "
                      f"config-4 model through the reference CPU backend's ops table "
                      f"(oracle/_ref/libvbs_ref.so), single thread, driven by "
                      f"host/vbs_decode.c in the bridge's order: {sec:.1f} s",
            "all_cores": all_cores}
    else:
        out["cpu_baseline"] = all_cores
    return out


def bench_batch_decode(dev, d, model, kc, vc, ctx, batch, n_tokens, eager=False):
    """Greedy decode of `batch` sequences at once (vbs_gfx950_bdecoder, one
    HIP graph per step) over the same device weights: every sequence's own
    cache holds the same N(0,1) prefill to `ctx`, the start tokens differ."""
    c = model.cfg
    bd = V.BatchDecoder(dev, d, batch, max_steps=n_tokens)
    for b in range(batch):
        bd.load_kv(b, kc, vc, ctx)
    tok0, pos0 = [1 + 7 * b for b in range(batch)], [ctx] * batch
    bd.greedy(tok0, pos0, 2, eager)
    dev.sync()
    t0 = time.perf_counter()
    toks, margins = bd.greedy(tok0, pos0, n_tokens, eager)
    dt = time.perf_counter() - t0
    bd.close()
    kvd = c["n_kv_heads"] * c["head_dim"]
    wbytes = model.weight_bytes() - model.tok_embd.nbytes
    kv_bytes = batch * sum(c["n_layers"] * (ctx + i + 1) * kvd * 2 * 2
                           for i in range(n_tokens)) / n_tokens
    step_s = dt / n_tokens
    return {"batch": batch, "tokens_per_s": round(batch * n_tokens / dt, 2),
            "ms_per_step": round(1e3 * step_s, 3), "steps": n_tokens,
            "bytes_per_step": int(wbytes + kv_bytes),
            "roofline_frac": round((wbytes + kv_bytes) / step_s / (PEAK_HBM_GBS * 1e9), 4),
            "path": ("vbs_gfx950_bdecoder kernels launched one by one" if eager else
                     "vbs_gfx950_bdecoder: one HIP graph launch per step of all sequences"),
            "first_tokens_seq0": [int(x) for x in toks[:8, 0]],
            "min_margin": float(np.min(margins))}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--ncopy", type=int, default=4)
    ap.add_argument("--roof-reps", type=int, default=50)
    ap.add_argument("--decode-tokens", type=int, default=128)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip configs 1 (Q4_0), 2 (the Q8_0 layer set) and 3 (the Q6_K head)")
    ap.add_argument("--no-batch8", action="store_true",
                    help="skip the config 5 batch-8 layer matvec set")
    ap.add_argument("--decode-70b-tokens", type=int, default=32,
                    help="greedy tokens of the 70B-shaped model (config 5, batch 1); 0 skips it")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first copy this many MiB device-to-device once (a known-size "
                         "transfer that scales HBM byte counters)")
    ap.add_argument("--decode-path", choices=("both", "dispatch", "eager"), default="both",
                    help="'dispatch' times only the per-dispatch ops-table decode; 'eager' "
                         "runs the graph decoder's kernels without the graph (for kernel "
                         "tracers)")
    ap.add_argument("--decode-geometry", choices=("7b", "70b"), default="7b",
                    help="model of the 'decode' entry: 7B (config 4) or 70B with its batch-8 "
                         "run (config 5); the default run adds 'decode_70b' anyway")
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print(json.dumps({"error": "this build drives exactly one GPU (one process, one device); "
                                   "run with --gpus 1"}))
        sys.exit(2)
    dev = V.DeviceLib()
    if not dev.init():
        raise SystemExit(f"gfx950 device unavailable: {dev.error()}")
    host = V.load_host()
    if a.copy_probe_mib:
        n = a.copy_probe_mib << 20
        src, dst = dev.alloc(n), dev.alloc(n)
        dev.check(dev._copy_d2d(dst, src, n), "copy probe")
        dev.sync()
        dev.free(src)
        dev.free(dst)
    r = bench_matvec(dev, host, a.steps, a.warmup, a.ncopy, a.roof_reps)
    value = r["step_bytes"] * a.steps / r["wall_s"] / 1e9
    achieved = r["big_bytes"] / (r["avg_big_ms"] * 1e-3) / 1e9
    rep = r["rep_big_ms"]
    out = {
        "metric": "Q4_K matvec HBM GB/s (% of peak); decode tokens/sec at 7B Q4_K_M, 1 GPU",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(1e3 * r["wall_s"] / a.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k", "data": "synthetic",
        "config": {"workload": "Llama-7B layer matvec set, Q4_K, batch 1 (config 2)",
                   "shapes": [[n, r, c] for n, r, c in LAYER_SET], "weight_copies": a.ncopy,
                   "rotating_bytes": a.ncopy * sum(V.row_bytes(V.Q4_K, c) * r
                                                   for _, r, c in LAYER_SET),
                   "issue": "one HIP graph of the 7 launches per step"},
        "pct_of_peak": round(100 * value / PEAK_HBM_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": TRAFFIC_BYTES,
                     "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, scaled by a "
                                       "256 MiB copy (profiles/q4k_matvec_7b_layer_set.md)",
                     "kernel": "Q4_K matvec: k_mvl (whole row range in flight) at 11008x4096, k_mvf at 4096x11008",
                     "algorithmic_bytes_per_launch": r["big_bytes"],
                     "avg_launch_us": round(1e3 * r["avg_big_ms"], 3),
                     "ceiling": r["ceiling"],
                     "frac_of_read_floor": round(r["ceiling"]["read_floor"]["us_per_launch"]
                                                 / (1e3 * r["avg_big_ms"]), 4),
                     "per_replay_GB_per_s": {
                         "median": round(r["big_bytes"] / (rep[len(rep) // 2] * 1e-3) / 1e9, 1),
                         "min": round(r["big_bytes"] / (rep[-1] * 1e-3) / 1e9, 1),
                         "max": round(r["big_bytes"] / (rep[0] * 1e-3) / 1e9, 1),
                         "replays": len(rep)}},
        "gpu_event_ms_per_step": round(r["gpu_ms"] / a.steps, 4),
        "graph_replay_equals_eager": r["replay_equals_eager"],
    }
    cpu_work = None if a.no_cpu else {}
    if not a.no_configs:
        out["configs"] = bench_configs(dev, host, cpu_work)
        out["hot_table"] = bench_hot_table(dev, host, cpu_work)
        out["weight_streaming"] = bench_weight_streaming(dev, host)
    if not a.no_batch8:
        out["batch8_70b"] = bench_batch8_70b(dev, host)
    if not a.no_decode and a.decode_geometry == "70b":
        out["decode"] = bench_decode(dev, host, a.decode_tokens, a.decode_path, geo=GEO_70B,
                                     n_layers=80, ctx=8192, n_dispatch_tokens=4, batch=8,
                                     batch_tokens=a.decode_tokens)
    elif not a.no_decode:
        out["decode"] = bench_decode(dev, host, a.decode_tokens, a.decode_path, seed=DECODE_SEED)
        if a.decode_70b_tokens and a.decode_path == "both":
            out["decode_70b"] = bench_decode(dev, host, a.decode_70b_tokens, geo=GEO_70B,
                                             n_layers=80, ctx=8192, n_dispatch_tokens=4,
                                             batch=8, batch_tokens=16)
    dec = out.get("decode", {})
    toks, margins = dec.pop("_tokens", None), dec.pop("_margins", None)
    out.get("decode_70b", {}).pop("_tokens", None)
    out.get("decode_70b", {}).pop("_margins", None)
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(host, r["weights_host"], r["xs_host"], beside=cpu_work)
        if toks is not None and a.decode_geometry == "7b" and "tokens_per_s" in dec:
            checked = decode_vs_checkers(host, toks, margins)
            dec["cpu_baseline"] = checked.pop("cpu_baseline", None)
            dec["checked"] = checked
    print(json.dumps(out))


if __name__ == "__main__":
    main()
