"""The drop-in boundary: g_vbs_hip_backend (host/vbs_backend_gfx950.c) and the
C ABI of libvbs_gfx950.so (include/vbs_gfx950.h).

CPU tests load private copies of the shim so that each one runs its own
init() (the shim probes once per process, as src/vbs_backend_hip.c:150-151
does) and point it with VBS_GFX950_LIB at a test-only mock device library
(tests/mock/mock_gfx950.c, built here over the CPU oracle) or at variants of it
with a wrong ABI version or a missing entry point. The GPU test runs the same
suite against the real library.
"""
import ctypes as C
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import vbs_gfx950 as V
from backend_suite import run_linear_batch, run_suite
from oracle_lib import Oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MOCK_SRC = os.path.join(ROOT, "tests", "mock", "mock_gfx950.c")
ORACLE_SRC = os.path.join(ROOT, "oracle", "vbs_oracle.c")


def build_mock(outdir, name, defines=()):
    so = os.path.join(outdir, name)
    cmd = ["gcc", "-std=c11", "-O2", "-fPIC", "-shared", "-ffp-contract=off",
           "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "oracle"),
           *[f"-D{d}" for d in defines], MOCK_SRC, ORACLE_SRC, "-o", so, "-lm", "-lpthread"]
    subprocess.run(cmd, check=True)
    return so


def fresh_shim(outdir, device_lib):
    """A private copy of the shim whose init() will load `device_lib`."""
    copy = os.path.join(outdir, f"shim_{len(os.listdir(outdir))}.so")
    shutil.copy(V.HOST_LIB, copy)
    old = os.environ.get("VBS_GFX950_LIB")
    if device_lib is None:
        os.environ.pop("VBS_GFX950_LIB", None)
    else:
        os.environ["VBS_GFX950_LIB"] = device_lib
    be = V.Backend(C.CDLL(copy), "g_vbs_hip_backend", "vbs_hip_last_error")
    ok = be.init()
    if old is None:
        os.environ.pop("VBS_GFX950_LIB", None)
    else:
        os.environ["VBS_GFX950_LIB"] = old
    return be, ok


@pytest.fixture(scope="module")
def tmpdir_mod(tmp_path_factory):
    return str(tmp_path_factory.mktemp("shim"))


def test_device_library_exports_every_declared_symbol():
    """Every function declared in include/vbs_gfx950.h is exported by the
    built library (loaded without touching a GPU)."""
    hdr = open(os.path.join(ROOT, "include", "vbs_gfx950.h")).read()
    declared = sorted(set(re.findall(r"\b(vbs_gfx950_\w+)\s*\(", hdr)))
    assert len(declared) >= 25
    lib = C.CDLL(V.DEVICE_LIB)
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(V.DEVICE_SYMBOLS)


def test_shim_exports_the_reference_symbols():
    lib = C.CDLL(V.HOST_LIB)
    ops = V.VbsOps.in_dll(lib, "g_vbs_hip_backend")
    assert C.sizeof(V.VbsOps) == 14 * C.sizeof(C.c_void_p)
    for name, _ in V.VbsOps._fields_[:-1]:
        assert getattr(ops, name), name
    assert not ops.launch_persistent_kernel  # must be NULL (include/vbs_backend.h:94-98)
    assert hasattr(lib, "vbs_hip_last_error")
    # the batched extension's entry points (include/vbs_hip_batch.h)
    hdr = open(os.path.join(ROOT, "include", "vbs_hip_batch.h")).read()
    declared = sorted(set(re.findall(r"\b(vbs_hip_\w+)\s*\(", hdr)) - {"vbs_hip_last_error"})
    assert declared == ["vbs_hip_dispatch_linear_batch", "vbs_hip_linear_batch_version"]
    for name in declared:
        assert hasattr(lib, name), name
    # the dispatch trace's (include/vbs_hip_trace.h)
    hdr = open(os.path.join(ROOT, "include", "vbs_hip_trace.h")).read()
    declared = sorted(set(re.findall(r"\b(vbs_hip_trace_\w+)\s*\(", hdr)))
    assert declared == ["vbs_hip_trace_counters", "vbs_hip_trace_level", "vbs_hip_trace_reset"]
    for name in declared:
        assert hasattr(lib, name), name


@pytest.mark.skipif(not os.path.isdir("/root/reference/include"),
                    reason="reference headers not mounted")
def test_abi_layout_matches_reference_headers(tmp_path):
    """sizeof/offsetof of every boundary struct and the enum values agree
    between include/vbs_abi.h and the reference's own headers."""
    probe = r'''
#include <stdio.h>
#include <stddef.h>
#include HDR
int main(void) {
  printf("%zu %zu %zu %zu %zu\n", sizeof(vbs_device_t), sizeof(vbs_buffer_t), sizeof(vbs_arg_t),
         sizeof(vbs_prim_pipeline_t), sizeof(vbs_backend_ops_t));
  printf("%zu %zu %zu %zu\n", offsetof(vbs_device_t, max_working_set_bytes),
         offsetof(vbs_device_t, internal_handle), offsetof(vbs_buffer_t, device),
         offsetof(vbs_arg_t, size));
  printf("%zu %zu %zu\n", offsetof(vbs_backend_ops_t, dispatch_linear_tile),
         offsetof(vbs_backend_ops_t, synchronize_device), offsetof(vbs_backend_ops_t, launch_persistent_kernel));
  printf("%d %d %d %d %d %d\n", VBS_GGML_TYPE_Q4_K, VBS_GGML_TYPE_Q6_K, VBS_GGML_TYPE_LNS8,
         VBS_OP_CACHE, VBS_OP_PROJECTION, VBS_BACKEND_HIP);
  return 0;
}
'''
    src = tmp_path / "probe.c"
    src.write_text(probe)
    outs = []
    for hdr, inc in (('"vbs_abi.h"', os.path.join(ROOT, "include")),
                     ('"vbs_backend.h"', "/root/reference/include")):
        exe = tmp_path / f"probe{len(outs)}"
        subprocess.run(["gcc", "-std=c11", "-D_GNU_SOURCE", f"-DHDR={hdr}", "-I" + inc,
                        str(src), "-o", str(exe)], check=True)
        outs.append(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout)
    assert outs[0] == outs[1]


def test_shim_without_gpu_reports_reason(tmpdir_mod):
    """Init fails with a reason when no gfx950 is visible (this container),
    so backend selection falls through to the CPU (vbs_backend_select.c:42-58)."""
    probe = V.DeviceLib()
    if probe.init():
        pytest.skip("a GPU is visible here")
    be, ok = fresh_shim(tmpdir_mod, V.DEVICE_LIB)
    assert not ok
    assert "gfx950 init" in be.last_error() and ("GPU" in be.last_error() or "gfx950" in be.last_error())
    assert be.ops.get_device_count() == 0


def test_shim_rejects_wrong_abi_version(tmpdir_mod):
    so = build_mock(tmpdir_mod, "mock_badabi.so", ["MOCK_ABI=999"])
    be, ok = fresh_shim(tmpdir_mod, so)
    assert not ok and "ABI version 999" in be.last_error()


def test_shim_rejects_library_missing_an_entry_point(tmpdir_mod):
    so = build_mock(tmpdir_mod, "mock_noadd.so", ["MOCK_DROP_ADD"])
    be, ok = fresh_shim(tmpdir_mod, so)
    assert not ok and "lacks vbs_gfx950_add" in be.last_error()


def test_shim_rejects_missing_library(tmpdir_mod):
    be, ok = fresh_shim(tmpdir_mod, os.path.join(tmpdir_mod, "does_not_exist.so"))
    assert not ok and "cannot load" in be.last_error()


def test_backend_suite_through_shim_on_host_mock(tmpdir_mod, host):
    """The restated reference self-test, through the shim's ops table, with
    the device library replaced by the host mock: checks the argument
    marshalling, both linear conventions, offsets/accumulate and refusals."""
    so = build_mock(tmpdir_mod, "mock_ok.so")
    be, ok = fresh_shim(tmpdir_mod, so)
    assert ok, be.last_error()
    dev = be.ops.get_device(0).contents
    assert dev.type == 2 and dev.max_working_set_bytes == 1 << 30 and b"mock" in dev.name
    res = run_suite(be, Oracle(), host)
    bad = [r[0] for r in res if not r[1]]
    assert not bad, bad
    assert len(res) >= 33


HELD_CASES = {
    # model mix, mock built to decline the grouped launches, expected joins
    # per step and layer: [RMSNorm, RoPE, add, SiLU, cache, grouped q/k/v,
    # grouped gate/up] as (per-layer count, once per step)
    "q4k_m": (None, False, [(0, 1), (0, 0), (2, 0), (0, 0), (0, 0), (1, 0), (1, 0)]),
    "q4k_m_groups_declined": (None, True, [(2, 1), (2, 0), (2, 0), (1, 0), (1, 0), (0, 0), (0, 0)]),
    "v_up_q6k": ({"v": V.Q6_K, "up": V.Q6_K}, False,
                 [(2, 1), (2, 0), (2, 0), (1, 0), (1, 0), (0, 0), (0, 0)]),
    "q8_0": ({r: V.Q8_0 for r in ("q", "k", "v", "o", "gate", "up", "down", "embd", "head")},
             False, [(0, 0)] * 7),
}


@pytest.mark.parametrize("case", list(HELD_CASES))
def test_held_ops_on_host_mock_keep_the_bridge_results(tmpdir_mod, host, case):
    """The shim holds back the bridge's NORMALIZE, q, ROTARY, k, ROTARY, v,
    CACHE run and its NORMALIZE, gate, up, ACTIVATION run and issues each as
    one grouped launch (vbs_gfx950_qkv_fused, vbs_gfx950_gate_up_fused), and
    otherwise joins a held LINEAR with its neighbours (RMSNorm + matvec,
    matvec + RoPE, + add, + SiLU gate, + K/V store) when
    vbs_gfx950_linear_fused takes them. Over the host mock (whose fused
    entries compose the oracle's ops and decline every type but Q4_K and
    Q6_K, so the Q8_0 model runs the ops one by one) the bridge-order decode
    driver's logits equal the oracle's forward pass bit for bit at every
    step, and the launches happened as expected: grouped for the Q4_K_M mix;
    pairwise where the mock declines the groups or the v and up matrices
    differ in type from q and gate."""
    from test_decode import TINY, full_cache
    mix_d, decline, want = HELD_CASES[case]
    so = build_mock(tmpdir_mod, f"mock_fuse_{case}.so",
                    ("MOCK_DECLINE_GROUPS",) if decline else ())
    be, ok = fresh_shim(tmpdir_mod, so)
    assert ok, be.last_error()
    mock = C.CDLL(so)
    mock.mock_fused_count.restype = C.c_uint
    if mix_d is not None:
        mix_d = {**V.Q4_K_M_MIX, **mix_d}
    model = V.SynthModel(host, **TINY, seed=99, mix=mix_d)
    d = V.Decoder(host, be, model)
    orc = Oracle()
    kc, vc = full_cache(model, None, None, 0)
    om = orc.model(model, kc, vc)
    before = [mock.mock_fused_count(i) for i in range(7)]
    tok, steps = 1, 6
    for pos in range(steps):
        got = d.step(tok, pos)
        want_logits = orc.forward(om, tok, pos, model.cfg["vocab"], 1)
        assert np.array_equal(got.view(np.uint32), want_logits.view(np.uint32)), pos
        tok = int(np.argmax(want_logits))
    d.close()
    joined = [mock.mock_fused_count(i) - before[i] for i in range(7)]
    L = TINY["n_layers"]
    assert joined == [steps * (per * L + once) for per, once in want], joined


class TraceCounter(C.Structure):
    _fields_ = [("calls", C.c_uint64), ("launches", C.c_uint64), ("ns", C.c_uint64)]


TRACE_KINDS = ["embedding", "normalize", "rotary", "cache", "attention", "activation",
               "elementwise", "linear", "linear_batch", "linear_joined", "qkv_group", "ffn_group"]


def test_dispatch_trace_counts_calls_and_launches(tmpdir_mod, host, tmp_path):
    """VBS_TRACE=2 (include/vbs_hip_trace.h): over the host mock, two decode
    steps of the Q4_K_M model count every table call by op kind and every
    launch by launch kind — per layer the grouped q/k/v and gate/up
    launches, the two matvec + add launches and the attention; per step the
    embedding and the RMSNorm + lm_head launch — each launch timed and
    written as one line of $VBS_TRACE_FILE. The logits are the oracle's, as
    without the trace."""
    from test_decode import TINY, full_cache
    so = build_mock(tmpdir_mod, "mock_trace.so")
    log = tmp_path / "trace.log"
    os.environ["VBS_TRACE"], os.environ["VBS_TRACE_FILE"] = "2", str(log)
    try:
        be, ok = fresh_shim(tmpdir_mod, so)
    finally:
        del os.environ["VBS_TRACE"], os.environ["VBS_TRACE_FILE"]
    assert ok, be.last_error()
    assert be.lib.vbs_hip_trace_level() == 2
    be.lib.vbs_hip_trace_reset()
    model = V.SynthModel(host, **TINY, seed=5)
    d = V.Decoder(host, be, model)
    orc = Oracle()
    kc, vc = full_cache(model, None, None, 0)  # (the oracle model writes into these)
    om = orc.model(model, kc, vc)
    steps, L = 2, TINY["n_layers"]
    for pos in range(steps):
        got = d.step(3 + pos, pos)
        want = orc.forward(om, 3 + pos, pos, model.cfg["vocab"], 1)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), pos
    d.close()
    tc = (TraceCounter * len(TRACE_KINDS))()
    be.lib.vbs_hip_trace_counters(tc)
    got = {k: (tc[i].calls, tc[i].launches) for i, k in enumerate(TRACE_KINDS)}
    want = {"embedding": (1, 1), "normalize": (2 * L + 1, 0), "rotary": (2 * L, 0),
            "cache": (L, 0), "attention": (L, L), "activation": (L, 0), "elementwise": (2 * L, 0),
            "linear": (7 * L + 1, 0), "linear_batch": (0, 0), "linear_joined": (0, 2 * L + 1),
            "qkv_group": (0, L), "ffn_group": (0, L)}
    assert got == {k: (steps * c, steps * n) for k, (c, n) in want.items()}, got
    assert all(tc[i].ns > 0 for i in range(len(TRACE_KINDS)) if tc[i].launches)
    lines = log.read_text().splitlines()
    assert len(lines) == sum(tc[i].launches for i in range(len(TRACE_KINDS)))
    assert all(ln.startswith("vbs_trace ") and ln.endswith(" us") for ln in lines)
    assert any(ln.startswith("vbs_trace qkv_group Q4_K") for ln in lines), lines[:8]


def test_held_ops_random_sequences_equal_ops_one_by_one(tmpdir_mod, host):
    """Random op sequences over a small pool of buffers — bridge-like q/k/v
    and gate/up runs with randomly chosen (often aliasing) buffers, a linear
    with the op after it, and single NORMALIZE, LINEAR, ROTARY, CACHE,
    ACTIVATION and ELEMENTWISE ops and read-backs — through two shims over
    the host mock (one whose fused and grouped entries run, one built to
    decline them all, so that the shim's fallbacks run) and, as the
    reference, through the oracle's ops one at a time on host arrays. Every
    buffer and both caches must agree bit for bit after every sequence: a
    difference is the held-op logic reordering, dropping or mis-joining an
    op (the mock's entries also expose aliasing inside one launch)."""
    n_buf, dim, hd, mc, layers = 6, 512, 64, 16, 2
    so_f = build_mock(tmpdir_mod, "mock_rand_fused.so")
    so_s = build_mock(tmpdir_mod, "mock_rand_single.so", ("MOCK_DECLINE_FUSED",))
    shims = [fresh_shim(tmpdir_mod, so) for so in (so_f, so_s)]
    for be, ok in shims:
        assert ok, be.last_error()
    orc = Oracle()
    mats = {r: V.synth_matrix(host, V.Q4_K, r, dim, 77, 200 + r) for r in (512, 256)}
    rng = np.random.default_rng(4242)
    A = V.Backend.buf_arg
    norm_w = rng.standard_normal(dim).astype(np.float32)
    states = []
    for be, _ in shims:
        dev = be.device()
        st = {"be": be, "dev": dev, "keep": [],
              "bufs": [be.upload(np.zeros(dim, np.float32)) for _ in range(n_buf)],
              "norm_w": be.upload(norm_w),
              "kc": be.upload(np.zeros(layers * mc * dim, np.uint16)),
              "vc": be.upload(np.zeros(layers * mc * dim, np.uint16)),
              "w": {r: be.upload(m) for r, m in mats.items()},
              "lin": be.ops.compile_linear_pipeline(dev, V.Q4_K, None, 0),
              "prim": {k: be.ops.compile_primitive_pipeline(dev, k, None, 0) for k in (
                  V.OP_NORMALIZE, V.OP_ROTARY, V.OP_CACHE, V.OP_ACTIVATION, V.OP_ELEMENTWISE)}}
        states.append(st)
    ref = {"kc": np.zeros(layers * mc * dim, np.uint16),
           "vc": np.zeros(layers * mc * dim, np.uint16)}

    def run_ref(op):
        b = ref["bufs"]
        kind = op[0]
        if kind == "read":
            return b[op[1]].copy()
        if kind == "lin":
            _, r, i, o = op
            b[o][:r] = orc.linear(V.Q4_K, mats[r], b[i], dim, r, threads=1)
        elif kind == "norm":
            _, i, o = op
            b[o][:] = orc.rms_norm(b[i], norm_w, 1e-5)
        elif kind == "rope":
            _, i, pos, nh, theta = op
            b[i][:nh * hd] = orc.rope(b[i][:nh * hd], pos, hd, nh, theta)
        elif kind == "cache":
            _, k, v, pos, layer, kvd = op
            orc.cache_store(np.ascontiguousarray(b[k][:kvd]), np.ascontiguousarray(b[v][:kvd]),
                            ref["kc"], ref["vc"], pos, layer, mc, kvd)
        elif kind == "act":
            _, g, u, o, n = op
            b[o][:n] = orc.silu_mul(b[g][:n].copy(), b[u][:n].copy())
        else:
            _, a_, b_, o, n = op
            b[o][:n] = orc.add(b[a_][:n].copy(), b[b_][:n].copy())
        return True

    def run(st, op):
        be, keep, b = st["be"], st["keep"], st["bufs"]
        U = lambda v: be.u32_arg(keep, v)
        F = lambda v: be.f32_arg(keep, v)
        kind = op[0]
        if kind == "read":
            return be.download(b[op[1]], dim, np.float32)
        if kind == "lin":
            _, r, i, o = op
            return bool(be.ops.dispatch_linear_tile(st["dev"], st["lin"], st["w"][r], None, 0, b[i],
                                                    b[o], dim, r, 0, 0, False))
        if kind == "norm":
            _, i, o = op
            args = [A(b[i]), A(st["norm_w"]), A(b[o]), U(dim), F(1e-5)]
        elif kind == "rope":
            _, i, pos, nh, theta = op
            args = [A(b[i]), U(pos), U(hd), U(nh), F(theta)]
        elif kind == "cache":
            _, k, v, pos, layer, kvd = op
            args = [A(b[k]), A(b[v]), A(st["kc"]), A(st["vc"]), U(pos), U(layer), U(mc), U(kvd)]
        elif kind == "act":
            _, g, u, o, n = op
            args = [A(b[g]), A(b[u]), A(b[o]), U(n)]
        else:  # add
            _, a_, b_, o, n = op
            args = [A(b[a_]), A(b[b_]), A(b[o]), U(n)]
        pk = {"norm": V.OP_NORMALIZE, "rope": V.OP_ROTARY, "cache": V.OP_CACHE,
              "act": V.OP_ACTIVATION, "add": V.OP_ELEMENTWISE}[kind]
        return be.dispatch(st["prim"][pk], args)

    def pick(k=1):
        return [int(v) for v in rng.integers(0, n_buf, k)]

    def pick_run(k):  # distinct buffers (a bridge-like run) or, now and then, any
        return [int(v) for v in rng.choice(n_buf, k, replace=False)] if rng.random() < 0.7 \
            else pick(k)

    def no_inplace_lin(ops):
        # (a linear whose output is its input is left out: its result depends
        # on the order in which an implementation writes rows; the bridge
        # never issues one)
        return [("lin", op[1], op[2], (op[3] + 1) % n_buf if op[3] == op[2] else op[3])
                if op[0] == "lin" else op for op in ops]

    def sequence():
        # (short, with a fresh cache row per block, so that a wrong value is
        # seldom overwritten before the buffers are compared)
        ops = []
        for _ in range(int(rng.integers(1, 4))):
            pos, layer = int(rng.integers(0, mc)), int(rng.integers(0, layers))
            c = rng.random()
            if c < 0.3:    # a q/k/v run: norm, q, rope, k, rope, v, cache
                x, n_, q, k, v = pick_run(5)
                kvr = int(rng.choice([256, 512]))
                # (now and then the k rope or the cache at another position or base)
                pk = pos if rng.random() < 0.85 else (pos + 1) % mc
                c3 = rng.random()
                pc = pos if c3 < 0.8 else pk if c3 < 0.9 else (pos + 3) % mc
                tk = 10000.0 if rng.random() < 0.85 else 500000.0
                xv = n_ if rng.random() < 0.9 else x  # (now and then v reads another vector)
                ops += [("norm", x, n_), ("lin", 512, n_, q), ("rope", q, pos, 512 // hd, 10000.0),
                        ("lin", kvr, n_, k), ("rope", k, pk, kvr // hd, tk), ("lin", kvr, xv, v),
                        ("cache", k, v, pc, layer, kvr)]
            elif c < 0.55:  # a gate/up run
                x, n_, g, u, h = pick_run(5)
                r = int(rng.choice([256, 512]))
                xu = n_ if rng.random() < 0.9 else x  # (now and then up reads another vector)
                ops += [("norm", x, n_), ("lin", r, n_, g), ("lin", r, xu, u), ("act", g, u, h, r)]
            elif c < 0.7:   # a linear and the op after it
                i, o, s_, h = pick(4)
                r = int(rng.choice([256, 512]))
                c2 = rng.random()
                ops += [("lin", r, i, o), ("add", s_, o, s_, r) if c2 < 0.3 else
                        ("cache", s_, o, pos, layer, r) if c2 < 0.55 else
                        ("act", s_, o, h, r) if c2 < 0.8 else ("rope", o, pos, r // hd, 10000.0)]
                if c2 >= 0.8 and rng.random() < 0.5:  # a second rotation of the same rows
                    ops.append(("rope", o, (pos + 1) % mc, r // hd, 10000.0))
            else:           # single ops
                c2 = rng.random()
                i, o, a_, r = *pick(3), int(rng.choice([256, 512]))
                ops.append(("norm", i, o) if c2 < 0.2 else ("lin", r, i, o) if c2 < 0.45 else
                           ("rope", i, pos, r // hd, 10000.0) if c2 < 0.6 else
                           ("cache", i, o, pos, layer, r) if c2 < 0.7 else
                           ("act", i, o, a_, r) if c2 < 0.8 else ("add", i, o, a_, r) if c2 < 0.9
                           else ("read", i))
        return ops

    finite = 0
    for seq_no in range(300):
        # fresh values each sequence (chained matvecs would grow to inf / NaN,
        # which then hides every difference)
        fresh = [rng.standard_normal(dim).astype(np.float32) for _ in range(n_buf)]
        ref["bufs"] = [f.copy() for f in fresh]
        for st in states:
            for buf_, val in zip(st["bufs"], fresh):
                assert st["be"].ops.copy_to_device(buf_, val.ctypes.data, val.nbytes)
        for op in no_inplace_lin(sequence()):
            want = run_ref(op)
            for n_st, st in enumerate(states):
                got = run(st, op)
                if op[0] == "read":
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
                        (seq_no, n_st, op)
                else:
                    assert got, (seq_no, n_st, op, st["be"].last_error())
        for i in range(n_buf):
            for n_st, st in enumerate(states):
                a = st["be"].download(st["bufs"][i], dim, np.float32)
                assert np.array_equal(a.view(np.uint32), ref["bufs"][i].view(np.uint32)), \
                    (seq_no, n_st, i)
            finite += bool(np.all(np.isfinite(ref["bufs"][i])))
        for c in ("kc", "vc"):
            for n_st, st in enumerate(states):
                a = st["be"].download(st[c], layers * mc * dim, np.uint16)
                assert np.array_equal(a, ref[c]), (seq_no, n_st, c)
    assert finite > 0.9 * 300 * n_buf, finite  # the comparisons were of numbers
    # every kind of join and group happened along the way
    mock = C.CDLL(so_f)
    mock.mock_fused_count.restype = C.c_uint
    counts = [mock.mock_fused_count(i) for i in range(7)]
    assert all(c > 0 for c in counts), counts


def test_shim_marshalling_rejects_malformed_arguments(tmpdir_mod):
    so = build_mock(tmpdir_mod, "mock_ok2.so")
    be, ok = fresh_shim(tmpdir_mod, so)
    assert ok
    keep = []
    x = be.upload(np.zeros(16, np.float32))
    pipe = be.ops.compile_primitive_pipeline(be.device(), V.OP_ELEMENTWISE, None, 0)
    A = V.Backend.buf_arg
    assert not be.dispatch(pipe, [A(x), A(x), A(x)])                      # too few
    assert "takes 4 arguments" in be.last_error()
    assert not be.dispatch(pipe, [A(x), be.u32_arg(keep, 1), A(x), be.u32_arg(keep, 4)])
    assert "malformed" in be.last_error()
    err = C.create_string_buffer(128)
    assert not be.ops.compile_primitive_pipeline(be.device(), V.OP_STATE_SPACE, err, 128)
    assert b"no primitive kernel" in err.value


def test_linear_batch_extension_through_shim_on_host_mock(tmpdir_mod, host):
    """The batched-linear extension (include/vbs_hip_batch.h) through the
    shim over the host mock: B vectors equal B oracle tiles; bad batches,
    strides and short buffers are refused."""
    so = build_mock(tmpdir_mod, "mock_batch.so")
    be, ok = fresh_shim(tmpdir_mod, so)
    assert ok, be.last_error()
    res = run_linear_batch(be, Oracle(), host, [(V.Q4_K, 40, 512), (V.Q8_0, 19, 256),
                                                (V.F16, 9, 96)], [1, 3, 16])
    bad = [r[0] for r in res if not r[1]]
    assert not bad, bad


@pytest.mark.gpu
def test_linear_batch_extension_on_gfx950(backend, host):
    res = run_linear_batch(backend, Oracle(), host,
                           [(V.Q4_K, 4096, 4096), (V.Q6_K, 4096, 11008), (V.Q8_0, 1000, 4096),
                            (V.Q4_0, 300, 512), (V.F32, 77, 1000)], [1, 5, 8, 16])
    bad = [r[0] for r in res if not r[1]]
    assert not bad, bad


@pytest.mark.gpu
def test_backend_suite_on_gfx950(backend, host):
    """The same suite through g_vbs_hip_backend on the MI355X."""
    lib = backend.lib
    lib.vbs_gfx950_shim_library_path.restype = C.c_char_p
    path = lib.vbs_gfx950_shim_library_path().decode()
    assert path.endswith("lib/libvbs_gfx950.so"), path
    dev = backend.ops.get_device(0).contents
    assert b"gfx950" in dev.name and dev.max_working_set_bytes > (200 << 30)
    res = run_suite(backend, Oracle(), host)
    bad = [r[0] for r in res if not r[1]]
    assert not bad, bad


@pytest.mark.gpu
def test_gpu_dispatch_trace_on_device(backend, host, tmpdir_mod, tmp_path):
    """VBS_TRACE=2 on the MI355X: a private copy of the shim over the real
    device library counts two decode steps of the Q4_K_M model as the host
    mock's trace does (grouped q/k/v and gate/up, two matvec + add launches
    per layer, the embedding and the RMSNorm + lm_head per step), times every
    launch, and leaves the logits equal to the untraced table's bit for
    bit."""
    from test_decode import TINY
    log = tmp_path / "trace.log"
    os.environ["VBS_TRACE"], os.environ["VBS_TRACE_FILE"] = "2", str(log)
    try:
        be, ok = fresh_shim(tmpdir_mod, V.DEVICE_LIB)
    finally:
        del os.environ["VBS_TRACE"], os.environ["VBS_TRACE_FILE"]
    assert ok, be.last_error()
    assert be.lib.vbs_hip_trace_level() == 2
    be.lib.vbs_hip_trace_reset()
    model = V.SynthModel(host, **TINY, seed=5)
    outs = []
    for b in (be, backend):
        d = V.Decoder(host, b, model)
        outs.append([d.step(3 + pos, pos) for pos in range(2)])
        d.close()
    for got, want in zip(*outs):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    tc = (TraceCounter * len(TRACE_KINDS))()
    be.lib.vbs_hip_trace_counters(tc)
    L, steps = TINY["n_layers"], 2
    launches = {k: tc[i].launches for i, k in enumerate(TRACE_KINDS)}
    assert launches["qkv_group"] == steps * L and launches["ffn_group"] == steps * L, launches
    assert launches["linear_joined"] == steps * (2 * L + 1) and launches["attention"] == steps * L
    assert launches["linear"] == 0 and launches["normalize"] == 0, launches
    assert all(tc[i].ns > 0 for i in range(len(TRACE_KINDS)) if tc[i].launches)
    assert len(log.read_text().splitlines()) == sum(launches.values())

