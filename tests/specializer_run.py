"""TEST-ONLY child process: the reference's specializer module over a backend.

    python tests/specializer_run.py --backend cpu|gfx950 --lib plain|q4k \\
        --gguf MODEL.gguf --workdir DIR --start TOKEN --steps N --out OUT.npz

Runs what `verum-slice --generate` does after loading a model
(src/main.c:873-932): the engine's set-up over the chosen ops table
(tests/ref_callers.py RefEngine, as src/vbs_engine.c:17-172), then
vbs_engine_compile's chain from the reference sources -- vbs_graph_compile,
vbs_planner_build, vbs_specializer_emit_source, vbs_specializer_compile (the
system C compiler), vbs_specializer_load, verum_init -- and greedy decoding
through the emitted verum_forward, one token per call, argmax = first
maximum (src/main.c:926-932). Writes the tokens and every step's logits.

A child process because the emitted module finds the bridge in the global
symbol scope (it is compiled without linking it, src/vbs_specializer.c:
408-436), so the callers library is loaded RTLD_GLOBAL, and a process may hold
only one such instance.

--lib q4k uses the callers library built with oracle/specializer_q4k.patch
(Q4_K on the specializer's allow-list); plain is the unpatched specializer.
--backend gfx950 is g_vbs_hip_backend of this build's shim; cpu is the
reference's own CPU backend (oracle/_ref/libvbs_ref.so).
"""
import argparse
import ctypes as C
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (os.path.join(ROOT, "verum-bespoke-singularity_amd"), HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

import vbs_gfx950 as V  # noqa: E402
from oracle_lib import REF_CALLERS_Q4K_SO, REF_CALLERS_SO, REF_SO  # noqa: E402
import ref_callers as rc  # noqa: E402


def log(msg):
    print(f"[specializer_run {time.strftime('%H:%M:%S')}] {msg}", flush=True)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--backend", choices=("cpu", "gfx950"), required=True)
    ap.add_argument("--lib", choices=("plain", "q4k"), required=True)
    ap.add_argument("--gguf", required=True)
    ap.add_argument("--workdir", required=True)
    ap.add_argument("--start", type=int, default=1)
    ap.add_argument("--steps", type=int, default=12)
    ap.add_argument("--out", required=True)
    a = ap.parse_args(argv)

    L = rc.load_callers(f"jit_{a.backend}_{a.lib}",
                        src=REF_CALLERS_Q4K_SO if a.lib == "q4k" else REF_CALLERS_SO,
                        global_scope=True)
    if a.backend == "cpu":
        be = V.Backend(C.CDLL(REF_SO), "g_vbs_cpu_backend")
    else:
        be = V.gfx950_backend()
    if not be.init():
        raise SystemExit(f"backend {a.backend} init failed: {be.last_error()}")
    log(f"backend {a.backend} ready; engine set-up over {a.gguf}")
    eng = rc.RefEngine(L, be, a.gguf)
    mod = None
    try:
        eng.zero_kv()
        log(f"specializing with the {a.lib} specializer into {a.workdir}")
        mod = eng.specialize(a.workdir)
        log(f"module {mod.path}: {mod.n_plans} planned nodes; decoding {a.steps} steps")
        tok, toks, logits = a.start, [], []
        for i in range(a.steps):
            lg = mod.forward([tok])
            tok = int(np.argmax(lg))
            toks.append(tok)
            logits.append(lg)
        log(f"tokens {toks}")
        np.savez(a.out, tokens=np.array(toks, np.int64), logits=np.stack(logits),
                 module=np.array(mod.path), n_plans=np.array(mod.n_plans))
    finally:
        if mod:
            mod.close()
        eng.close()
    log("done")


if __name__ == "__main__":
    main()
