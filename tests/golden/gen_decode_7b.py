#!/usr/bin/env python3
"""Write tests/golden/decode_7b_greedy.npz: 128 greedy tokens of the full
7B-shaped Q4_K_M model (32 layers, hidden 4096, ffn 11008, 32/8 heads of
128, vocab 32000; synthetic weights, seed 7) from token 1 at position 2048,
its KV cache prefilled N(0,1) over positions 0..2047, decoded by the
reference's own CPU backend (oracle/_ref/libvbs_ref.so, built from
src/vbs_backend_cpu.c, src/vbs_dequant.c and src/vbs_gguf.c by
`make -C oracle ref`) in the bridge's op order (src/vbs_specializer.c:353-357).

Stored: the 128 tokens (first maximum, src/main.c:929-932), every step's
top-1 and top-2 logits, and the whole logits of the first and last steps.
Only data is written. The reference backend is single-threaded: the run
takes about 80 minutes.

    python tests/golden/gen_decode_7b.py
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "verum-bespoke-singularity_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, HERE)
import vbs_gfx950 as V  # noqa: E402
from gen_golden import ref_backend  # noqa: E402

GEO_7B = dict(hidden=4096, ffn=11008, n_heads=32, n_kv_heads=8, head_dim=128, vocab=32000)
CTX, N_TOK, SEED, START = 2048, 128, 7, 1
OUT = os.path.join(HERE, "decode_7b_greedy.npz")


def main():
    host = V.load_host()
    model = V.SynthModel(host, n_layers=32, **GEO_7B, max_ctx=CTX + N_TOK + 1, seed=SEED)
    kc_p, vc_p = model.kv_prefill(host, CTX)
    d = V.Decoder(host, ref_backend(), model)
    d.load_kv(kc_p, vc_p, CTX)
    toks, top2, first, last = [], [], None, None
    tok = START
    t0 = time.time()
    for i in range(N_TOK):
        lg = d.step(tok, CTX + i)
        tok = int(np.argmax(lg))
        toks.append(tok)
        top2.append(np.sort(lg)[-2:][::-1])
        first = lg.copy() if first is None else first
        last = lg
        print(f"step {i}: token {tok} margin {top2[-1][0] - top2[-1][1]:.4f} "
              f"({time.time() - t0:.0f} s)", flush=True)
    d.close()
    np.savez_compressed(OUT, tokens=np.array(toks, np.uint32), top2=np.array(top2, np.float32),
                        logits_first=first, logits_last=last,
                        config=np.array([CTX, N_TOK, SEED, START, 32], np.uint32))
    print("wrote", OUT)


if __name__ == "__main__":
    main()
