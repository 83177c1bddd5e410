"""Write a synthetic llama-style Q4_K_M model as a GGUF v3 file.

    python verum-bespoke-singularity_amd/synth_gguf.py --geometry 7b out.gguf
    python verum-bespoke-singularity_amd/synth_gguf.py --geometry 70b --layers 80 out.gguf

The file holds the tensors in the decode order of the reference's graph
(src/vbs_graph.c:61-96) and the llama.* metadata its profiler and CPU model
require (src/vbs_profiler.c:328-352, src/vbs_cpu.c:396-476): the reference's
GGUF parser and CPU model open it, and its `verum-slice --inspect` /
`--benchmark <file>` modes (src/main.c:810-860) read the same keys.
Weights are the same synthetic bytes the decode tests and bench.py use for
the same seed; nothing is held in memory beyond a 32 MiB piece.
"""
import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import vbs_gfx950 as V  # noqa: E402

GEOMETRIES = {
    "7b": dict(n_layers=32, hidden=4096, ffn=11008, n_heads=32, n_kv_heads=8, head_dim=128,
               vocab=32000, context_length=2176),
    "70b": dict(n_layers=80, hidden=8192, ffn=28672, n_heads=64, n_kv_heads=8, head_dim=128,
                vocab=32000, context_length=8320),
}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("path")
    ap.add_argument("--geometry", choices=sorted(GEOMETRIES), default="7b")
    ap.add_argument("--layers", type=int, default=0, help="layer count (default: the geometry's)")
    ap.add_argument("--context-length", type=int, default=0)
    ap.add_argument("--seed", type=int, default=1234)
    a = ap.parse_args(argv)
    g = dict(GEOMETRIES[a.geometry])
    if a.layers:
        g["n_layers"] = a.layers
    if a.context_length:
        g["context_length"] = a.context_length
    V.write_gguf_geometry(V.load_host(), a.path, seed=a.seed, **g)
    print(f"{a.path}: {os.path.getsize(a.path)} bytes, {g['n_layers']} layers")
    return 0


if __name__ == "__main__":
    sys.exit(main())
