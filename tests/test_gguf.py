"""The synthetic models as GGUF files, read back by the reference's own loader.

`vbs_synth_write_gguf` (host/vbs_synth.c) writes a synthetic llama-style
model as GGUF v3; the reference parser (src/vbs_gguf.c, compiled into
oracle/_ref) must accept it, report every tensor with the type, shape and
byte length the loader derives (src/vbs_gguf.c:155-213), in the plan order
of src/vbs_graph.c:61-96, with the metadata src/vbs_profiler.c:328-341 and
src/vbs_cpu.c:396-476 read, and the tensor bytes must be those of the
in-memory model the decode tests use.
"""
import ctypes as C
import os

import numpy as np
import pytest

import vbs_gfx950 as V
from oracle_lib import REF_SO

pytestmark = pytest.mark.skipif(not os.path.exists(REF_SO),
                                reason="oracle/_ref (the reference parser) is not built")


class RefTensor(C.Structure):
    """vbs_tensor_t (include/vbs_gguf.h of the reference)."""
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_uint32), ("shape", C.c_uint64 * 4),
                ("type", C.c_int), ("data_offset", C.c_uint64), ("byte_length", C.c_uint64),
                ("columns", C.c_uint64), ("rows", C.c_uint64), ("packed_row_bytes", C.c_uint64)]


def ref_parser():
    lib = C.CDLL(REF_SO)
    lib.vbs_gguf_open.restype = C.c_void_p
    lib.vbs_gguf_open.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
    lib.vbs_gguf_close.argtypes = [C.c_void_p]
    lib.vbs_gguf_get_tensor.restype = C.POINTER(RefTensor)
    lib.vbs_gguf_get_tensor.argtypes = [C.c_void_p, C.c_char_p]
    lib.vbs_gguf_get_uint32_metadata.restype = C.c_bool
    lib.vbs_gguf_get_uint32_metadata.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_uint32)]
    lib.vbs_gguf_get_float32_metadata.restype = C.c_bool
    lib.vbs_gguf_get_float32_metadata.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_float)]
    lib.vbs_gguf_get_string_metadata.restype = C.c_char_p
    lib.vbs_gguf_get_string_metadata.argtypes = [C.c_void_p, C.c_char_p]
    return lib


def expected_tensors(model):
    """(name, type, rows, cols, array) in the plan order."""
    c, mix = model.cfg, model.mix
    out = [("token_embd.weight", mix["embd"], c["vocab"], c["hidden"], model.tok_embd)]
    names = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output",
             "gate": "ffn_gate", "up": "ffn_up", "down": "ffn_down"}
    H, F = c["hidden"], c["ffn"]
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    shapes = {"q": (qd, H), "k": (kvd, H), "v": (kvd, H), "o": (H, qd), "gate": (F, H),
              "up": (F, H), "down": (H, F)}
    for L in range(c["n_layers"]):
        out.append((f"blk.{L}.attn_norm.weight", V.F32, 1, H, model.attn_norm[L]))
        for k, role in enumerate(V.MAT_ROLES):
            if role == "gate":
                out.append((f"blk.{L}.ffn_norm.weight", V.F32, 1, H, model.ffn_norm[L]))
            r, cc = shapes[role]
            out.append((f"blk.{L}.{names[role]}.weight", mix[role], r, cc, model.w[7 * L + k]))
    out.append(("output_norm.weight", V.F32, 1, H, model.out_norm))
    out.append(("output.weight", mix["head"], c["vocab"], H, model.lm_head))
    return out


@pytest.mark.parametrize("mix", [None, {"q": V.Q4_0, "k": V.Q4_1, "v": V.Q8_0, "o": V.F16,
                                        "gate": V.Q4_K, "up": V.Q6_K, "down": V.F32,
                                        "embd": V.Q8_0, "head": V.Q4_K}],
                         ids=["q4_k_m", "every_type"])
def test_synthetic_gguf_reads_back_through_the_reference_loader(host, tmp_path, mix):
    model = V.SynthModel(host, n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2,
                         head_dim=64, vocab=512, max_ctx=64, seed=21, mix=mix)
    path = str(tmp_path / "synth.gguf")
    V.write_gguf(host, path, model, context_length=2176)
    lib = ref_parser()
    err = C.create_string_buffer(512)
    m = lib.vbs_gguf_open(path.encode(), err, 512)
    assert m, err.value.decode()
    try:
        c = model.cfg
        u = C.c_uint32()
        for key, want in [("llama.block_count", c["n_layers"]), ("llama.context_length", 2176),
                          ("llama.embedding_length", c["hidden"]),
                          ("llama.feed_forward_length", c["ffn"]),
                          ("llama.attention.head_count", c["n_heads"]),
                          ("llama.attention.head_count_kv", c["n_kv_heads"]),
                          ("llama.rope.dimension_count", c["head_dim"]),
                          ("llama.vocab_size", c["vocab"]), ("general.alignment", 32)]:
            assert lib.vbs_gguf_get_uint32_metadata(m, key.encode(), C.byref(u)), key
            assert u.value == want, key
        f = C.c_float()
        assert lib.vbs_gguf_get_float32_metadata(m, b"llama.rope.freq_base", C.byref(f))
        assert f.value == np.float32(c["theta"])
        assert lib.vbs_gguf_get_float32_metadata(m, b"llama.attention.layer_norm_rms_epsilon",
                                                 C.byref(f))
        assert f.value == np.float32(c["eps"])
        assert lib.vbs_gguf_get_string_metadata(m, b"general.architecture") == b"llama"
        raw = np.fromfile(path, dtype=np.uint8)
        last = -1
        for name, t, rows, cols, arr in expected_tensors(model):
            tp = lib.vbs_gguf_get_tensor(m, name.encode())
            assert tp, name
            tt = tp.contents
            assert (tt.type, tt.rows, tt.columns) == (t, rows, cols), name
            assert tt.byte_length == arr.nbytes, name
            assert tt.data_offset % 32 == 0 and tt.data_offset > last, name  # plan order
            last = tt.data_offset
            got = raw[tt.data_offset:tt.data_offset + tt.byte_length]
            assert np.array_equal(got, np.ascontiguousarray(arr).view(np.uint8).ravel()), name
    finally:
        lib.vbs_gguf_close(m)


def test_7b_geometry_file_from_the_command_line(tmp_path):
    """synth_gguf.py at the 7B geometry (one layer; the writer streams, so 32
    layers differ only in length): the reference loader accepts it and the
    tensors sit where the byte lengths of the A22 order put them."""
    import subprocess
    import sys
    path = str(tmp_path / "synth7b.gguf")
    tool = os.path.join(os.path.dirname(V.__file__), "synth_gguf.py")
    subprocess.run([sys.executable, tool, "--geometry", "7b", "--layers", "1", path],
                   check=True, capture_output=True, timeout=300)
    lib = ref_parser()
    err = C.create_string_buffer(512)
    m = lib.vbs_gguf_open(path.encode(), err, 512)
    assert m, err.value.decode()
    try:
        u = C.c_uint32()
        assert lib.vbs_gguf_get_uint32_metadata(m, b"llama.context_length", C.byref(u))
        assert u.value >= 2176
        order = ["token_embd.weight", "blk.0.attn_norm.weight", "blk.0.attn_q.weight",
                 "blk.0.attn_k.weight", "blk.0.attn_v.weight", "blk.0.attn_output.weight",
                 "blk.0.ffn_norm.weight", "blk.0.ffn_gate.weight", "blk.0.ffn_up.weight",
                 "blk.0.ffn_down.weight", "output_norm.weight", "output.weight"]
        want = {"token_embd.weight": (V.Q6_K, 32000, 4096), "blk.0.attn_q.weight": (V.Q4_K, 4096, 4096),
                "blk.0.attn_k.weight": (V.Q4_K, 1024, 4096), "blk.0.ffn_up.weight": (V.Q4_K, 11008, 4096),
                "blk.0.ffn_down.weight": (V.Q6_K, 4096, 11008), "output.weight": (V.Q6_K, 32000, 4096)}
        end = None
        for name in order:
            tt = lib.vbs_gguf_get_tensor(m, name.encode()).contents
            if name in want:
                assert (tt.type, tt.rows, tt.columns) == want[name], name
            assert tt.byte_length == tt.rows * V.row_bytes(tt.type, tt.columns), name
            if end is not None:
                assert tt.data_offset == (end + 31) // 32 * 32, name
            end = tt.data_offset + tt.byte_length
        assert os.path.getsize(path) == end
    finally:
        lib.vbs_gguf_close(m)


def test_writer_refuses_bad_geometry(host, tmp_path):
    """Empty dimensions and rows that are not whole blocks of their type are
    refused with the reason, and no file is left half-written as success."""
    base = dict(n_layers=1, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
                context_length=2176)
    with pytest.raises(RuntimeError, match="empty model dimension"):
        V.write_gguf_geometry(host, str(tmp_path / "a.gguf"), **dict(base, n_layers=0))
    with pytest.raises(RuntimeError, match="does not fit"):
        V.write_gguf_geometry(host, str(tmp_path / "b.gguf"), **dict(base, hidden=100))
    with pytest.raises(RuntimeError):
        V.write_gguf_geometry(host, str(tmp_path / "missing_dir" / "c.gguf"), **base)
