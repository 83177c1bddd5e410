"""ctypes access to the CPU oracle (oracle/liboracle.so) and, where it was
built, the reference's own CPU backend (oracle/_ref/libvbs_ref.so).

Test infrastructure: the oracle is the parity checker, never the thing
measured or shipped.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libvbs_ref.so")
REF_HOT_SO = os.path.join(ROOT, "oracle", "_ref", "libvbs_hotpath_ref.so")
REF_CPU_SO = os.path.join(ROOT, "oracle", "_ref", "libvbs_cpu_ref.so")
REF_CALLERS_SO = os.path.join(ROOT, "oracle", "_ref", "libvbs_callers_ref.so")
REF_CALLERS_Q4K_SO = os.path.join(ROOT, "oracle", "_ref", "libvbs_callers_q4k_ref.so")

_P, _U32, _I, _F = C.c_void_p, C.c_uint32, C.c_int, C.c_float
F16FN = C.CFUNCTYPE(C.c_uint16, C.c_float)


class OracleModel(C.Structure):
    """vbs_oracle_model_t (oracle/vbs_oracle.h)."""
    _fields_ = [("n_layers", C.c_uint32), ("hidden", C.c_uint32), ("ffn", C.c_uint32),
                ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("vocab", C.c_uint32), ("max_ctx", C.c_uint32),
                ("rope_theta", C.c_float), ("rms_eps", C.c_float),
                ("embd_type", C.c_int), ("tok_embd", C.c_void_p), ("out_norm", C.c_void_p),
                ("head_type", C.c_int), ("lm_head", C.c_void_p),
                ("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
                ("wtype", C.c_void_p), ("wdata", C.c_void_p),
                ("kc", C.c_void_p), ("vc", C.c_void_p)]


def _ptr(a):
    return None if a is None else a.ctypes.data


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        sig = {
            "f16_to_f32": (C.c_float, [C.c_uint16]),
            "f32_to_f16": (C.c_uint16, [C.c_float]),
            "digest_f32_to_f16": (C.c_uint64, [F16FN, _I]),
            "dequant_block": (_I, [_I, _P, _P]),
            "dequant_row": (_I, [_I, _P, _U32, _P]),
            "linear_tile": (_I, [_I, _P, _P, _P, _U32, _U32, _U32, _U32, _I]),
            "linear_tile_mt": (_I, [_I, _P, _P, _P, _U32, _U32, _U32, _U32, _I, _I]),
            "embed_row": (_I, [_I, _P, _U32, _P, _U32]),
            "rms_norm": (None, [_P, _P, _P, _U32, _F]),
            "rope": (None, [_P, _U32, _U32, _U32, _F]),
            "silu_mul": (None, [_P, _P, _P, _U32]),
            "add": (None, [_P, _P, _P, _U32]),
            "cache_store": (None, [_P, _P, _P, _P, _U32, _U32, _U32, _U32]),
            "attention": (None, [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _F]),
            "forward_token": (_I, [_P, _U32, _U32, _P, _I]),
            "f32_to_f16_rne": (C.c_uint16, [C.c_float]),
            "quantize_q8": (None, [_P, _U32, _P, _P, _P]),
            "hot_matvec": (_I, [_I, _P, _U32, _U32, _P, _P, _P, _P, _P]),
        }
        for k, (r, a) in sig.items():
            f = getattr(L, "vbs_oracle_" + k)
            f.restype, f.argtypes = r, a
            setattr(self, "_" + k, f)
        self.f16_fn = F16FN(("vbs_oracle_f32_to_f16", L))

    # numpy-friendly wrappers ------------------------------------------------
    def dequant_row(self, t, row: np.ndarray, cols: int) -> np.ndarray:
        out = np.empty(cols, np.float32)
        assert self._dequant_row(t, _ptr(np.ascontiguousarray(row)), cols, _ptr(out))
        return out

    def linear(self, t, w, x, cols, rows, y=None, col_off=0, row_off=0, accumulate=False,
               threads=8):
        w = np.ascontiguousarray(w)
        x = np.ascontiguousarray(x, dtype=np.float32)
        if y is None:
            y = np.zeros(row_off + rows, np.float32)
        assert self._linear_tile_mt(t, _ptr(w), _ptr(x), _ptr(y), cols, rows, col_off, row_off,
                                    int(accumulate), threads)
        return y

    def embed(self, t, table, token, dim):
        out = np.empty(dim, np.float32)
        assert self._embed_row(t, _ptr(table), token, _ptr(out), dim)
        return out

    def rms_norm(self, x, w, eps):
        out = np.empty_like(x)
        self._rms_norm(_ptr(x), _ptr(w), _ptr(out), x.size, eps)
        return out

    def rope(self, x, pos, hd, nh, theta):
        y = np.array(x, dtype=np.float32, copy=True)
        self._rope(_ptr(y), pos, hd, nh, theta)
        return y

    def silu_mul(self, g, u):
        out = np.empty_like(g)
        self._silu_mul(_ptr(g), _ptr(u), _ptr(out), g.size)
        return out

    def add(self, a, b):
        out = np.empty_like(a)
        self._add(_ptr(a), _ptr(b), _ptr(out), a.size)
        return out

    def cache_store(self, k, v, kc, vc, pos, layer, max_ctx, kv_dim):
        self._cache_store(_ptr(k), _ptr(v), _ptr(kc), _ptr(vc), pos, layer, max_ctx, kv_dim)

    def attention(self, q, kc, vc, seq_len, layer, max_ctx, nqh, nkh, hd, scale):
        out = np.empty(nqh * hd, np.float32)
        self._attention(_ptr(q), _ptr(kc), _ptr(vc), _ptr(out), seq_len, layer, max_ctx, nqh, nkh,
                        hd, scale)
        return out

    def f32_to_f16(self, a: np.ndarray) -> np.ndarray:
        return np.array([self._f32_to_f16(float(v)) for v in a.ravel()], np.uint16).reshape(a.shape)

    def quantize_q8(self, x: np.ndarray):
        """(xq int8[cols], qd f32[cols/32], qsum f32[cols/32])."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        nb = x.size // 32
        xq, qd, qs = np.empty(nb * 32, np.int8), np.empty(nb, np.float32), np.empty(nb, np.float32)
        self._quantize_q8(_ptr(x), x.size, _ptr(xq), _ptr(qd), _ptr(qs))
        return xq, qd, qs

    def hot_matvec(self, t, w, rows, cols, xq=None, qd=None, qsum=None, x=None):
        y = np.empty(rows, np.float32)
        assert self._hot_matvec(t, _ptr(np.ascontiguousarray(w)), rows, cols, _ptr(xq), _ptr(qd),
                                _ptr(qsum), _ptr(x), _ptr(y))
        return y

    def model(self, synth_model, kc: np.ndarray, vc: np.ndarray) -> OracleModel:
        s = synth_model.decode_struct()
        m = OracleModel()
        for name, _ in s._fields_:
            setattr(m, name, getattr(s, name))
        m.kc, m.vc = kc.ctypes.data, vc.ctypes.data
        return m

    def forward(self, model: OracleModel, token: int, pos: int, vocab: int, threads=8):
        logits = np.empty(vocab, np.float32)
        assert self._forward_token(C.addressof(model), token, pos, logits.ctypes.data, threads)
        return logits


def reference_cpu():
    """The reference's CPU backend + dequantiser, or None if not built here."""
    if not os.path.exists(REF_SO):
        return None
    lib = C.CDLL(REF_SO)
    lib.vbs_f16_to_f32.restype, lib.vbs_f16_to_f32.argtypes = C.c_float, [C.c_uint16]
    lib.vbs_f32_to_f16.restype, lib.vbs_f32_to_f16.argtypes = C.c_uint16, [C.c_float]
    lib.vbs_dequant_block.restype, lib.vbs_dequant_block.argtypes = C.c_int, [C.c_int, _P, _P]
    return lib


def reference_hot():
    """The reference's CPU hot-kernel table and module loader
    (src/vbs_hotpath.c), or None if not built here."""
    if not os.path.exists(REF_HOT_SO):
        return None
    import vbs_gfx950 as V
    lib = C.CDLL(REF_HOT_SO)
    lib.vbs_hot_builtin.restype = C.POINTER(V.HotKernels)
    lib.vbs_hot_current.restype = C.POINTER(V.HotKernels)
    lib.vbs_hot_load.restype, lib.vbs_hot_load.argtypes = C.c_bool, [C.c_char_p, C.c_char_p, C.c_size_t]
    lib.vbs_hot_rollback.restype, lib.vbs_hot_rollback.argtypes = C.c_bool, [C.c_char_p, C.c_size_t]
    lib.vbs_hot_current_name.restype = C.c_char_p
    lib.vbs_hot_current_path.restype = C.c_char_p
    lib.vbs_hot_has_rollback.restype = C.c_bool
    sz = C.c_size_t
    for n in ("q8_0", "q4_0"):
        f = getattr(lib, "vbs_hot_matvec_" + n)
        f.restype, f.argtypes = None, [_P, sz, sz, _P, _P, _P]
    lib.vbs_hot_matvec_q4_1.restype = None
    lib.vbs_hot_matvec_q4_1.argtypes = [_P, sz, sz, _P, _P, _P, _P]
    for n in ("f32", "f16"):
        f = getattr(lib, "vbs_hot_matvec_" + n)
        f.restype, f.argtypes = None, [_P, sz, sz, _P, _P]
    return lib


def reference_cpu_model():
    """The reference's model-level CPU inference (src/vbs_cpu.c and the hot
    table it calls through), or None if not built here."""
    if not os.path.exists(REF_CPU_SO):
        return None
    lib = C.CDLL(REF_CPU_SO)
    sz = C.c_size_t
    lib.vbs_cpu_open.restype, lib.vbs_cpu_open.argtypes = _P, [C.c_char_p, sz, C.c_char_p, sz]
    lib.vbs_cpu_close.restype, lib.vbs_cpu_close.argtypes = None, [_P]
    lib.vbs_cpu_reset.restype, lib.vbs_cpu_reset.argtypes = None, [_P]
    lib.vbs_cpu_step.restype = C.c_bool
    lib.vbs_cpu_step.argtypes = [_P, C.c_uint32, C.c_char_p, sz]
    lib.vbs_cpu_logits.restype, lib.vbs_cpu_logits.argtypes = C.POINTER(C.c_float), [_P]
    lib.vbs_cpu_vocab_size.restype, lib.vbs_cpu_vocab_size.argtypes = sz, [_P]
    lib.vbs_cpu_context_capacity.restype, lib.vbs_cpu_context_capacity.argtypes = sz, [_P]
    lib.vbs_hot_load.restype, lib.vbs_hot_load.argtypes = C.c_bool, [C.c_char_p, C.c_char_p, sz]
    lib.vbs_hot_rollback.restype, lib.vbs_hot_rollback.argtypes = C.c_bool, [C.c_char_p, sz]
    lib.vbs_hot_current_name.restype = C.c_char_p
    return lib


def cpu_model_logits(lib, path, tokens, capacity=64):
    """Logits after each token of `tokens` (positions 0, 1, ...) from the
    reference CPU model opened on the GGUF file `path`."""
    err = C.create_string_buffer(512)
    m = lib.vbs_cpu_open(str(path).encode(), capacity, err, 512)
    if not m:
        raise RuntimeError(f"vbs_cpu_open: {err.value.decode()}")
    try:
        vocab = lib.vbs_cpu_vocab_size(m)
        out = []
        for t in tokens:
            if not lib.vbs_cpu_step(m, t, err, 512):
                raise RuntimeError(f"vbs_cpu_step: {err.value.decode()}")
            out.append(np.ctypeslib.as_array(lib.vbs_cpu_logits(m), (vocab,)).copy())
        return out
    finally:
        lib.vbs_cpu_close(m)
