"""ctypes bindings for the gfx950 backend of Verum's decode hot path.

Two native libraries, both built in-tree under ``lib/`` (see the Makefile):

* ``libvbs_gfx950.so`` -- the gfx950 kernels behind the C ABI declared in
  ``include/vbs_gfx950.h``;
* ``libvbs_backend_gfx950.so`` -- the C11 host side: ``g_vbs_hip_backend``
  (the reference's ``vbs_backend_ops_t`` slot, ``include/vbs_abi.h``), the
  decode-step driver (``host/vbs_decode.h``) and the synthetic weight
  generator (``host/vbs_synth.h``).

Nothing here computes: every operation is a call into those libraries. If
they are missing the import still succeeds but every loader raises, so a
caller cannot silently run without the native code.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG_DIR, "lib")
DEVICE_LIB = os.path.join(LIB_DIR, "libvbs_gfx950.so")
# The two host libraries can be taken from another directory, such as the
# sanitizer build of `make sanitize` (lib-san/); the device library cannot.
HOST_LIB_DIR = os.environ.get("VBS_GFX950_HOST_LIB_DIR") or LIB_DIR
HOST_LIB = os.path.join(HOST_LIB_DIR, "libvbs_backend_gfx950.so")
HOT_LIB = os.path.join(HOST_LIB_DIR, "libvbs_hot_gfx950.so")

# GGUF type ids (include/vbs_abi.h, reference include/vbs_gguf.h:13-48)
F32, F16, Q4_0, Q4_1, Q8_0, Q8_K, Q4_K, Q5_K, Q6_K, LNS8 = 0, 1, 2, 3, 8, 15, 12, 13, 14, 40
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q8_0: "Q8_0",
              Q4_K: "Q4_K", Q6_K: "Q6_K", LNS8: "LNS8"}
GEOMETRY = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34),
            Q4_K: (256, 144), Q6_K: (256, 210), LNS8: (32, 36)}

# vbs_op_kind_t (reference include/vbs_graph.h:11-23)
OP_EMBEDDING, OP_LINEAR, OP_NORMALIZE, OP_ATTENTION, OP_ROTARY, OP_ACTIVATION, \
    OP_ELEMENTWISE, OP_STATE_SPACE, OP_CONVOLUTION, OP_CACHE, OP_PROJECTION = range(11)


def row_bytes(t: int, cols: int) -> int:
    e, b = GEOMETRY[t]
    return (cols // e) * b


class NativeMissing(RuntimeError):
    """The in-tree native library was not built (run __graft_entry__.build())."""


def _cdll(path: str) -> C.CDLL:
    if not os.path.exists(path):
        raise NativeMissing(f"{path} is missing: build it with __graft_entry__.build()")
    return C.CDLL(path)


# --------------------------------------------------------------------------
# HIP runtime: events and stream capture (timing and graph tests)
# --------------------------------------------------------------------------
class Hip:
    """hipEvent timing and stream capture on the device library's stream."""

    def __init__(self):
        h = self.h = C.CDLL("libamdhip64.so")
        vp, pvp = C.c_void_p, C.POINTER(C.c_void_p)
        h.hipEventCreate.argtypes = [pvp]
        h.hipEventRecord.argtypes = [vp, vp]
        h.hipEventSynchronize.argtypes = [vp]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        h.hipEventDestroy.argtypes = [vp]
        h.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        h.hipStreamEndCapture.argtypes = [vp, pvp]
        h.hipGraphInstantiate.argtypes = [pvp, vp, vp, vp, C.c_size_t]
        h.hipGraphLaunch.argtypes = [vp, vp]
        h.hipGraphExecDestroy.argtypes = [vp]
        h.hipGraphDestroy.argtypes = [vp]

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed ({rc})")

    def event(self):
        e = C.c_void_p()
        self._ok(self.h.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e

    def record(self, ev, stream):
        self._ok(self.h.hipEventRecord(ev, C.c_void_p(stream)), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self._ok(self.h.hipEventSynchronize(b), "hipEventSynchronize")
        ms = C.c_float()
        self._ok(self.h.hipEventElapsedTime(C.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def capture(self, stream, enqueue):
        """Graph of the work `enqueue()` puts on `stream` (thread-local capture)."""
        self._ok(self.h.hipStreamBeginCapture(C.c_void_p(stream), 1), "hipStreamBeginCapture")
        try:
            enqueue()
        finally:
            g = C.c_void_p()
            rc = self.h.hipStreamEndCapture(C.c_void_p(stream), C.byref(g))
        self._ok(rc, "hipStreamEndCapture")
        ex = C.c_void_p()
        self._ok(self.h.hipGraphInstantiate(C.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        return g, ex

    def launch(self, graph, stream):
        self._ok(self.h.hipGraphLaunch(graph[1], C.c_void_p(stream)), "hipGraphLaunch")

    def destroy(self, graph):
        self.h.hipGraphExecDestroy(graph[1])
        self.h.hipGraphDestroy(graph[0])


# --------------------------------------------------------------------------
# device library (include/vbs_gfx950.h)
# --------------------------------------------------------------------------
_P, _U32, _I, _SZ, _F, _U64 = C.c_void_p, C.c_uint32, C.c_int, C.c_size_t, C.c_float, C.c_uint64

class LinearJoin(C.Structure):
    """vbs_gfx950_linear_join_t: the neighbours vbs_gfx950_linear_fused takes."""
    _fields_ = [("norm_w", _P), ("norm_eps", _F), ("x_normed", _P), ("acc", _P), ("rope", _I),
                ("pos", _U32), ("head_dim", _U32), ("theta", _F), ("gate", _P), ("hidden", _P),
                ("k_row", _P), ("kc", _P), ("vc", _P), ("kv_off", _U64)]


_DEVICE_SIGS = {
    "abi_version": (_I, []),
    "init": (_I, []),
    "last_error": (C.c_char_p, []),
    "device_count": (_I, []),
    "device_info": (_I, [_I, C.c_char_p, _SZ, C.POINTER(_U64), C.POINTER(_U64)]),
    "alloc": (_P, [_SZ]),
    "free": (_I, [_P]),
    "host_alloc": (_P, [_SZ]),
    "host_free": (_I, [_P]),
    "copy_h2d": (_I, [_P, _P, _SZ]),
    "copy_d2h": (_I, [_P, _P, _SZ]),
    "copy_d2d": (_I, [_P, _P, _SZ]),
    "synchronize": (_I, []),
    "linear_supported": (_I, [_I]),
    "linear": (_I, [_I, _P, _P, _P, _U32, _U32, _U32, _U32, _I]),
    "embed": (_I, [_I, _P, _U32, _P, _U32]),
    "rms_norm": (_I, [_P, _P, _P, _U32, _F]),
    "linear_fused": (_I, [_I, _P, _P, _P, _U32, _U32, C.POINTER(LinearJoin)]),
    "qkv_fused": (_I, [_I, _P, _P, _P, _P, _U32, _U32, _U32, _P, _F, _P, _P, _P, _P, _U32, _U32,
                       _F, _P, _P, _U32, _U32]),
    "gate_up_fused": (_I, [_I, _P, _P, _P, _U32, _U32, _P, _F, _P, _P, _P, _P]),
    "rope": (_I, [_P, _U32, _U32, _U32, _F]),
    "cache_store": (_I, [_P, _P, _P, _P, _U32, _U32, _U32, _U32]),
    "attention": (_I, [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _F]),
    "attention_noalloc": (_I, [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _U32, _F]),
    "silu_mul": (_I, [_P, _P, _P, _U32]),
    "add": (_I, [_P, _P, _P, _U32]),
    "dequant_rows": (_I, [_I, _P, _P, _U32, _U32, _P]),
    "linear_batch": (_I, [_I, _P, _P, _U32, _P, _U32, _U32, _U32, _U32]),
    "linear_batch_multi": (_I, [_I, _U32, _P, _P, _P, _U32, _P, _P, _U32, _U32]),
    "stream": (_P, []),
    "checksum_partials": (_U32, [_SZ]),
    "checksum": (_I, [_P, _SZ, _P]),
    "checksum_variant_partials": (_U32, [_SZ, _I]),
    "checksum_variant": (_I, [_P, _SZ, _P, _I]),
    "decoder_create": (_I, [_P, _U32, C.POINTER(C.c_void_p)]),
    "decoder_step": (_I, [_P, _U32, _U32, _P]),
    "decoder_greedy": (_I, [_P, _U32, _U32, _U32, _P, _P]),
    "decoder_greedy_eager": (_I, [_P, _U32, _U32, _U32, _P, _P]),
    "decoder_attn_o_fallbacks": (_I, [_P, _P]),
    "decoder_destroy": (_I, [_P]),
    "bdecoder_create": (_I, [_P, _U32, _U64, _U32, C.POINTER(C.c_void_p)]),
    "bdecoder_greedy": (_I, [_P, _P, _P, _U32, _P, _P]),
    "bdecoder_greedy_eager": (_I, [_P, _P, _P, _U32, _P, _P]),
    "bdecoder_step": (_I, [_P, _P, _P, _P]),
    "bdecoder_destroy": (_I, [_P]),
    "quantize_q8": (_I, [_P, _U32, _P, _P, _P]),
    "hot_matvec": (_I, [_I, _P, _U32, _U32, _P, _P, _P, _P]),
}

DEVICE_SYMBOLS = ["vbs_gfx950_" + k for k in _DEVICE_SIGS]


class GpuError(RuntimeError):
    pass


class DeviceLib:
    """Thin wrapper over libvbs_gfx950.so; methods raise GpuError on failure."""

    def __init__(self, path: str = DEVICE_LIB):
        self.path = path
        self.lib = _cdll(path)
        for name, (res, args) in _DEVICE_SIGS.items():
            fn = getattr(self.lib, "vbs_gfx950_" + name)
            fn.restype, fn.argtypes = res, args
            setattr(self, "_" + name, fn)

    def error(self) -> str:
        return self._last_error().decode()

    def check(self, ok, what: str):
        if not ok:
            raise GpuError(f"{what}: {self.error()}")
        return ok

    def init(self) -> bool:
        return bool(self._init())

    def info(self):
        name = C.create_string_buffer(128)
        tot, fr = _U64(), _U64()
        self.check(self._device_info(0, name, 128, C.byref(tot), C.byref(fr)), "device_info")
        return name.value.decode(), tot.value, fr.value

    # memory ------------------------------------------------------------
    def alloc(self, nbytes: int) -> int:
        p = self._alloc(nbytes)
        if not p:
            raise GpuError(f"alloc({nbytes}): {self.error()}")
        return p

    def free(self, p: int):
        self.check(self._free(p), "free")

    def upload(self, arr: np.ndarray) -> int:
        arr = np.ascontiguousarray(arr)
        p = self.alloc(max(arr.nbytes, 1))
        self.check(self._copy_h2d(p, arr.ctypes.data, arr.nbytes), "copy_h2d")
        return p

    def write(self, p: int, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        self.check(self._copy_h2d(p, arr.ctypes.data, arr.nbytes), "copy_h2d")

    def download(self, p: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        self.check(self._copy_d2h(out.ctypes.data, p, out.nbytes), "copy_d2h")
        return out

    def sync(self):
        self.check(self._synchronize(), "synchronize")

    # kernels -----------------------------------------------------------
    def linear(self, t, w, x, y, cols, rows, col_off=0, row_off=0, accumulate=False):
        self.check(self._linear(t, w, x, y, cols, rows, col_off, row_off, int(accumulate)), "linear")

    def linear_batch(self, t, w, x, xs, y, ys, cols, rows, batch):
        self.check(self._linear_batch(t, w, x, xs, y, ys, cols, rows, batch), "linear_batch")

    def linear_batch_multi(self, t, ws, rows, x, xs, ys, y_strides, cols, batch):
        """Up to three matrices (device pointers ws, outputs ys) over the same vectors."""
        n = len(ws)
        arr = lambda ctype, v: (ctype * n)(*v)
        self.check(self._linear_batch_multi(t, n, arr(C.c_void_p, ws), arr(C.c_uint32, rows), x, xs,
                                            arr(C.c_void_p, ys), arr(C.c_uint32, y_strides), cols,
                                            batch), "linear_batch_multi")

    def linear_fused(self, t, w, x, y, cols, rows, **join) -> bool:
        """y = W x with the neighbours named in `join` (the LinearJoin fields)
        in the same launch; False when no fused kernel takes the combination
        (nothing launched), an exception on an error."""
        r = self._linear_fused(t, w, x, y, cols, rows, C.byref(LinearJoin(**join)))
        if r == 2:
            return False
        self.check(r, "linear_fused")
        return True

    def qkv_fused(self, t, wq, wk, wv, x, cols, q_rows, kv_rows, norm_w, eps, xn, q, k, v, pos,
                  hd, theta, kc, vc, layer, max_ctx) -> bool:
        """The grouped attention-input ops in one launch; False when no grouped
        kernel takes the shape (nothing launched)."""
        r = self._qkv_fused(t, wq, wk, wv, x, cols, q_rows, kv_rows, norm_w or None, eps,
                            xn or None, q, k, v, pos, hd, theta, kc, vc, layer, max_ctx)
        if r == 2:
            return False
        self.check(r, "qkv_fused")
        return True

    def gate_up_fused(self, t, wg, wu, x, cols, rows, norm_w, eps, xn, gate, up, hidden) -> bool:
        """The grouped FFN-input ops in one launch; False when no grouped
        kernel takes the shape (nothing launched)."""
        r = self._gate_up_fused(t, wg, wu, x, cols, rows, norm_w or None, eps, xn or None, gate,
                                up, hidden)
        if r == 2:
            return False
        self.check(r, "gate_up_fused")
        return True

    def embed(self, t, w, token, out, dim):
        self.check(self._embed(t, w, token, out, dim), "embed")

    def quantize_q8(self, x, cols, xq, qd, qsum):
        self.check(self._quantize_q8(x, cols, xq, qd, qsum), "quantize_q8")

    def hot_matvec(self, t, w, rows, cols, act, qd, qsum, y):
        self.check(self._hot_matvec(t, w, rows, cols, act, qd or None, qsum or None, y),
                   "hot_matvec")

    def checksum(self, p, nbytes: int, variant: int = 0) -> int:
        """XOR of the 32-bit words of device bytes [p, p + nbytes) (16-byte
        aligned, a multiple of 16 bytes), from the per-wave partials of the
        read shape `variant` (vbs_gfx950_checksum_variant)."""
        n = int(self._checksum_variant_partials(nbytes, variant))
        if n == 0:
            return 0
        part = self.alloc(4 * n)
        try:
            self.check(self._checksum_variant(p, nbytes, part, variant), "checksum")
            return int(np.bitwise_xor.reduce(self.download(part, n, np.uint32)))
        finally:
            self.free(part)

    def dequant_rows(self, t, w, ids, n_rows, dim, out):
        self.check(self._dequant_rows(t, w, ids or None, n_rows, dim, out), "dequant_rows")

    def rms_norm(self, x, w, out, n, eps):
        self.check(self._rms_norm(x, w, out, n, eps), "rms_norm")

    def rope(self, x, pos, hd, nh, theta):
        self.check(self._rope(x, pos, hd, nh, theta), "rope")

    def cache_store(self, k, v, kc, vc, pos, layer, max_ctx, kv_dim):
        self.check(self._cache_store(k, v, kc, vc, pos, layer, max_ctx, kv_dim), "cache_store")

    def attention(self, q, kc, vc, out, seq_len, layer, max_ctx, nqh, nkh, hd, scale):
        self.check(self._attention(q, kc, vc, out, seq_len, layer, max_ctx, nqh, nkh, hd, scale),
                   "attention")

    def silu_mul(self, g, u, out, n):
        self.check(self._silu_mul(g, u, out, n), "silu_mul")

    def add(self, a, b, out, n):
        self.check(self._add(a, b, out, n), "add")

    def stream(self) -> int:
        return self._stream() or 0


# --------------------------------------------------------------------------
# vbs_backend_ops_t (include/vbs_abi.h)
# --------------------------------------------------------------------------
class VbsDevice(C.Structure):
    _fields_ = [("name", C.c_char * 128), ("type", C.c_int),
                ("max_working_set_bytes", C.c_uint64), ("max_buffer_bytes", C.c_uint64),
                ("internal_handle", C.c_void_p)]


class VbsBuffer(C.Structure):
    _fields_ = [("internal_handle", C.c_void_p), ("host_ptr", C.c_void_p),
                ("size", C.c_size_t), ("device", C.POINTER(VbsDevice))]


class VbsArg(C.Structure):
    _fields_ = [("tag", C.c_int), ("value", C.c_void_p), ("size", C.c_size_t)]


_PD, _PB = C.POINTER(VbsDevice), C.POINTER(VbsBuffer)


class VbsOps(C.Structure):
    _fields_ = [
        ("init", C.CFUNCTYPE(C.c_bool)),
        ("get_device_count", C.CFUNCTYPE(C.c_size_t)),
        ("get_device", C.CFUNCTYPE(_PD, C.c_size_t)),
        ("alloc_buffer", C.CFUNCTYPE(_PB, _PD, C.c_size_t, C.c_bool)),
        ("free_buffer", C.CFUNCTYPE(None, _PB)),
        ("copy_to_device", C.CFUNCTYPE(C.c_bool, _PB, C.c_void_p, C.c_size_t)),
        ("copy_to_host", C.CFUNCTYPE(C.c_bool, C.c_void_p, _PB, C.c_size_t)),
        ("compile_linear_pipeline", C.CFUNCTYPE(C.c_void_p, _PD, C.c_int, C.c_char_p, C.c_size_t)),
        ("compile_embed_pipeline", C.CFUNCTYPE(C.c_void_p, _PD, C.c_int, C.c_char_p, C.c_size_t)),
        ("compile_primitive_pipeline", C.CFUNCTYPE(C.c_void_p, _PD, C.c_int, C.c_char_p, C.c_size_t)),
        ("dispatch_linear_tile", C.CFUNCTYPE(C.c_bool, _PD, C.c_void_p, _PB, _PB, C.c_size_t, _PB, _PB,
                                             C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_bool)),
        ("dispatch_primitive", C.CFUNCTYPE(C.c_bool, _PD, C.c_void_p, C.POINTER(VbsArg), C.c_size_t,
                                           C.c_size_t, C.c_size_t)),
        ("synchronize_device", C.CFUNCTYPE(None, _PD)),
        ("launch_persistent_kernel", C.c_void_p),
    ]


class Backend:
    """A vbs_backend_ops_t table exported by a shared library under `symbol`."""

    def __init__(self, lib: C.CDLL, symbol: str, error_symbol: str | None = None):
        self.lib = lib
        self.ops = VbsOps.in_dll(lib, symbol)
        self._err = None
        if error_symbol:
            self._err = getattr(lib, error_symbol)
            self._err.restype = C.c_char_p

    def last_error(self) -> str:
        return self._err().decode() if self._err else ""

    def init(self) -> bool:
        return bool(self.ops.init())

    def device(self):
        return self.ops.get_device(0)

    # helpers mirroring the reference self-test's usage --------------------
    def alloc(self, nbytes, shared=False):
        b = self.ops.alloc_buffer(self.device(), nbytes, shared)
        if not b:
            raise GpuError(f"alloc_buffer({nbytes}) failed: {self.last_error()}")
        return b

    def upload(self, arr: np.ndarray, shared=False):
        arr = np.ascontiguousarray(arr)
        b = self.alloc(max(arr.nbytes, 1), shared)
        if not self.ops.copy_to_device(b, arr.ctypes.data, arr.nbytes):
            raise GpuError(f"copy_to_device failed: {self.last_error()}")
        return b

    def download(self, buf, shape, dtype):
        out = np.empty(shape, dtype=dtype)
        if not self.ops.copy_to_host(out.ctypes.data, buf, out.nbytes):
            raise GpuError(f"copy_to_host failed: {self.last_error()}")
        return out

    @staticmethod
    def buf_arg(buf) -> VbsArg:
        return VbsArg(0, buf.contents.internal_handle, 0)

    @staticmethod
    def u32_arg(keep: list, v: int) -> VbsArg:
        c = C.c_uint32(v)
        keep.append(c)
        return VbsArg(1, C.addressof(c), 4)

    @staticmethod
    def f32_arg(keep: list, v: float) -> VbsArg:
        c = C.c_float(v)
        keep.append(c)
        return VbsArg(1, C.addressof(c), 4)

    def dispatch(self, pipe, args, grid=1, block=256) -> bool:
        arr = (VbsArg * len(args))(*args)
        return bool(self.ops.dispatch_primitive(self.device(), pipe, arr, len(args), grid, block))


def load_host() -> C.CDLL:
    lib = _cdll(HOST_LIB)
    lib.vbs_gfx950_shim_library_path.restype = C.c_char_p
    lib.vbs_hip_last_error.restype = C.c_char_p
    lib.vbs_synth_blocks.restype = C.c_int
    lib.vbs_synth_blocks.argtypes = [C.c_int, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64,
                                     C.c_void_p, C.c_int]
    lib.vbs_synth_normal_f32.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_size_t, C.c_float,
                                         C.c_float, C.c_void_p, C.c_int]
    lib.vbs_synth_normal_f16.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_size_t, C.c_float,
                                         C.c_void_p, C.c_int]
    lib.vbs_synth_tokens.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32, C.c_size_t, C.c_void_p]
    lib.vbs_synth_write_gguf.restype = C.c_int
    lib.vbs_synth_write_gguf.argtypes = [C.c_char_p, C.c_void_p, C.c_char_p, C.c_size_t]
    lib.vbs_decode_create.restype = C.c_void_p
    lib.vbs_decode_create.argtypes = [C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
    lib.vbs_decode_destroy.argtypes = [C.c_void_p]
    lib.vbs_decode_load_kv.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32]
    lib.vbs_decode_read_kv.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32]
    lib.vbs_decode_step.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p]
    lib.vbs_decode_greedy.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_void_p,
                                      C.c_void_p]
    lib.vbs_decode_dispatch_count.restype = C.c_uint32
    lib.vbs_decode_dispatch_count.argtypes = [C.c_void_p]
    lib.vbs_decode_weight_bytes.restype = C.c_uint64
    lib.vbs_decode_weight_bytes.argtypes = [C.c_void_p]
    lib.vbs_decode_device_model.argtypes = [C.c_void_p, C.c_void_p]
    return lib


def gfx950_backend() -> Backend:
    """g_vbs_hip_backend of the shim (not yet initialised)."""
    return Backend(load_host(), "g_vbs_hip_backend", "vbs_hip_last_error")


# --------------------------------------------------------------------------
# synthetic data (host/vbs_synth.h)
# --------------------------------------------------------------------------
_THREADS = max(1, min(16, os.cpu_count() or 1))


def synth_matrix(host: C.CDLL, t: int, rows: int, cols: int, seed: int, stream: int) -> np.ndarray:
    """rows x cols packed matrix of type t as a uint8 array (rows, row_bytes)."""
    e, b = GEOMETRY[t]
    nblk = rows * (cols // e)
    out = np.empty(nblk * b, dtype=np.uint8)
    if t == F32:
        host.vbs_synth_normal_f32(seed, stream, 0, rows * cols, 1.0, 0.0, out.ctypes.data, _THREADS)
    elif t == F16:
        host.vbs_synth_normal_f16(seed, stream, 0, rows * cols, 1.0, out.ctypes.data, _THREADS)
    elif not host.vbs_synth_blocks(t, seed, stream, 0, nblk, out.ctypes.data, _THREADS):
        raise ValueError(f"no generator for type {t}")
    return out.reshape(rows, row_bytes(t, cols))


def synth_normal(host: C.CDLL, n: int, seed: int, stream: int, scale=1.0, offset=0.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    host.vbs_synth_normal_f32(seed, stream, 0, n, scale, offset, out.ctypes.data, _THREADS)
    return out


def synth_normal_f16(host: C.CDLL, n: int, seed: int, stream: int, scale=1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    host.vbs_synth_normal_f16(seed, stream, 0, n, scale, out.ctypes.data, _THREADS)
    return out


# --------------------------------------------------------------------------
# synthetic llama-style model (host/vbs_decode.h: vbs_decode_model_t)
# --------------------------------------------------------------------------
class DecodeModelStruct(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("hidden", C.c_uint32), ("ffn", C.c_uint32),
                ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("vocab", C.c_uint32), ("max_ctx", C.c_uint32),
                ("rope_theta", C.c_float), ("rms_eps", C.c_float),
                ("embd_type", C.c_int), ("tok_embd", C.c_void_p), ("out_norm", C.c_void_p),
                ("head_type", C.c_int), ("lm_head", C.c_void_p),
                ("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
                ("wtype", C.c_void_p), ("wdata", C.c_void_p)]


MAT_ROLES = ("q", "k", "v", "o", "gate", "up", "down")

Q4_K_M_MIX = {"q": Q4_K, "k": Q4_K, "v": Q4_K, "o": Q4_K, "gate": Q4_K, "up": Q4_K,
              "down": Q6_K, "embd": Q6_K, "head": Q6_K}


class SynthModel:
    """Host-resident synthetic model; arrays are kept alive by this object.

    Weight streams: token_embd 1, output 2, output_norm 3, layer L matrix k
    100 + 16*L + k, layer norms 100 + 16*L + 8 / + 9.
    """

    def __init__(self, host, *, n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, vocab,
                 max_ctx, mix=None, seed=1234, theta=10000.0, eps=1e-5):
        mix = dict(Q4_K_M_MIX if mix is None else mix)
        self.cfg = dict(n_layers=n_layers, hidden=hidden, ffn=ffn, n_heads=n_heads,
                        n_kv_heads=n_kv_heads, head_dim=head_dim, vocab=vocab, max_ctx=max_ctx,
                        theta=theta, eps=eps)
        self.mix, self.seed = mix, seed
        H, F, qd, kvd = hidden, ffn, n_heads * head_dim, n_kv_heads * head_dim
        shapes = {"q": (qd, H), "k": (kvd, H), "v": (kvd, H), "o": (H, qd),
                  "gate": (F, H), "up": (F, H), "down": (H, F)}
        self.tok_embd = synth_matrix(host, mix["embd"], vocab, H, seed, 1)
        self.lm_head = synth_matrix(host, mix["head"], vocab, H, seed, 2)
        self.out_norm = synth_normal(host, H, seed, 3, 0.1, 1.0)
        self.attn_norm, self.ffn_norm, self.w = [], [], []
        for L in range(n_layers):
            self.attn_norm.append(synth_normal(host, H, seed, 100 + 16 * L + 8, 0.1, 1.0))
            self.ffn_norm.append(synth_normal(host, H, seed, 100 + 16 * L + 9, 0.1, 1.0))
            for k, role in enumerate(MAT_ROLES):
                r, c = shapes[role]
                self.w.append(synth_matrix(host, mix[role], r, c, seed, 100 + 16 * L + k))
        self.wtype = np.array([mix[r] for _ in range(n_layers) for r in MAT_ROLES], dtype=np.int32)
        self._attn_ptrs = (C.c_void_p * n_layers)(*[a.ctypes.data for a in self.attn_norm])
        self._ffn_ptrs = (C.c_void_p * n_layers)(*[a.ctypes.data for a in self.ffn_norm])
        self._w_ptrs = (C.c_void_p * (7 * n_layers))(*[a.ctypes.data for a in self.w])

    def weight_bytes(self) -> int:
        return (self.tok_embd.nbytes + self.lm_head.nbytes + self.out_norm.nbytes +
                sum(a.nbytes for a in self.attn_norm) + sum(a.nbytes for a in self.ffn_norm) +
                sum(a.nbytes for a in self.w))

    def decode_struct(self) -> DecodeModelStruct:
        c = self.cfg
        return DecodeModelStruct(
            c["n_layers"], c["hidden"], c["ffn"], c["n_heads"], c["n_kv_heads"], c["head_dim"],
            c["vocab"], c["max_ctx"], c["theta"], c["eps"],
            self.mix["embd"], self.tok_embd.ctypes.data, self.out_norm.ctypes.data,
            self.mix["head"], self.lm_head.ctypes.data,
            C.addressof(self._attn_ptrs), C.addressof(self._ffn_ptrs),
            self.wtype.ctypes.data, C.addressof(self._w_ptrs))

    def kv_prefill(self, host, n_pos: int):
        """N(0,1) f16 caches for positions [0, n_pos): arrays [L][n_pos][kv_dim]."""
        c = self.cfg
        n = c["n_layers"] * n_pos * c["n_kv_heads"] * c["head_dim"]
        return (synth_normal_f16(host, n, self.seed, 10), synth_normal_f16(host, n, self.seed, 11))


class SynthGgufCfg(C.Structure):
    """vbs_synth_gguf_cfg_t (host/vbs_synth.h)."""
    _fields_ = [("n_layers", C.c_uint32), ("hidden", C.c_uint32), ("ffn", C.c_uint32),
                ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("vocab", C.c_uint32), ("context_length", C.c_uint32),
                ("rope_theta", C.c_float), ("rms_eps", C.c_float),
                ("embd_type", C.c_int), ("head_type", C.c_int), ("wtype", C.c_int * 7),
                ("seed", C.c_uint64), ("nthreads", C.c_int)]


def write_gguf(host, path: str, model: "SynthModel", context_length: int = 0):
    """The synthetic model `model` (same generator streams, same bytes) as a
    GGUF v3 file for the reference loader (src/vbs_gguf.c)."""
    c = model.cfg
    write_gguf_geometry(host, path, n_layers=c["n_layers"], hidden=c["hidden"], ffn=c["ffn"],
                        n_heads=c["n_heads"], n_kv_heads=c["n_kv_heads"],
                        head_dim=c["head_dim"], vocab=c["vocab"],
                        context_length=context_length or c["max_ctx"], mix=model.mix,
                        seed=model.seed, theta=c["theta"], eps=c["eps"])


def write_gguf_geometry(host, path: str, *, n_layers, hidden, ffn, n_heads, n_kv_heads,
                        head_dim, vocab, context_length, mix=None, seed=1234, theta=10000.0,
                        eps=1e-5):
    """A synthetic model of any size written straight to disk: the bytes
    SynthModel would hold for the same arguments, generated and written in
    32 MiB pieces, so 7B- and 70B-shaped files need no host copy."""
    mix = dict(Q4_K_M_MIX if mix is None else mix)
    cfg = SynthGgufCfg(n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, vocab,
                       context_length, theta, eps, mix["embd"], mix["head"],
                       (C.c_int * 7)(*[mix[r] for r in MAT_ROLES]), seed, _THREADS)
    err = C.create_string_buffer(512)
    if not host.vbs_synth_write_gguf(path.encode(), C.addressof(cfg), err, 512):
        raise RuntimeError(f"vbs_synth_write_gguf: {err.value.decode()}")


class HotKernels(C.Structure):
    """vbs_hot_kernels_t (include/vbs_hot_abi.h; the reference's vbs_hotpath.h:43-57)."""
    _fields_ = [("abi_version", C.c_uint32), ("name", C.c_char_p),
                ("matvec_q8_0", C.CFUNCTYPE(None, _P, _SZ, _SZ, _P, _P, _P)),
                ("matvec_q4_0", C.CFUNCTYPE(None, _P, _SZ, _SZ, _P, _P, _P)),
                ("matvec_q4_1", C.CFUNCTYPE(None, _P, _SZ, _SZ, _P, _P, _P, _P)),
                ("matvec_f32", C.CFUNCTYPE(None, _P, _SZ, _SZ, _P, _P)),
                ("matvec_f16", C.CFUNCTYPE(None, _P, _SZ, _SZ, _P, _P))]


class HotModule:
    """lib/libvbs_hot_gfx950.so: the CPU hot-kernel module (ABI v1) whose
    matvecs run on the device. Host numpy arrays in, host y out."""

    def __init__(self, path: str = HOT_LIB):
        self.path = path
        self.lib = _cdll(path)
        self.lib.vbs_hot_abi_version.restype = C.c_uint32
        self.lib.vbs_hot_kernels.restype = C.POINTER(HotKernels)
        self.lib.vbs_hot_gfx950_last_error.restype = C.c_char_p
        self.table = self.lib.vbs_hot_kernels().contents

    def abi_version(self) -> int:
        return self.lib.vbs_hot_abi_version()

    def last_error(self) -> str:
        return self.lib.vbs_hot_gfx950_last_error().decode()

    def matvec(self, t: int, w: np.ndarray, rows: int, cols: int, xq=None, qd=None, qsum=None,
               x=None) -> np.ndarray:
        y = np.empty(rows, np.float32)
        w = np.ascontiguousarray(w)
        tb = self.table
        if t == Q8_0:
            tb.matvec_q8_0(w.ctypes.data, rows, cols, xq.ctypes.data, qd.ctypes.data, y.ctypes.data)
        elif t == Q4_0:
            tb.matvec_q4_0(w.ctypes.data, rows, cols, xq.ctypes.data, qd.ctypes.data, y.ctypes.data)
        elif t == Q4_1:
            tb.matvec_q4_1(w.ctypes.data, rows, cols, xq.ctypes.data, qd.ctypes.data,
                           qsum.ctypes.data, y.ctypes.data)
        elif t == F32:
            tb.matvec_f32(w.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data)
        elif t == F16:
            tb.matvec_f16(w.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data)
        else:
            raise ValueError(f"type {t} is not in the hot-kernel table")
        return y


class Decoder:
    """vbs_decode_t over a backend table (g_vbs_hip_backend by default)."""

    def __init__(self, host, backend: Backend, model: SynthModel):
        self.host, self.model = host, model
        self._struct = model.decode_struct()
        err = C.create_string_buffer(512)
        self.h = host.vbs_decode_create(C.addressof(backend.ops), C.addressof(self._struct), err, 512)
        if not self.h:
            raise GpuError(f"vbs_decode_create: {err.value.decode()} / {backend.last_error()}")

    def load_kv(self, kc: np.ndarray, vc: np.ndarray, n_pos: int):
        if not self.host.vbs_decode_load_kv(self.h, kc.ctypes.data, vc.ctypes.data, n_pos):
            raise GpuError("vbs_decode_load_kv failed")

    def read_kv(self, n_pos: int):
        c = self.model.cfg
        n = c["n_layers"] * n_pos * c["n_kv_heads"] * c["head_dim"]
        kc, vc = np.empty(n, np.uint16), np.empty(n, np.uint16)
        if not self.host.vbs_decode_read_kv(self.h, kc.ctypes.data, vc.ctypes.data, n_pos):
            raise GpuError("vbs_decode_read_kv failed")
        return kc, vc

    def step(self, token: int, pos: int, want_logits=True):
        out = np.empty(self.model.cfg["vocab"], np.float32) if want_logits else None
        ok = self.host.vbs_decode_step(self.h, token, pos, out.ctypes.data if want_logits else None)
        if not ok:
            raise GpuError("vbs_decode_step failed")
        return out

    def greedy(self, token: int, pos: int, n: int):
        toks = np.empty(n, np.uint32)
        margins = np.empty(n, np.float32)
        if not self.host.vbs_decode_greedy(self.h, token, pos, n, toks.ctypes.data,
                                           margins.ctypes.data):
            raise GpuError("vbs_decode_greedy failed")
        return toks, margins

    def dispatch_count(self) -> int:
        return self.host.vbs_decode_dispatch_count(self.h)

    def close(self):
        if self.h:
            self.host.vbs_decode_destroy(self.h)
            self.h = None


class Gfx950ModelStruct(C.Structure):
    """vbs_gfx950_model_t (include/vbs_gfx950.h)."""
    _fields_ = [("n_layers", C.c_uint32), ("hidden", C.c_uint32), ("ffn", C.c_uint32),
                ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("vocab", C.c_uint32), ("max_ctx", C.c_uint32),
                ("rope_theta", C.c_float), ("rms_eps", C.c_float),
                ("embd_type", C.c_int), ("tok_embd", C.c_void_p), ("out_norm", C.c_void_p),
                ("head_type", C.c_int), ("lm_head", C.c_void_p),
                ("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p),
                ("wtype", C.c_void_p), ("wdata", C.c_void_p),
                ("kc", C.c_void_p), ("vc", C.c_void_p)]


class GraphDecoder:
    """vbs_gfx950_decoder over the device memory a Decoder uploaded.

    Shares the Decoder's weights and KV caches: both paths write the same
    cache rows, so a test may drive one and check the other's state."""

    def __init__(self, dev: DeviceLib, decoder: Decoder, max_steps: int = 256):
        self.dev, self.decoder = dev, decoder
        self.vocab = decoder.model.cfg["vocab"]
        self._view = Gfx950ModelStruct()
        if not decoder.host.vbs_decode_device_model(decoder.h, C.addressof(self._view)):
            raise GpuError("vbs_decode_device_model failed")
        h = C.c_void_p()
        dev.check(dev._decoder_create(C.addressof(self._view), max_steps, C.byref(h)),
                  "decoder_create")
        self.h = h.value

    def step(self, token: int, pos: int, want_logits=True):
        out = np.empty(self.vocab, np.float32) if want_logits else None
        self.dev.check(self.dev._decoder_step(self.h, token, pos,
                                              out.ctypes.data if want_logits else None),
                       "decoder_step")
        return out

    def greedy(self, token: int, pos: int, n: int, eager: bool = False):
        toks = np.empty(n, np.uint32)
        margins = np.empty(n, np.float32)
        fn = self.dev._decoder_greedy_eager if eager else self.dev._decoder_greedy
        self.dev.check(fn(self.h, token, pos, n, toks.ctypes.data, margins.ctypes.data),
                       "decoder_greedy")
        return toks, margins

    def attn_o_fallbacks(self):
        """(whether the O launch merges the attention, waves that merged
        their own heads since create): vbs_gfx950_decoder_attn_o_fallbacks."""
        c = C.c_uint32(0)
        r = self.dev._decoder_attn_o_fallbacks(self.h, C.byref(c))
        if r < 0:
            raise GpuError(f"decoder_attn_o_fallbacks: {self.dev.error()}")
        return bool(r), c.value

    def close(self):
        if self.h:
            self.dev._decoder_destroy(self.h)
            self.h = None


class BatchDecoder:
    """vbs_gfx950_bdecoder over the weights a Decoder uploaded, with `batch`
    sequences of their own: one device block per cache holding every
    sequence's [layer][max_ctx][kv_dim] f16 rows back to back."""

    def __init__(self, dev: DeviceLib, decoder: Decoder, batch: int, max_steps: int = 256):
        c = decoder.model.cfg
        self.dev, self.batch = dev, batch
        self.vocab, self.max_ctx = c["vocab"], c["max_ctx"]
        self.kvd = c["n_kv_heads"] * c["head_dim"]
        self.n_layers = c["n_layers"]
        self.seq = self.n_layers * self.max_ctx * self.kvd  # cache elements per sequence
        self.h = None
        self.kc = dev.alloc(2 * self.seq * batch)
        self.vc = dev.alloc(2 * self.seq * batch)
        self._view = Gfx950ModelStruct()
        if not decoder.host.vbs_decode_device_model(decoder.h, C.addressof(self._view)):
            raise GpuError("vbs_decode_device_model failed")
        self._view.kc, self._view.vc = self.kc, self.vc
        h = C.c_void_p()
        if not dev._bdecoder_create(C.addressof(self._view), batch, self.seq, max_steps,
                                    C.byref(h)):
            err = dev.error()
            self.close()
            raise GpuError(f"bdecoder_create: {err}")
        self.h = h.value

    def load_kv(self, b: int, kc: np.ndarray, vc: np.ndarray, n_pos: int):
        """Sequence b's caches from [n_layers][n_pos][kv_dim] f16 prefills."""
        rows = n_pos * self.kvd
        for L in range(self.n_layers):
            off = 2 * (b * self.seq + L * self.max_ctx * self.kvd)
            for dst, src in ((self.kc, kc), (self.vc, vc)):
                part = np.ascontiguousarray(src[L * rows:(L + 1) * rows])
                self.dev.check(self.dev._copy_h2d(dst + off, part.ctypes.data, part.nbytes),
                               "copy_h2d")

    def greedy(self, tokens0, pos0, n: int, eager: bool = False):
        """tokens (n, batch) and margins (n, batch) of every sequence's greedy run."""
        t0 = np.ascontiguousarray(tokens0, np.uint32)
        p0 = np.ascontiguousarray(pos0, np.uint32)
        toks = np.empty((n, self.batch), np.uint32)
        margins = np.empty((n, self.batch), np.float32)
        fn = self.dev._bdecoder_greedy_eager if eager else self.dev._bdecoder_greedy
        self.dev.check(fn(self.h, t0.ctypes.data, p0.ctypes.data, n, toks.ctypes.data,
                          margins.ctypes.data), "bdecoder_greedy")
        return toks, margins

    def step(self, tokens, pos) -> np.ndarray:
        """Logits (batch, vocab) of one step of every sequence fed tokens[b]
        at pos[b] (teacher forcing); the caches at pos[b] are written."""
        t = np.ascontiguousarray(tokens, np.uint32)
        p = np.ascontiguousarray(pos, np.uint32)
        out = np.empty((self.batch, self.vocab), np.float32)
        self.dev.check(self.dev._bdecoder_step(self.h, t.ctypes.data, p.ctypes.data,
                                               out.ctypes.data), "bdecoder_step")
        return out

    def read_kv(self, b: int, layer: int, pos: int):
        """Sequence b's f16 K and V rows (kv_dim each) of `layer` at `pos`."""
        off = 2 * (b * self.seq + (layer * self.max_ctx + pos) * self.kvd)
        out = []
        for src in (self.kc, self.vc):
            row = np.empty(self.kvd, np.uint16)
            self.dev.check(self.dev._copy_d2h(row.ctypes.data, src + off, row.nbytes), "copy_d2h")
            out.append(row)
        return out

    def close(self):
        if self.h:
            self.dev._bdecoder_destroy(self.h)
            self.h = None
        for p in (self.kc, self.vc):
            if p:
                self.dev.free(p)
        self.kc = self.vc = None
