"""TEST-ONLY driver of a backend table through the reference's own callers
(oracle/_ref/libvbs_callers_ref.so, built by `make -C oracle ref` from
src/vbs_specializer_bridge.c, src/vbs_fabric.c, src/vbs_slice_executor.c and
src/vbs_gguf.c where they lie, plus oracle/ref_callers.c).

RefEngine repeats vbs_engine_create's set-up (src/vbs_engine.c:43-56,
150-169): the GGUF opened by vbs_gguf_open, every tensor registered into a
vbs_fabric in file order, the activation, KV, logits and scratch buffers
allocated through the table, and the bridge bound to all of it. Its step()
makes the calls, in order and with the arguments, that the specializer emits
into forward_token for a llama model without Q/K norms
(src/vbs_specializer.c:231-349), followed by vbs_gpu_readback_logits as
verum_forward does (src/vbs_specializer.c:351-357). Every block pointer comes
from vbs_bridge_get_block_dptr, as the emitted verum_init takes it
(src/vbs_specializer.c:360-366).
"""
import ctypes as C
import os
import shutil
import tempfile

import numpy as np

import vbs_gfx950 as V
from oracle_lib import REF_CALLERS_SO

TIER_VRAM, TIER_HOST_PAGED = 0, 3
TYPE_SUFFIX = {V.F32: "f32", V.F16: "f16", V.Q4_0: "q4_0", V.Q4_1: "q4_1", V.Q8_0: "q8_0",
               V.Q4_K: "q4_k", V.Q6_K: "q6_k", V.LNS8: "lns8"}
_VP, _SZ, _U32, _F32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_float


def load_callers(tag, src=REF_CALLERS_SO, global_scope=False):
    """A private copy of the callers library: the bridge keeps its runtime
    and pipeline caches in file-scope statics, so each backend under test
    gets its own instance. `global_scope` loads it RTLD_GLOBAL, which a
    specializer module needs to find the bridge; only one such instance may
    live in a process (a module binds to the first one loaded)."""
    d = tempfile.mkdtemp(prefix="vbs_callers_")
    path = os.path.join(d, f"libvbs_callers_{tag}.so")
    shutil.copy(src, path)
    L = C.CDLL(path, mode=(os.RTLD_GLOBAL | os.RTLD_NOW) if global_scope else C.DEFAULT_MODE)
    sig = {
        "vbs_gguf_open": (_VP, [C.c_char_p, C.c_char_p, _SZ]),
        "vbs_gguf_close": (None, [_VP]),
        "vbs_gguf_get_float32_metadata": (C.c_bool, [_VP, C.c_char_p, C.POINTER(_F32)]),
        "vbs_gguf_get_uint32_metadata": (C.c_bool, [_VP, C.c_char_p, C.POINTER(_U32)]),
        "vbs_callers_profile": (_VP, [_VP, C.c_uint64]),
        "vbs_callers_profile_hip": (_VP, [_VP]),
        "vbs_callers_n_tensors": (_SZ, [_VP]),
        "vbs_callers_tensor": (_VP, [_VP, _SZ]),
        "vbs_callers_tensor_name": (C.c_char_p, [_VP]),
        "vbs_callers_tensor_type": (_U32, [_VP]),
        "vbs_callers_tensor_rows": (C.c_uint64, [_VP]),
        "vbs_callers_tensor_cols": (C.c_uint64, [_VP]),
        "vbs_callers_tensor_data": (_VP, [_VP, _VP]),
        "vbs_callers_block_tier": (C.c_int, [_VP, _SZ]),
        "vbs_fabric_create": (_VP, [_VP, _VP, _SZ, _SZ, C.c_char_p]),
        "vbs_fabric_free": (None, [_VP]),
        "vbs_fabric_register_tensor": (_VP, [_VP, _VP, _VP, C.c_int, _VP]),
        "vbs_bridge_bind_runtime": (None, [_VP, _VP, _VP]),
        "vbs_bridge_set_activations": (None, [_VP, _VP, _VP, _VP, _VP]),
        "vbs_bridge_set_scratch": (None, [_VP, _SZ]),
        "vbs_bridge_get_block_dptr": (_VP, [_SZ]),
        "vbs_gpu_get_act_buffer_a": (_VP, []), "vbs_gpu_get_act_buffer_b": (_VP, []),
        "vbs_gpu_get_kv_k": (_VP, []), "vbs_gpu_get_kv_v": (_VP, []),
        "vbs_gpu_get_logits": (_VP, []), "vbs_gpu_get_scratch": (_VP, [_SZ]),
        "vbs_gpu_dispatch_norm": (None, [_VP, _VP, _VP, _SZ, _F32]),
        "vbs_gpu_dispatch_rope": (None, [_VP, _U32, _SZ, _SZ, _F32]),
        "vbs_gpu_dispatch_cache": (None, [_VP, _VP, _VP, _VP, _U32, _U32, _U32, _SZ]),
        "vbs_gpu_dispatch_attn": (None, [_VP, _VP, _VP, _VP, _U32, _U32, _U32, _SZ, _SZ, _SZ]),
        "vbs_gpu_dispatch_silu": (None, [_VP, _VP, _VP, _SZ]),
        "vbs_gpu_dispatch_add": (None, [_VP, _VP, _VP, _SZ]),
        "vbs_gpu_readback_logits": (None, [_VP, _VP, _SZ]),
        "vbs_slice_executor_create": (_VP, [_VP, _VP, _VP, _SZ, C.c_char_p, _SZ]),
        "vbs_slice_executor_free": (None, [_VP]),
        "vbs_slice_executor_run_linear": (C.c_bool, [_VP, _VP, _VP, _VP, C.c_char_p, _SZ]),
        "vbs_callers_specialize": (_VP, [_VP, _VP, _VP, _VP, _U32, C.c_char_p, C.c_char_p, _SZ]),
        "vbs_callers_jit_forward": (None, [_VP, _VP, _SZ, _VP]),
        "vbs_callers_jit_reset": (None, [_VP]),
        "vbs_callers_jit_free": (None, [_VP]),
        "vbs_callers_jit_path": (C.c_char_p, [_VP]),
        "vbs_callers_jit_n_plans": (_SZ, [_VP]),
    }
    for suffix in TYPE_SUFFIX.values():
        sig[f"vbs_gpu_dispatch_vram_{suffix}"] = (None, [_VP, _VP, _VP, _SZ, _SZ])
        if suffix != "lns8":
            sig[f"vbs_gpu_dispatch_embed_{suffix}"] = (None, [_VP, _U32, _VP, _SZ])
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    return L


class GgufModel:
    """A GGUF file opened by the reference's loader (src/vbs_gguf.c)."""

    def __init__(self, L, path):
        err = C.create_string_buffer(512)
        self.L, self.ptr = L, L.vbs_gguf_open(path.encode(), err, 512)
        if not self.ptr:
            raise RuntimeError(f"vbs_gguf_open: {err.value.decode()}")
        self.tensors = [L.vbs_callers_tensor(self.ptr, i)
                        for i in range(L.vbs_callers_n_tensors(self.ptr))]
        self.index = {L.vbs_callers_tensor_name(t).decode(): i for i, t in enumerate(self.tensors)}

    def tensor(self, name):
        return self.tensors[self.index[name]]

    def shape(self, name):
        t = self.tensor(name)
        return (int(self.L.vbs_callers_tensor_rows(t)), int(self.L.vbs_callers_tensor_cols(t)),
                int(self.L.vbs_callers_tensor_type(t)))

    def u32(self, key):
        v = _U32()
        assert self.L.vbs_gguf_get_uint32_metadata(self.ptr, key.encode(), C.byref(v)), key
        return int(v.value)

    def f32(self, key):
        v = _F32()
        assert self.L.vbs_gguf_get_float32_metadata(self.ptr, key.encode(), C.byref(v)), key
        return float(v.value)

    def close(self):
        if self.ptr:
            self.L.vbs_gguf_close(self.ptr)
            self.ptr = None


class RefEngine:
    """vbs_engine_create's set-up and the specializer's emitted token step
    over `backend` (a vbs_gfx950.Backend, initialised)."""

    def __init__(self, L, backend, gguf_path, tier=TIER_VRAM, vram_bytes=8 << 30,
                 profile="fixed"):
        self.L, self.be = L, backend
        self.model = m = GgufModel(L, gguf_path)
        self.n_layers = m.u32("llama.block_count")
        self.H = m.u32("llama.embedding_length")
        self.F = m.u32("llama.feed_forward_length")
        self.nq = m.u32("llama.attention.head_count")
        self.nkv = m.u32("llama.attention.head_count_kv")
        self.hd = m.u32("llama.rope.dimension_count")
        self.vocab = m.u32("llama.vocab_size")
        self.kv_cap = m.u32("llama.context_length")
        self.theta = m.f32("llama.rope.freq_base")
        self.eps = m.f32("llama.attention.layer_norm_rms_epsilon")
        self.kvd = self.nkv * self.hd
        dev = self.dev = backend.device()
        ops = self.ops = C.addressof(backend.ops)
        # "fixed": one GPU with vram_bytes free; "hip": the profile the
        # reference's profiler derives from the device's own byte counts
        self.sys = (L.vbs_callers_profile_hip(C.cast(dev, _VP)) if profile == "hip" else
                    L.vbs_callers_profile(C.cast(dev, _VP), vram_bytes))
        self.fabric = L.vbs_fabric_create(self.sys, ops, 16, 0, None)
        for t in m.tensors:  # src/vbs_engine.c:51-56
            L.vbs_fabric_register_tensor(self.fabric, t, L.vbs_callers_tensor_data(m.ptr, t), tier,
                                         C.cast(dev, _VP))
        self.tiers_at_registration = [L.vbs_callers_block_tier(self.fabric, i)
                                      for i in range(len(m.tensors))]
        H, F, qd = self.H, self.F, self.nq * self.hd
        big = max(H, F, qd, self.kvd)
        kv_bytes = self.n_layers * self.kv_cap * self.kvd * 2
        self.bufs = [backend.alloc(H * 4), backend.alloc(H * 4), backend.alloc(kv_bytes),
                     backend.alloc(kv_bytes), backend.alloc(self.vocab * 4)]
        self.scratch = [backend.alloc(big * 4) for _ in range(10)]
        vp = [C.cast(b, _VP) for b in self.bufs]
        L.vbs_bridge_bind_runtime(C.cast(dev, _VP), ops, self.fabric)  # src/vbs_engine.c:167-169
        L.vbs_bridge_set_activations(*vp)
        arr = (_VP * 10)(*[C.cast(b, _VP) for b in self.scratch])
        L.vbs_bridge_set_scratch(arr, 10)
        # verum_init: one block pointer per weight, faulted in on first use
        self.blk = {name: L.vbs_bridge_get_block_dptr(i) for name, i in m.index.items()}
        assert all(self.blk.values()), [n for n, p in self.blk.items() if not p]
        self.tiers_after_init = [L.vbs_callers_block_tier(self.fabric, i)
                                 for i in range(len(m.tensors))]

    def zero_kv(self):
        z = np.zeros(self.n_layers * self.kv_cap * self.kvd, np.uint16)
        for b in (self.bufs[2], self.bufs[3]):
            assert self.be.ops.copy_to_device(b, z.ctypes.data, z.nbytes)

    def _vram(self, name, x, y):
        rows, cols, t = self.model.shape(name)
        getattr(self.L, f"vbs_gpu_dispatch_vram_{TYPE_SUFFIX[t]}")(self.blk[name], x, y, rows, cols)

    def step(self, tok, pos):
        """forward_token(tok) at position `pos`, then the logits read back."""
        L, s = self.L, self.L.vbs_gpu_get_scratch
        STREAM, TMP = L.vbs_gpu_get_act_buffer_a(), L.vbs_gpu_get_act_buffer_b()
        QB, KB, VB, AB, GATE, UP, HIDDEN, NORMED = (s(i) for i in range(8))
        KC, VC = L.vbs_gpu_get_kv_k(), L.vbs_gpu_get_kv_v()
        H, F, hd, nq, nkv = self.H, self.F, self.hd, self.nq, self.nkv
        _, _, et = self.model.shape("token_embd.weight")
        getattr(L, f"vbs_gpu_dispatch_embed_{TYPE_SUFFIX[et]}")(self.blk["token_embd.weight"],
                                                                tok, STREAM, H)
        for layer in range(self.n_layers):
            b = f"blk.{layer}."
            L.vbs_gpu_dispatch_norm(self.blk[b + "attn_norm.weight"], STREAM, NORMED, H, self.eps)
            self._vram(b + "attn_q.weight", NORMED, QB)
            L.vbs_gpu_dispatch_rope(QB, pos, hd, nq, self.theta)
            self._vram(b + "attn_k.weight", NORMED, KB)
            L.vbs_gpu_dispatch_rope(KB, pos, hd, nkv, self.theta)
            self._vram(b + "attn_v.weight", NORMED, VB)
            L.vbs_gpu_dispatch_cache(KB, VB, KC, VC, pos, layer, self.kv_cap, self.kvd)
            L.vbs_gpu_dispatch_attn(QB, KC, VC, AB, pos, layer, self.kv_cap, nq, nkv, hd)
            self._vram(b + "attn_output.weight", AB, TMP)
            L.vbs_gpu_dispatch_add(STREAM, TMP, STREAM, H)
            L.vbs_gpu_dispatch_norm(self.blk[b + "ffn_norm.weight"], STREAM, NORMED, H, self.eps)
            self._vram(b + "ffn_gate.weight", NORMED, GATE)
            self._vram(b + "ffn_up.weight", NORMED, UP)
            L.vbs_gpu_dispatch_silu(GATE, UP, HIDDEN, F)
            self._vram(b + "ffn_down.weight", HIDDEN, TMP)
            L.vbs_gpu_dispatch_add(STREAM, TMP, STREAM, H)
        L.vbs_gpu_dispatch_norm(self.blk["output_norm.weight"], STREAM, NORMED, H, self.eps)
        self._vram("output.weight", NORMED, L.vbs_gpu_get_logits())
        out = np.empty(self.vocab, np.float32)
        L.vbs_gpu_readback_logits(L.vbs_gpu_get_logits(), out.ctypes.data, self.vocab)
        return out

    def specialize(self, workdir):
        """vbs_engine_compile over this set-up: the reference's graph, planner
        and specializer emit the model's C module into `workdir`, compile it
        with the system compiler and bind it (verum_init). Needs the library
        loaded with global_scope=True."""
        err = C.create_string_buffer(1024)
        jit = self.L.vbs_callers_specialize(self.model.ptr, self.sys, self.fabric, self.ops,
                                            self.kv_cap, workdir.encode(), err, 1024)
        if not jit:
            raise RuntimeError(f"specializer: {err.value.decode()}")
        return Module(self.L, jit, self.vocab)

    def close(self):
        for b in self.bufs + self.scratch:
            self.be.ops.free_buffer(b)
        self.bufs, self.scratch = [], []
        if self.fabric:
            self.L.vbs_fabric_free(self.fabric)
            self.fabric = None
        self.model.close()


class SliceExecutor:
    """src/vbs_slice_executor.c over a backend: a packed tensor streamed
    through two `window` byte staging windows (convention B tiles)."""

    def __init__(self, L, backend, model: GgufModel, window):
        err = C.create_string_buffer(512)
        self.L, self.be, self.model = L, backend, model
        self.ptr = L.vbs_slice_executor_create(model.ptr, C.addressof(backend.ops),
                                               C.cast(backend.device(), _VP), window, err, 512)
        if not self.ptr:
            raise RuntimeError(f"vbs_slice_executor_create: {err.value.decode()}")

    def run_linear(self, name, x_buf, y_buf):
        err = C.create_string_buffer(512)
        ok = self.L.vbs_slice_executor_run_linear(self.ptr, self.model.tensor(name),
                                                  C.cast(x_buf, _VP), C.cast(y_buf, _VP), err, 512)
        return ok, err.value.decode()

    def close(self):
        if self.ptr:
            self.L.vbs_slice_executor_free(self.ptr)
            self.ptr = None


class Module:
    """A specializer-emitted module bound to a RefEngine's set-up."""

    def __init__(self, L, jit, vocab):
        self.L, self.jit, self.vocab = L, jit, vocab
        self.path = L.vbs_callers_jit_path(jit).decode()
        self.n_plans = int(L.vbs_callers_jit_n_plans(jit))

    def forward(self, tokens):
        """verum_forward(tokens): one token step per token at the module's
        running position, then the logits read back."""
        t = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.vocab, np.float32)
        self.L.vbs_callers_jit_forward(self.jit, t.ctypes.data, t.size, out.ctypes.data)
        return out

    def reset(self):
        self.L.vbs_callers_jit_reset(self.jit)

    def close(self):
        if self.jit:
            self.L.vbs_callers_jit_free(self.jit)
            self.jit = None
