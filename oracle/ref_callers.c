/* ref_callers.c -- TEST-ONLY. The reference's own caller side of the backend
 * table, for driving g_vbs_hip_backend the way Verum does:
 *
 *   - the specializer bridge, src/vbs_specializer_bridge.c, compiled where it
 *     lies (included below through -I$(REF)/src, not copied), with the two
 *     Q4_K entry points it lacks added after it. The bridge declares linear
 *     and embedding dispatch for Q8_0/Q4_0/Q4_1/Q6_K/F16/F32/LNS8 only
 *     (include/vbs_specializer_bridge.h:36-60), which is why the specializer
 *     refuses Q4_K models (src/vbs_specializer.c:69-71, 203-221). The two
 *     functions have the bodies of the bridge's Q6_K pair with the type
 *     changed; they are the whole reference-side change a Q4_K_M model needs;
 *   - a one-GPU system profile for vbs_fabric_create (the fields
 *     src/vbs_fabric.c reads: n_gpus, gpus[].device, gpus[].free_vram_bytes),
 *     and accessors for the reference's GGUF model and tensor structs, so the
 *     Python tests need no restated layout of them.
 *
 * Linked by oracle/Makefile (ref target) with src/vbs_fabric.c,
 * src/vbs_slice_executor.c and src/vbs_gguf.c from the reference tree into
 * oracle/_ref/libvbs_callers_ref.so.
 */
#include "vbs_specializer_bridge.c"

#include <string.h>

#include "vbs_profiler.h"

void vbs_gpu_dispatch_vram_q4_k(void *w, void *in, void *out, size_t r, size_t c) {
    dispatch_linear(VBS_GGML_TYPE_Q4_K, w, in, out, r, c);
}

void vbs_gpu_dispatch_embed_q4_k(void *w, uint32_t token, void *out, size_t dim) {
    dispatch_embed_typed(VBS_GGML_TYPE_Q4_K, w, token, out, dim);
}

const vbs_system_profile_t *vbs_callers_profile(vbs_device_t *dev, uint64_t free_vram) {
    static vbs_system_profile_t p;
    memset(&p, 0, sizeof p);
    p.n_gpus = 1;
    p.gpus[0].device = dev;
    p.gpus[0].total_vram_bytes = free_vram;
    p.gpus[0].free_vram_bytes = free_vram;
    p.gpus[0].max_alloc_bytes = free_vram;
    p.total_vram_bytes = free_vram;
    return &p;
}

/* The system profile vbs_profiler_scan_system builds on a machine whose only
 * GPU backend is HIP: its HIP branch (src/vbs_profiler.c:194-210) takes the
 * device's max_working_set_bytes as total VRAM, 85% of it as free, and
 * max_buffer_bytes as the largest allocation. The bandwidth it measures is
 * left at zero (the planner then keeps device 0). */
const vbs_system_profile_t *vbs_callers_profile_hip(vbs_device_t *dev) {
    static vbs_system_profile_t p;
    memset(&p, 0, sizeof p);
    vbs_gpu_profile_t *g = &p.gpus[0];
    p.n_gpus = 1;
    snprintf(g->name, sizeof g->name, "%s", dev->name);
    g->type = VBS_BACKEND_HIP;
    g->device = dev;
    g->total_vram_bytes = dev->max_working_set_bytes;
    g->free_vram_bytes = dev->max_working_set_bytes * 85 / 100;
    g->max_alloc_bytes = dev->max_buffer_bytes;
    g->sm_count = 60;
    g->warp_size = 64;
    p.total_vram_bytes = g->total_vram_bytes;
    return &p;
}

size_t vbs_callers_n_tensors(const vbs_gguf_model_t *m) { return m->n_tensors; }
const vbs_tensor_t *vbs_callers_tensor(const vbs_gguf_model_t *m, size_t i) {
    return i < m->n_tensors ? &m->tensors[i] : NULL;
}
const char *vbs_callers_tensor_name(const vbs_tensor_t *t) { return t->name; }
uint32_t vbs_callers_tensor_type(const vbs_tensor_t *t) { return (uint32_t)t->type; }
uint64_t vbs_callers_tensor_rows(const vbs_tensor_t *t) { return t->rows; }
uint64_t vbs_callers_tensor_cols(const vbs_tensor_t *t) { return t->columns; }
uint64_t vbs_callers_tensor_bytes(const vbs_tensor_t *t) { return t->byte_length; }
const void *vbs_callers_tensor_data(const vbs_gguf_model_t *m, const vbs_tensor_t *t) {
    return (const uint8_t *)m->map + t->data_offset;
}
/* Where the fabric keeps block i: its tier (vbs_memory_tier_t) and whether a
 * device buffer holds it. */
int vbs_callers_block_tier(const vbs_fabric_t *f, size_t i) {
    return i < f->n_blocks ? (int)f->blocks[i]->current_tier : -1;
}

/* ---- The specializer's emitted module (src/vbs_specializer.c) -------------
 *
 * vbs_engine_compile (src/vbs_engine.c:174-223) turns the model into a C
 * module and runs it: vbs_graph_compile -> vbs_planner_build ->
 * vbs_specializer_emit_source -> vbs_specializer_compile (the system C
 * compiler) -> vbs_specializer_load -> verum_init(fabric, backend). The
 * module's forward pass then calls the bridge functions above through the
 * process's global symbol scope, so this library must be loaded with
 * RTLD_GLOBAL (one instance per process) before a module is loaded.
 *
 * Two pieces of the engine that cannot be built here are restated:
 *   - the layer-energy table vbs_engine.c:416-420 owns, which the emitter
 *     reads (vbs_specializer.c:259-275): every layer alive, as
 *     vbs_engine_reset_energy leaves it;
 *   - the model profile of vbs_profiler_scan_model (src/vbs_profiler.c:
 *     290-355): vbs_profiler.c itself also probes the CUDA and Vulkan
 *     backends, whose sources embed prebuilt kernel images this build does
 *     not use, so it does not link here.
 */
#include "vbs_graph.h"
#include "vbs_planner.h"
#include "vbs_specializer.h"
#include "vbs_engine.h"

float g_vbs_layer_energy[VBS_MAX_LAYERS];

/* The fields vbs_profiler_scan_model fills, from the same metadata keys and
 * name rules, with the KV capacity the engine stores after sizing its caches
 * (src/vbs_engine.c:138-139). NULL if an essential dimension is missing. */
vbs_model_profile_t *vbs_callers_model_profile(const vbs_gguf_model_t *m, uint32_t kv_capacity) {
    vbs_model_profile_t *mp = calloc(1, sizeof *mp);
    if (!mp) return NULL;
    mp->model = m;
    mp->n_tensor_profiles = m->n_tensors;
    mp->tensor_profiles = calloc(m->n_tensors ? m->n_tensors : 1, sizeof *mp->tensor_profiles);
    for (size_t i = 0; i < m->n_tensors; i++) {
        const vbs_tensor_t *t = &m->tensors[i];
        vbs_tensor_profile_t *tp = &mp->tensor_profiles[i];
        int hot = strstr(t->name, "token_embd") || strstr(t->name, "output") || strstr(t->name, "norm");
        int warm = !hot && (strstr(t->name, "attn") || strstr(t->name, ".q.") ||
                            strstr(t->name, ".k.") || strstr(t->name, ".v."));
        tp->tensor = t;
        tp->bytes = t->byte_length;
        tp->is_hot_path = hot;
        tp->access_frequency = hot ? 100 : warm ? 50 : 10;
        tp->estimated_compute_cost = 2.0 * (double)t->byte_length;
        mp->total_model_bytes += t->byte_length;
        if (hot) mp->hot_working_set_bytes += t->byte_length;
        else if (warm) mp->warm_working_set_bytes += t->byte_length;
        else mp->cold_working_set_bytes += t->byte_length;
        if (hot && (strstr(t->name, "token_embd.weight") || strstr(t->name, "output.weight")))
            mp->vocab_size = (uint32_t)t->rows;
    }
    vbs_gguf_get_uint32_metadata(m, "llama.block_count", &mp->n_layers);
    vbs_gguf_get_uint32_metadata(m, "llama.attention.head_count", &mp->n_heads);
    vbs_gguf_get_uint32_metadata(m, "llama.attention.head_count_kv", &mp->n_kv_heads);
    vbs_gguf_get_uint32_metadata(m, "llama.embedding_length", &mp->embedding_dim);
    vbs_gguf_get_uint32_metadata(m, "llama.context_length", &mp->context_length);
    if (mp->n_heads && mp->embedding_dim) mp->head_dim = mp->embedding_dim / mp->n_heads;
    mp->rope_theta = 10000.0f;
    mp->rms_eps = 1e-5f;
    vbs_gguf_get_float32_metadata(m, "llama.rope.freq_base", &mp->rope_theta);
    vbs_gguf_get_float32_metadata(m, "llama.attention.layer_norm_rms_epsilon", &mp->rms_eps);
    if (!mp->n_layers || !mp->n_heads || !mp->n_kv_heads || !mp->embedding_dim ||
        !mp->vocab_size || !mp->head_dim || !mp->context_length) {
        free(mp->tensor_profiles);
        free(mp);
        return NULL;
    }
    mp->kv_ctx_capacity = kv_capacity;
    return mp;
}

typedef struct {
    vbs_graph_t *graph;
    vbs_execution_plan_t *plan;
    vbs_model_profile_t *mp;
    vbs_specialized_binary_t *bin;
} vbs_callers_jit_t;

void vbs_callers_jit_free(vbs_callers_jit_t *j) {
    if (!j) return;
    if (j->bin) vbs_specializer_free(j->bin);
    if (j->plan) vbs_planner_free(j->plan);
    if (j->graph) vbs_graph_free(j->graph);
    if (j->mp) { free(j->mp->tensor_profiles); free(j->mp); }
    free(j);
}

/* vbs_engine_compile's steps in its order, without the module cache lookup
 * (every call emits and compiles afresh into `dir`). The system profile is
 * vbs_callers_profile's; `fabric` already holds every tensor, registered in
 * file order as vbs_engine_create does (src/vbs_engine.c:51-56), and the
 * bridge is bound. The emitted source is kept at dir/verum_<hash>.c. */
vbs_callers_jit_t *vbs_callers_specialize(const vbs_gguf_model_t *m, const vbs_system_profile_t *sys,
                                          vbs_fabric_t *fabric, const vbs_backend_ops_t *backend,
                                          uint32_t kv_capacity, const char *dir,
                                          char *err, size_t err_cap) {
    vbs_callers_jit_t *j = calloc(1, sizeof *j);
    char hash[65] = {0}, src[1024], bin[1024];
    double compile_sec = 0;
    for (size_t i = 0; i < VBS_MAX_LAYERS; i++) g_vbs_layer_energy[i] = 1.0f;
    if (!j) { snprintf(err, err_cap, "out of memory"); return NULL; }
    if (!(j->mp = vbs_callers_model_profile(m, kv_capacity))) {
        snprintf(err, err_cap, "model profile refused");
        goto fail;
    }
    if (!(j->graph = vbs_graph_compile(m, err, err_cap))) goto fail;
    if (!(j->plan = vbs_planner_build(j->graph, sys, j->mp, fabric))) {
        snprintf(err, err_cap, "Planner failed to generate execution plan");
        goto fail;
    }
    vbs_specializer_compute_hash(j->graph, sys, j->plan, hash, sizeof hash);
    snprintf(src, sizeof src, "%s/verum_%s.c", dir, hash);
    snprintf(bin, sizeof bin, "%s/verum_%s%s", dir, hash, VBS_DYLIB_EXT);
    if (!vbs_specializer_emit_source(j->graph, sys, j->plan, j->mp, src)) {
        snprintf(err, err_cap, "Failed emitting bespoke C source for specialization");
        goto fail;
    }
    if (!vbs_specializer_compile(src, bin, sys, &compile_sec)) {
        snprintf(err, err_cap, "Specializer compilation failed");
        goto fail;
    }
    if (!(j->bin = vbs_specializer_load(bin, hash))) {
        snprintf(err, err_cap, "Failed loading specialized binary module: %s", vbs_dlerror());
        goto fail;
    }
    j->bin->compile_time_sec = compile_sec;
    j->bin->n_kernels_emitted = j->plan->n_plans;
    j->bin->init_fn(fabric, (void *)backend);
    return j;
fail:
    vbs_callers_jit_free(j);
    return NULL;
}

/* vbs_engine_forward (src/vbs_engine.c:225-229): the module's verum_forward. */
void vbs_callers_jit_forward(vbs_callers_jit_t *j, const uint32_t *tokens, size_t n, float *logits) {
    j->bin->forward_fn(tokens, n, logits);
}

void vbs_callers_jit_reset(vbs_callers_jit_t *j) {
    if (j->bin->reset_cache_fn) j->bin->reset_cache_fn();
}

const char *vbs_callers_jit_path(const vbs_callers_jit_t *j) { return j->bin->binary_path; }
size_t vbs_callers_jit_n_plans(const vbs_callers_jit_t *j) { return j->plan->n_plans; }
