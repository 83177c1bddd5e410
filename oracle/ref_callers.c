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
