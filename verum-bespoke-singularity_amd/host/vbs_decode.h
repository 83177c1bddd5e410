/* vbs_decode.h — the caller side of one decode step, driven through a
 * vbs_backend_ops_t table exactly as Verum's generated forward pass drives
 * its bridge (src/vbs_specializer.c:231-359, src/vbs_specializer_bridge.c).
 *
 * It owns what vbs_engine_create allocates for the generated module
 * (src/vbs_engine.c:84-164): the two activation buffers, the ten named
 * scratch buffers, the logits buffer and the two f16 KV caches sized
 * [n_layers][max_ctx][n_kv_heads*head_dim]; it uploads every weight as the
 * fabric does (src/vbs_fabric.c:81-93) and then issues, per token,
 * embed -> per layer [attn_norm, Q, rope, K, rope, V, cache, attention, O,
 * add, ffn_norm, gate, up, silu, down, add] -> output_norm -> lm_head ->
 * logits readback, with the bridge's scalar arguments.
 */
#ifndef VBS_DECODE_H
#define VBS_DECODE_H

#include "vbs_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Host-side description of a llama-style model in GGUF block layout. The
 * seven per-layer matrices are q, k, v, o, gate, up, down (rows x cols:
 * q nq*hd x H, k/v nkv*hd x H, o H x nq*hd, gate/up F x H, down H x F). */
typedef struct {
    uint32_t n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, vocab, max_ctx;
    float rope_theta, rms_eps;
    int embd_type;
    const uint8_t *tok_embd;
    const float *out_norm;
    int head_type;
    const uint8_t *lm_head;
    const float *const *attn_norm;
    const float *const *ffn_norm;
    const int *wtype;              /* n_layers x 7 */
    const uint8_t *const *wdata;   /* n_layers x 7 */
} vbs_decode_model_t;

typedef struct vbs_decode vbs_decode_t;

/* Uploads the model and allocates runtime buffers on device 0 of `ops`
 * (ops->init() must already have succeeded). NULL + err on failure. */
vbs_decode_t *vbs_decode_create(const vbs_backend_ops_t *ops, const vbs_decode_model_t *m,
                                char *err, size_t err_cap);
void vbs_decode_destroy(vbs_decode_t *d);

/* Overwrite positions [0, n_pos) of both caches of every layer
 * (host arrays laid out [layer][n_pos][kv_dim], f16 bits). */
int vbs_decode_load_kv(vbs_decode_t *d, const uint16_t *kc, const uint16_t *vc, uint32_t n_pos);
/* Read back positions [0, n_pos) of both caches. */
int vbs_decode_read_kv(vbs_decode_t *d, uint16_t *kc, uint16_t *vc, uint32_t n_pos);

/* One token at position `pos` (attends to 0..pos); logits may be NULL to
 * skip the readback. Returns 1 on success. */
int vbs_decode_step(vbs_decode_t *d, uint32_t token, uint32_t pos, float *logits);

/* Greedy decode: feed `token` at `pos`, take the first maximum of the logits
 * (as main.c:929-932), repeat n times. tokens_out[i] is the i-th argmax;
 * margins_out (optional) the top-1 minus top-2 logit of each step. */
int vbs_decode_greedy(vbs_decode_t *d, uint32_t token, uint32_t pos, uint32_t n,
                      uint32_t *tokens_out, float *margins_out);

/* Dispatches issued by the last vbs_decode_step. */
uint32_t vbs_decode_dispatch_count(const vbs_decode_t *d);

/* Total bytes of weights resident on the device. */
uint64_t vbs_decode_weight_bytes(const vbs_decode_t *d);

/* Device-side view of the uploaded model (weights, norms and KV caches as
 * device pointers) for the gfx950 graph decoder, vbs_gfx950_decoder_create
 * (include/vbs_gfx950.h). Valid while `d` lives. */
int vbs_decode_device_model(vbs_decode_t *d, void *out_vbs_gfx950_model_t);

#ifdef __cplusplus
}
#endif
#endif
