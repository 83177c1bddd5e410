/* vbs_gfx950.h — C ABI of libvbs_gfx950.so, the MI355X (gfx950) device
 * library behind Verum's HIP backend slot.
 *
 * The reference's HIP backend (src/vbs_backend_hip.c) dlopens the ROCm
 * runtime and host-stages every op through src/vbs_host_math.h. This library
 * replaces that: it owns one device, one in-order HIP stream and the
 * hand-written gfx950 kernels, and exposes them through plain pointers and
 * sizes (no HIP or torch types). The C11 shim
 * (host/vbs_backend_gfx950.c) dlopens it, checks vbs_gfx950_abi_version()
 * and every symbol below, and maps the vbs_backend_ops_t slots onto it.
 *
 * Conventions
 *   - Every function returns 1 on success and 0 on failure; the reason is
 *     then in vbs_gfx950_last_error(). Nothing aborts or throws.
 *   - Device pointers come from vbs_gfx950_alloc (or point inside such an
 *     allocation). All work is enqueued on the library's single stream in
 *     call order; copies to the host wait for it, so results are visible to
 *     the caller exactly as with the reference's synchronous backends.
 *   - `type` values are GGUF type ids (vbs_ggml_type_t): F32 0, F16 1,
 *     Q4_0 2, Q4_1 3, Q8_0 8, Q4_K 12, Q6_K 14, LNS8 40.
 */
#ifndef VBS_GFX950_H
#define VBS_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VBS_GFX950_ABI_VERSION 3

/* ---- library / device ------------------------------------------------ */

/* ABI version of the loaded library; the shim refuses a mismatch, as
 * vbs_hot_load does for the CPU hot table (src/vbs_hotpath.c:96-101). */
int vbs_gfx950_abi_version(void);

/* Probe and open the first gfx950 device. Idempotent; a failure is sticky and
 * explained by vbs_gfx950_last_error(). Replaces hip_init
 * (src/vbs_backend_hip.c:149-225). */
int vbs_gfx950_init(void);

/* Last failure reason ("ok" when none). Replaces vbs_hip_last_error
 * (src/vbs_backend_hip.c:110). */
const char *vbs_gfx950_last_error(void);

/* Number of usable devices (0 or 1: the backend drives one GPU). Replaces
 * hip_get_device_count (src/vbs_backend_hip.c:227). */
int vbs_gfx950_device_count(void);

/* Name, total and free HBM of device `index`. Fills what the reference's HIP
 * backend left unset (max_working_set_bytes / max_buffer_bytes,
 * src/vbs_backend_hip.c:214-220). */
int vbs_gfx950_device_info(int index, char *name, size_t name_cap, uint64_t *total_bytes,
                           uint64_t *free_bytes);

/* ---- memory (src/vbs_backend_hip.c:230-264) ---------------------------- */

void *vbs_gfx950_alloc(size_t bytes);          /* device memory, 256-B aligned */
int vbs_gfx950_free(void *dptr);
void *vbs_gfx950_host_alloc(size_t bytes);     /* pinned host memory */
int vbs_gfx950_host_free(void *hptr);
/* Stream-ordered copies that have completed when they return. */
int vbs_gfx950_copy_h2d(void *dst, const void *src, size_t bytes);
int vbs_gfx950_copy_d2h(void *dst, const void *src, size_t bytes);
int vbs_gfx950_copy_d2d(void *dst, const void *src, size_t bytes);
/* Wait for all enqueued work (src/vbs_backend_hip.c:548-551). */
int vbs_gfx950_synchronize(void);

/* ---- hot-path kernels --------------------------------------------------- */

/* 1 if `type` has a gfx950 linear kernel: F32, F16, Q4_0, Q4_1, Q8_0, Q4_K,
 * Q6_K, and LNS8 (the bridge's seventh dispatch type). Mirrors the reference's refusal contract (vbs_host_type_supported,
 * src/vbs_host_math.h:69-89, and the Q8_K refusal checked by
 * src/vbs_backend_test.c:952-955). */
int vbs_gfx950_linear_supported(int type);

/* y[row_off + r] (+)= sum_c deq(W[r, c]) * x[col_off + c] for r < rows,
 * W row-major in native GGUF blocks, row stride = (cols / block) * bytes.
 * Replaces hip_dispatch_linear_tile (src/vbs_backend_hip.c:346-394); same
 * meaning as vbs_host_linear_tile (src/vbs_host_math.h:223-267) with fp32
 * accumulation. */
int vbs_gfx950_linear(int type, const void *w, const float *x, float *y, uint32_t cols,
                      uint32_t rows, uint32_t col_off, uint32_t row_off, int accumulate);

/* out[0..dim) = deq(row `token` of table w), bit-identical to
 * vbs_host_embed_row (src/vbs_host_math.h:136-142). The EMBEDDING op of
 * src/vbs_backend_hip.c:405-423. */
int vbs_gfx950_embed(int type, const void *w, uint32_t token, float *out, uint32_t dim);

/* rms_norm (src/vbs_host_math.h:28-36; NORMALIZE, src/vbs_backend_hip.c:424-439). */
int vbs_gfx950_rms_norm(const float *in, const float *w, float *out, uint32_t dim, float eps);

/* In-place RoPE on n_heads x head_dim (src/vbs_host_math.h:38-51; ROTARY,
 * src/vbs_backend_hip.c:440-454). head_dim <= 512. */
int vbs_gfx950_rope(float *x, uint32_t pos, uint32_t head_dim, uint32_t n_heads, float theta);

/* f16 KV store at ((layer*max_ctx + pos)*kv_dim + i) with the reference
 * rounding (src/vbs_host_math.h:150-159; CACHE, src/vbs_backend_hip.c:455-481). */
int vbs_gfx950_cache_store(const float *k, const float *v, uint16_t *kc, uint16_t *vc,
                           uint32_t pos, uint32_t layer, uint32_t max_ctx, uint32_t kv_dim);

/* Single-query GQA attention over the f16 cache (src/vbs_host_math.h:170-209;
 * ATTENTION, src/vbs_backend_hip.c:482-512). */
int vbs_gfx950_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                         uint32_t seq_len, uint32_t layer, uint32_t max_ctx,
                         uint32_t n_q_heads, uint32_t n_kv_heads, uint32_t head_dim,
                         float scale);

/* vbs_gfx950_attention without any device allocation: no counterpart in the
 * reference. For callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same arguments and
 * result as vbs_gfx950_attention; the per-chunk partial results live in a
 * fixed 8 MiB device array of the library instead of the growable scratch, so
 * calls whose partials exceed it (nqh x max(ceil(640 / nkh), ceil(seq_len /
 * 64)) x (head_dim + 2) x 4 bytes, 640 being the workgroup target of the
 * sequence split, kMfmaTargetWgs in csrc/vbs_attn_common.h; e.g. 70B shapes
 * up to seq_len 16128) fail with a reason and launch nothing. Every call on the device shares that
 * array: calls that overlap on the device race (the library's own calls are
 * ordered on its one stream and never overlap). */
int vbs_gfx950_attention_noalloc(const float *q, const uint16_t *kc, const uint16_t *vc,
                                 float *out, uint32_t seq_len, uint32_t layer, uint32_t max_ctx,
                                 uint32_t n_q_heads, uint32_t n_kv_heads, uint32_t head_dim,
                                 float scale);

/* out = gate / (1 + expf(-gate)) * up (src/vbs_host_math.h:53-57; ACTIVATION). */
int vbs_gfx950_silu_mul(const float *gate, const float *up, float *out, uint32_t n);

/* out = a + b, out may alias a (src/vbs_host_math.h:59-62; ELEMENTWISE). */
int vbs_gfx950_add(const float *a, const float *b, float *out, uint32_t n);

/* ---- extensions (no slot in vbs_backend_ops_t) -------------------------- */

/* Dequantise rows of a packed tensor: out[i*dim .. +dim) = deq(row ids[i])
 * (ids == NULL means rows 0..n_rows-1). `ids` is a device array. The batched
 * form of the one-token-per-dispatch EMBEDDING op, and the bit-exactness
 * probe of every block decoder. */
int vbs_gfx950_dequant_rows(int type, const void *w, const uint32_t *ids, uint32_t n_rows,
                            uint32_t dim, float *out);

/* The neighbours of a linear matvec that vbs_gfx950_linear_fused takes into
 * the same launch; NULL / 0 fields are absent. */
typedef struct vbs_gfx950_linear_join {
    const float *norm_w;   /* NORMALIZE before: x_normed = rms_norm(x, norm_w, norm_eps) */
    float norm_eps;
    float *x_normed;
    float *acc;            /* ELEMENTWISE after: acc = acc + y */
    int rope;              /* ROTARY after: y rotated at pos in heads of head_dim, base theta */
    uint32_t pos, head_dim;
    float theta;
    const float *gate;     /* ACTIVATION after: hidden = silu(gate) * y */
    float *hidden;
    const float *k_row;    /* CACHE after: kc[kv_off + i] = f16(k_row[i]), vc[kv_off + i] = f16(y[i]) */
    uint16_t *kc, *vc;
    uint64_t kv_off;       /* (layer * max_ctx + pos) * kv_dim */
} vbs_gfx950_linear_join_t;

/* The linear matvec y = W x fused with its neighbours in the bridge's op
 * sequence, for the backend shim's per-dispatch path (no counterpart in the
 * reference: the shim holds back one op and joins it with the next when they
 * fit one of these kernels; results are bit-identical to the ops one by one,
 * and y is always written):
 *   - norm_w and x_normed: the NORMALIZE before it (src/vbs_host_math.h:28-36),
 *     x_normed stored as that op would, then y = W x_normed; alone or with rope;
 *   - acc: the ELEMENTWISE add after it (src/vbs_host_math.h:59-62);
 *   - rope: the ROTARY after it (src/vbs_host_math.h:38-51);
 *   - gate and hidden: the ACTIVATION after the up matvec
 *     (src/vbs_host_math.h:53-57);
 *   - k_row, kc, vc: the CACHE after the V matvec, with the reference's f16
 *     rounding (src/vbs_host_math.h:150-159).
 * At most one of acc / rope / gate / k_row. Q4_K and Q6_K rows of a multiple
 * of 256; returns 1 when launched, 0 with a reason on an error, and 2
 * (nothing launched) when no fused kernel takes this combination or shape.
 * The RoPE rows live in a device table the library builds for (theta,
 * head_dim) and regrows for later positions (it allocates; not for graph
 * capture). */
int vbs_gfx950_linear_fused(int type, const void *w, const float *x, float *y, uint32_t cols,
                            uint32_t rows, const vbs_gfx950_linear_join_t *join);

/* Grouped ops of the backend shim's per-dispatch path (no counterpart in the
 * reference: the shim holds back the bridge's attention-input and FFN-input
 * runs and issues each as one launch; results are bit-identical to the ops
 * one by one, and every buffer those ops write is written):
 *
 * vbs_gfx950_qkv_fused -- NORMALIZE (when norm_w and x_normed are given),
 * LINEAR q, ROTARY q, LINEAR k, ROTARY k, LINEAR v, CACHE
 * (src/vbs_specializer.c:282-302): x_normed = rms_norm(x), q = rope(Wq xn),
 * k = rope(Wk xn), v = Wv xn, and f16(k), f16(v) stored at
 * ((layer * max_ctx + pos) * kv_rows + i) of kc / vc, the rotations at pos
 * in heads of head_dim with base theta. The three matrices share the type. */
int vbs_gfx950_qkv_fused(int type, const void *wq, const void *wk, const void *wv, const float *x,
                         uint32_t cols, uint32_t q_rows, uint32_t kv_rows, const float *norm_w,
                         float eps, float *x_normed, float *q, float *k, float *v, uint32_t pos,
                         uint32_t head_dim, float theta, uint16_t *kc, uint16_t *vc,
                         uint32_t layer, uint32_t max_ctx);

/* vbs_gfx950_gate_up_fused -- NORMALIZE (optional, as above), LINEAR gate,
 * LINEAR up, ACTIVATION (src/vbs_specializer.c:282-284, 319-329): gate = Wg xn,
 * up = Wu xn, hidden = silu(gate) * up.
 *
 * Both: Q4_K and Q6_K rows of a multiple of 256, row counts of a multiple
 * of 16; 1 when launched, 0 with a reason on an error, 2 (nothing launched)
 * when no grouped kernel takes the shape. The RoPE rows come from the same
 * device table as vbs_gfx950_linear_fused's (it allocates; not for graph
 * capture). */
int vbs_gfx950_gate_up_fused(int type, const void *wg, const void *wu, const float *x,
                             uint32_t cols, uint32_t rows, const float *norm_w, float eps,
                             float *x_normed, float *gate, float *up, float *hidden);

/* Batched decode: Y[b*y_stride + r] = sum_c deq(W[r,c]) * X[b*x_stride + c]
 * for b < batch (<= 16). Equal to `batch` calls of vbs_gfx950_linear; the
 * weights are read once. The reference has no batched matvec
 * (src/vbs_specializer.c:353-357 loops tokens one by one). */
int vbs_gfx950_linear_batch(int type, const void *w, const float *x, uint32_t x_stride,
                            float *y, uint32_t y_stride, uint32_t cols, uint32_t rows,
                            uint32_t batch);

/* Up to three matrices of one type and column count over the same vectors
 * (Q, K and V, or gate and up): for m < n_mat, Y_m[b*y_stride[m] + r] =
 * sum_c deq(W_m[r,c]) * X[b*x_stride + c], b < batch (<= 16). Equal to n_mat
 * calls of vbs_gfx950_linear_batch; for Q4_K and Q6_K the vectors are
 * prepared once and every matrix shares one matrix-core launch, as the
 * batched decoder runs a layer's Q/K/V and gate/up. w, rows, y and y_stride
 * are host arrays of n_mat entries (w[m] and y[m] device pointers). No
 * counterpart in the reference (it has no batched matvec). */
int vbs_gfx950_linear_batch_multi(int type, uint32_t n_mat, const void *const *w,
                                  const uint32_t *rows, const float *x, uint32_t x_stride,
                                  float *const *y, const uint32_t *y_stride, uint32_t cols,
                                  uint32_t batch);

/* XOR checksum of a device region, as partial words, for
 * i < vbs_gfx950_checksum_partials(bytes): the region is cut into consecutive
 * spans of up to 112 KB, one per workgroup of 16 waves, and partials[16 w + v]
 * is the XOR of the 32-bit words of wave v's share of span w (its interleaved
 * 1 KB runs v, v + 16, v + 32, ... of the span). Their XOR is the region's. p is 16-byte aligned and bytes a multiple of 16; partials is
 * device memory.
 * Verifies uploads (the host XORs the same words) and, reading every byte
 * exactly once and nothing else, it is the read floor beside the matvec
 * roofline. No counterpart in the reference. */
uint32_t vbs_gfx950_checksum_partials(size_t bytes);
int vbs_gfx950_checksum(const void *p, size_t bytes, uint32_t *partials);
/* The same checksum read in another shape, to show how tight the read floor
 * is: variant 0 is vbs_gfx950_checksum; 1 reads 56 KB spans with two 8-wave
 * workgroups per CU (8 partials per workgroup); 2 is variant 0's shape with
 * 16-byte vector loads into registers instead of LDS DMA. The XOR of the
 * partials is the region's in every variant. No counterpart in the
 * reference. */
uint32_t vbs_gfx950_checksum_variant_partials(size_t bytes, int variant);
int vbs_gfx950_checksum_variant(const void *p, size_t bytes, uint32_t *partials, int variant);

/* The library's stream (a hipStream_t), for callers that time kernels with
 * HIP events or capture the stream into a graph.
 *
 * Capture and the library's scratch: vbs_gfx950_linear_batch (Q4_K / Q6_K)
 * and vbs_gfx950_attention keep intermediate results in a device scratch
 * that the library owns. It only grows, and a buffer that a larger call
 * replaces stays allocated until the process ends, so a captured graph keeps
 * valid memory whatever is called after the capture. Growing allocates, so a
 * call made while the stream is being captured fails (0, reason "operation
 * not permitted when stream is capturing") if it needs more scratch than
 * earlier uncaptured calls have sized: make one uncaptured call of the
 * largest shape before capturing. */
void *vbs_gfx950_stream(void);

/* ---- graph-replayed decode step (extension) -------------------------------
 * The caller side of one token (src/vbs_specializer.c:231-359) issues ~16
 * dispatches per layer through the ops table, each a separate host launch.
 * The decoder below runs the same sequence, with the same kernels and the
 * same arithmetic, from one HIP graph per model: the token and position live
 * in device memory (RoPE angles come from a table computed once with the host
 * libm, exactly as src/vbs_host_math.h:43-44), and a greedy argmax kernel
 * (first maximum, as main.c:929-932) writes the next token and advances the
 * position, so consecutive tokens replay the graph back to back. */
typedef struct {
    uint32_t n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, vocab, max_ctx;
    float rope_theta, rms_eps;
    int embd_type;
    const void *tok_embd;            /* device: vocab x hidden packed */
    const float *out_norm;           /* device: hidden */
    int head_type;
    const void *lm_head;             /* device: vocab x hidden packed */
    const float *const *attn_norm;   /* host array of n_layers device pointers */
    const float *const *ffn_norm;    /* host array of n_layers device pointers */
    const int *wtype;                /* host array n_layers x 7 (q,k,v,o,gate,up,down) */
    const void *const *wdata;        /* host array n_layers x 7 device pointers */
    uint16_t *kc, *vc;               /* device f16 caches [n_layers][max_ctx][n_kv_heads*head_dim] */
} vbs_gfx950_model_t;

/* Build the per-token graph (the model's device memory is borrowed, not
 * copied). max_steps bounds one vbs_gfx950_decoder_greedy call. */
int vbs_gfx950_decoder_create(const vbs_gfx950_model_t *m, uint32_t max_steps, void **handle);
/* One token at `pos`; logits (vocab floats, host) may be NULL. */
int vbs_gfx950_decoder_step(void *handle, uint32_t token, uint32_t pos, float *logits);
/* Greedy: feed `token` at `pos`, then n-1 further argmax tokens; tokens[i]
 * is the i-th argmax, margins (may be NULL) top-1 minus top-2 logit. */
int vbs_gfx950_decoder_greedy(void *handle, uint32_t token, uint32_t pos, uint32_t n,
                              uint32_t *tokens, float *margins);
/* The same steps as vbs_gfx950_decoder_greedy, each kernel launched directly
 * instead of replaying the graph (identical results; for tools that trace
 * kernel launches but not graph replays). */
int vbs_gfx950_decoder_greedy_eager(void *handle, uint32_t token, uint32_t pos, uint32_t n,
                                    uint32_t *tokens, float *margins);
/* No counterpart in the reference (a diagnostic of this decoder). Where every
 * layer's O is Q4_K over a 4096-wide q of 128-dim heads, the decoder merges
 * the attention partials inside the O launch: each workgroup merges one head
 * and the workgroups on one XCD share the heads through its L2; a workgroup
 * whose bounded wait for them runs out (one placed or started unexpectedly)
 * merges every head itself, with identical results. Returns 1 when the
 * decoder takes that path, with *count (may be NULL) the workgroups that
 * merged every head themselves since it was created, 0 when it does not, -1
 * on error. The environment variable VBS_ATTN_O_SPIN, read at create, sets
 * the wait's bound in polls (0: no workgroup waits). */
int vbs_gfx950_decoder_attn_o_fallbacks(void *handle, uint32_t *count);
int vbs_gfx950_decoder_destroy(void *handle);

/* ---- batched decode (extension) --------------------------------------------
 * The decode step above for `batch` (1..8) independent sequences over one copy
 * of the weights (the Llama-70B case at batch 8): each sequence has its own
 * caches, m->kc / m->vc + b * kv_seq_stride elements (the model's layout per
 * sequence), its own token and position. Every matrix must be Q4_K or Q6_K
 * (the batched matrix-core kernels; q/k/v and gate/up pairwise of one type).
 * The reference has no batched decode (src/vbs_specializer.c:353-357 loops
 * tokens one by one); each sequence computes the single-sequence step. */
int vbs_gfx950_bdecoder_create(const vbs_gfx950_model_t *m, uint32_t batch, uint64_t kv_seq_stride,
                               uint32_t max_steps, void **handle);
/* Greedy for every sequence: feed tokens0[b] at pos0[b], then n-1 further
 * argmax tokens; tokens[i * batch + b] is sequence b's i-th argmax, margins
 * (may be NULL) its top-1 minus top-2 logit. */
int vbs_gfx950_bdecoder_greedy(void *handle, const uint32_t *tokens0, const uint32_t *pos0,
                               uint32_t n, uint32_t *tokens, float *margins);
/* The same with every kernel launched directly (for kernel tracers). */
int vbs_gfx950_bdecoder_greedy_eager(void *handle, const uint32_t *tokens0, const uint32_t *pos0,
                                     uint32_t n, uint32_t *tokens, float *margins);
/* One step of every sequence with the given tokens[b] at pos[b] (teacher
 * forcing: the graph of vbs_gfx950_bdecoder_greedy, replayed once); the caches
 * at pos[b] are written as by a greedy step, and logits (batch x vocab floats,
 * host, sequence b at b * vocab) may be NULL. */
int vbs_gfx950_bdecoder_step(void *handle, const uint32_t *tokens, const uint32_t *pos,
                             float *logits);
int vbs_gfx950_bdecoder_destroy(void *handle);

/* ---- CPU hot-kernel table on the device (parity adapter) --------------------
 * The arithmetic of the reference's CPU hot-kernel ABI v1
 * (include/vbs_hotpath.h:38-57, src/hotkernels/vbs_hot_ref_impl.h:49-129) on
 * device buffers, bit-identical to its built-in table; the host-pointer
 * module over these is lib/libvbs_hot_gfx950.so (host/vbs_hot_gfx950.c). */

/* Q8 activations of x as the CPU model forms them (src/vbs_cpu.c:166-182):
 * per 32-element block d = amax/127, xq = round(x/d) clamped to +-127,
 * qd = f16(d), qsum = f16(sum(xq)*d) (round to nearest even). cols must be a
 * multiple of 32; x is assumed finite (the CPU model screens non-finite
 * inputs first, src/vbs_cpu.c:185-190). All buffers 4-byte aligned. */
int vbs_gfx950_quantize_q8(const float *x, uint32_t cols, int8_t *xq, float *qd, float *qsum);

/* y[r] = the hot table's matvec of row r (replaces matvec_q8_0 / q4_0 / q4_1 /
 * f32 / f16 of vbs_hot_kernels_t). type Q8_0, Q4_0, Q4_1: act = xq (int8),
 * qd and (Q4_1) qsum as vbs_gfx950_quantize_q8 makes them, cols a multiple
 * of 32; type F32, F16: act = x (f32). w packed row-major. */
int vbs_gfx950_hot_matvec(int type, const void *w, uint32_t rows, uint32_t cols, const void *act,
                          const float *qd, const float *qsum, float *y);

#ifdef __cplusplus
}
#endif
#endif
