/* vbs_oracle.h — CPU oracle for the quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a clean-room restatement of the
 * reference CPU semantics (src/vbs_dequant.c, src/vbs_host_math.h,
 * src/vbs_gguf.c) used as the parity checker for the gfx950 kernels.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it; the product library never links or calls it.
 *
 * Numeric contract: identical expression order to the reference, no FMA
 * contraction (built with -ffp-contract=off), double accumulation where
 * the reference accumulates in double. Every function names the reference
 * lines it follows. Pinning of each function (golden vectors generated
 * from the reference C, closed forms, exhaustive checks) is done by the
 * tests in tests/test_oracle*.py.
 */
#ifndef VBS_ORACLE_H
#define VBS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- half precision (src/vbs_dequant.c:21-74) ---- */
float vbs_oracle_f16_to_f32(uint16_t h);
uint16_t vbs_oracle_f32_to_f16(float f);
/* 64-bit digest of fn(x) over all 2^32 float bit patterns (multi-threaded).
 * Lets a test compare any f32->f16 converter against a stored digest. */
uint64_t vbs_oracle_digest_f32_to_f16(uint16_t (*fn)(float), int nthreads);

/* ---- block geometry (src/vbs_gguf.c:12-40) ---- */
int vbs_oracle_geometry(int type, uint32_t *elems_per_block, uint32_t *bytes_per_block);
uint64_t vbs_oracle_row_bytes(int type, uint32_t cols);

/* ---- dequantisation (src/vbs_dequant.c:123-356, src/vbs_host_math.h:94-129) ---- */
/* One block of `type` -> 32 or 256 floats. Returns elements written, 0 if
 * the type is not on the hot path (Q4_0, Q4_1, Q8_0, Q4_K, Q6_K). */
int vbs_oracle_dequant_block(int type, const uint8_t *blk, float *out);
/* One packed row of `cols` elements (also F32/F16). Returns 1 on success. */
int vbs_oracle_dequant_row(int type, const uint8_t *row, uint32_t cols, float *out);

/* ---- linear tile (src/vbs_host_math.h:223-267) ---- */
int vbs_oracle_linear_tile(int type, const uint8_t *w, const float *x, float *y,
                           uint32_t cols, uint32_t rows, uint32_t col_off,
                           uint32_t row_off, int accumulate);
/* Same result, rows split over threads (rows are independent, so the output
 * is bit-identical to the single-threaded call). */
int vbs_oracle_linear_tile_mt(int type, const uint8_t *w, const float *x, float *y,
                              uint32_t cols, uint32_t rows, uint32_t col_off,
                              uint32_t row_off, int accumulate, int nthreads);

/* ---- primitives (src/vbs_host_math.h:28-62, 136-209) ---- */
int vbs_oracle_embed_row(int type, const uint8_t *table, uint32_t token, float *out, uint32_t dim);
void vbs_oracle_rms_norm(const float *in, const float *w, float *out, uint32_t n, float eps);
void vbs_oracle_rope(float *x, uint32_t pos, uint32_t head_dim, uint32_t n_heads, float theta);
void vbs_oracle_silu_mul(const float *gate, const float *up, float *out, uint32_t n);
void vbs_oracle_add(const float *a, const float *b, float *out, uint32_t n);
void vbs_oracle_cache_store(const float *k, const float *v, uint16_t *kc, uint16_t *vc,
                            uint32_t pos, uint32_t layer, uint32_t max_ctx, uint32_t kv_dim);
void vbs_oracle_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                          uint32_t seq_len, uint32_t layer, uint32_t max_ctx, uint32_t n_q_heads,
                          uint32_t n_kv_heads, uint32_t head_dim, float scale);
/* The same, its q heads split over up to nthreads threads (identical results). */
void vbs_oracle_attention_mt(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                             uint32_t seq_len, uint32_t layer, uint32_t max_ctx, uint32_t nqh,
                             uint32_t nkh, uint32_t hd, float scale, int nthreads);

/* ---- one decode step in the specializer's order ----
 * src/vbs_specializer.c:270-349 (sequence) with the bridge's scalar
 * arguments (src/vbs_specializer_bridge.c:148-183): embed -> per layer
 * [attn_norm, Q, rope(Q), K, rope(K), V, cache, attention(seq=pos+1), O,
 * add, ffn_norm, gate, up, silu, down, add] -> output_norm -> lm_head.
 * The model is described by flat arrays so the caller (ctypes) can build it
 * without sharing a struct layout with product code. */
typedef struct {
    uint32_t n_layers, hidden, ffn, n_heads, n_kv_heads, head_dim, vocab, max_ctx;
    float rope_theta, rms_eps;
    int embd_type;
    const uint8_t *tok_embd;   /* vocab x hidden packed */
    const float *out_norm;     /* hidden */
    int head_type;
    const uint8_t *lm_head;    /* vocab x hidden packed */
    /* per layer, arrays of n_layers entries */
    const float *const *attn_norm;
    const float *const *ffn_norm;
    const int *wtype;               /* n_layers x 7 (q,k,v,o,gate,up,down) */
    const uint8_t *const *wdata;    /* n_layers x 7 */
    uint16_t *kc, *vc;              /* [layer][max_ctx][n_kv_heads*head_dim] */
} vbs_oracle_model_t;

int vbs_oracle_forward_token(const vbs_oracle_model_t *m, uint32_t token, uint32_t pos,
                             float *logits, int nthreads);

/* ---- CPU hot-kernel table, ABI v1 (include/vbs_hotpath.h:38-57) ----
 * The Q8-activation matvecs of src/hotkernels/vbs_hot_ref_impl.h:49-129 and
 * the CPU model's activation quantiser (src/vbs_cpu.c:166-182) with its
 * round-to-nearest-even f16 conversion (src/vbs_cpu.c:74-93). */
uint16_t vbs_oracle_f32_to_f16_rne(float f);
void vbs_oracle_quantize_q8(const float *x, uint32_t cols, int8_t *xq, float *qd, float *qsum);
/* type 8 (Q8_0), 2 (Q4_0), 3 (Q4_1): xq/qd (+ qsum for Q4_1) are the
 * activations; type 0 (F32), 1 (F16): x is. Returns 0 for other types. */
int vbs_oracle_hot_matvec(int type, const void *w, uint32_t rows, uint32_t cols,
                          const int8_t *xq, const float *qd, const float *qsum, const float *x,
                          float *y);

#ifdef __cplusplus
}
#endif
#endif
