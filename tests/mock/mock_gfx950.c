/* mock_gfx950.c -- TEST-ONLY stand-in for libvbs_gfx950.so.
 *
 * Implements the device library's C ABI (include/vbs_gfx950.h) on host memory
 * with the CPU oracle, so the C11 backend shim and its calling conventions can
 * be exercised without a GPU. It is built by tests/test_backend_contract.py
 * into a temporary directory and loaded only through VBS_GFX950_LIB; the
 * product never loads it. MOCK_ABI / MOCK_DROP let a test build variants with
 * a wrong ABI version or a missing entry point.
 */
#include <stdlib.h>
#include <string.h>
#include "vbs_gfx950.h"
#include "vbs_oracle.h"

#ifndef MOCK_ABI
#define MOCK_ABI VBS_GFX950_ABI_VERSION
#endif

int vbs_gfx950_abi_version(void) { return MOCK_ABI; }
int vbs_gfx950_init(void) { return 1; }
const char *vbs_gfx950_last_error(void) { return "ok"; }
int vbs_gfx950_device_count(void) { return 1; }
int vbs_gfx950_device_info(int i, char *name, size_t cap, uint64_t *t, uint64_t *f) {
    if (i) return 0;
    if (name && cap) { strncpy(name, "host mock of gfx950", cap - 1); name[cap - 1] = 0; }
    if (t) *t = 1ull << 30;
    if (f) *f = 1ull << 30;
    return 1;
}
void *vbs_gfx950_alloc(size_t n) { return calloc(1, n ? n : 1); }
int vbs_gfx950_free(void *p) { free(p); return 1; }
void *vbs_gfx950_host_alloc(size_t n) { return calloc(1, n ? n : 1); }
int vbs_gfx950_host_free(void *p) { free(p); return 1; }
int vbs_gfx950_copy_h2d(void *d, const void *s, size_t n) { memmove(d, s, n); return 1; }
int vbs_gfx950_copy_d2h(void *d, const void *s, size_t n) { memmove(d, s, n); return 1; }
int vbs_gfx950_copy_d2d(void *d, const void *s, size_t n) { memmove(d, s, n); return 1; }
int vbs_gfx950_synchronize(void) { return 1; }
void *vbs_gfx950_stream(void) { return NULL; }
int vbs_gfx950_linear_supported(int t) { return vbs_oracle_geometry(t, NULL, NULL); }
int vbs_gfx950_linear(int t, const void *w, const float *x, float *y, uint32_t cols, uint32_t rows,
                      uint32_t co, uint32_t ro, int acc) {
    return vbs_oracle_linear_tile(t, (const uint8_t *)w, x, y, cols, rows, co, ro, acc);
}
int vbs_gfx950_linear_batch(int t, const void *w, const float *x, uint32_t xs, float *y,
                            uint32_t ys, uint32_t cols, uint32_t rows, uint32_t batch) {
    for (uint32_t b = 0; b < batch; b++)
        if (!vbs_oracle_linear_tile(t, (const uint8_t *)w, x + (size_t)b * xs, y + (size_t)b * ys,
                                    cols, rows, 0, 0, 0)) return 0;
    return 1;
}
int vbs_gfx950_embed(int t, const void *w, uint32_t tok, float *out, uint32_t dim) {
    return vbs_oracle_embed_row(t, (const uint8_t *)w, tok, out, dim);
}
int vbs_gfx950_dequant_rows(int t, const void *w, const uint32_t *ids, uint32_t n, uint32_t dim,
                            float *out) {
    for (uint32_t r = 0; r < n; r++)
        if (!vbs_oracle_embed_row(t, (const uint8_t *)w, ids ? ids[r] : r, out + (size_t)r * dim, dim))
            return 0;
    return 1;
}
int vbs_gfx950_rms_norm(const float *in, const float *w, float *out, uint32_t n, float eps) {
    vbs_oracle_rms_norm(in, w, out, n, eps); return 1;
}
int vbs_gfx950_rope(float *x, uint32_t pos, uint32_t hd, uint32_t nh, float theta) {
    vbs_oracle_rope(x, pos, hd, nh, theta); return 1;
}
int vbs_gfx950_cache_store(const float *k, const float *v, uint16_t *kc, uint16_t *vc, uint32_t pos,
                           uint32_t layer, uint32_t mc, uint32_t kvd) {
    vbs_oracle_cache_store(k, v, kc, vc, pos, layer, mc, kvd); return 1;
}
int vbs_gfx950_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                         uint32_t sl, uint32_t layer, uint32_t mc, uint32_t nq, uint32_t nk,
                         uint32_t hd, float scale) {
    vbs_oracle_attention(q, kc, vc, out, sl, layer, mc, nq, nk, hd, scale); return 1;
}
int vbs_gfx950_silu_mul(const float *g, const float *u, float *out, uint32_t n) {
    vbs_oracle_silu_mul(g, u, out, n); return 1;
}
#ifndef MOCK_DROP_ADD
int vbs_gfx950_add(const float *a, const float *b, float *out, uint32_t n) {
    vbs_oracle_add(a, b, out, n); return 1;
}
#endif
/* The fused neighbours of a linear (vbs_gfx950_linear_fused) as the ops one
 * by one; like the device library, only for Q4_K and Q6_K and for the same
 * combinations (else 2: nothing done, the shim issues the ops itself). */
static unsigned g_fused[7]; /* launches joined with a NORMALIZE, ROTARY, add, ACTIVATION, CACHE;
                               grouped q/k/v and gate/up launches */
unsigned mock_fused_count(int which) { return which >= 0 && which < 7 ? g_fused[which] : 0u; }

int vbs_gfx950_linear_fused(int t, const void *w, const float *x, float *y, uint32_t cols,
                            uint32_t rows, const vbs_gfx950_linear_join_t *j) {
    if (!j) return 0;
    if ((j->norm_w != NULL) != (j->x_normed != NULL) || (j->gate != NULL) != (j->hidden != NULL) ||
        (j->k_row != NULL) != (j->kc != NULL) || (j->k_row != NULL) != (j->vc != NULL))
        return 0;
    if (t != 12 && t != 14) return 2;
    const int after = (j->acc != NULL) + (j->rope != 0) + (j->gate != NULL) + (j->k_row != NULL);
    if (after > 1 || (!after && !j->norm_w) || (j->norm_w && after && !j->rope)) return 2;
    if (j->norm_w) {
        vbs_oracle_rms_norm(x, j->norm_w, j->x_normed, cols, j->norm_eps);
        x = j->x_normed;
    }
    if (!vbs_oracle_linear_tile(t, (const uint8_t *)w, x, y, cols, rows, 0, 0, 0)) return 0;
    if (j->rope) vbs_oracle_rope(y, j->pos, j->head_dim, rows / j->head_dim, j->theta);
    if (j->acc) vbs_oracle_add(j->acc, y, j->acc, rows);
    if (j->gate) vbs_oracle_silu_mul(j->gate, y, j->hidden, rows);
    if (j->k_row) vbs_oracle_cache_store(j->k_row, y, j->kc + j->kv_off, j->vc + j->kv_off, 0, 0, 1, rows);
    g_fused[0] += j->norm_w != NULL;
    g_fused[1] += j->rope != 0;
    g_fused[2] += j->acc != NULL;
    g_fused[3] += j->gate != NULL;
    g_fused[4] += j->k_row != NULL;
    return 1;
}

/* The grouped q/k/v and gate/up launches as the ops one by one (built with
 * MOCK_DECLINE_GROUPS they decline every shape, so the shim's fallbacks run). */
int vbs_gfx950_qkv_fused(int t, const void *wq, const void *wk, const void *wv, const float *x,
                         uint32_t cols, uint32_t q_rows, uint32_t kv_rows, const float *norm_w,
                         float eps, float *x_normed, float *q, float *k, float *v, uint32_t pos,
                         uint32_t hd, float theta, uint16_t *kc, uint16_t *vc, uint32_t layer,
                         uint32_t max_ctx) {
    if ((norm_w != NULL) != (x_normed != NULL) || pos >= max_ctx) return 0;
#ifdef MOCK_DECLINE_GROUPS
    return 2;
#endif
    if (t != 12 && t != 14) return 2;
    if (norm_w) {
        vbs_oracle_rms_norm(x, norm_w, x_normed, cols, eps);
        x = x_normed;
    }
    if (!vbs_oracle_linear_tile(t, (const uint8_t *)wq, x, q, cols, q_rows, 0, 0, 0) ||
        !vbs_oracle_linear_tile(t, (const uint8_t *)wk, x, k, cols, kv_rows, 0, 0, 0) ||
        !vbs_oracle_linear_tile(t, (const uint8_t *)wv, x, v, cols, kv_rows, 0, 0, 0))
        return 0;
    vbs_oracle_rope(q, pos, hd, q_rows / hd, theta);
    vbs_oracle_rope(k, pos, hd, kv_rows / hd, theta);
    vbs_oracle_cache_store(k, v, kc, vc, pos, layer, max_ctx, kv_rows);
    g_fused[5]++;
    return 1;
}

int vbs_gfx950_gate_up_fused(int t, const void *wg, const void *wu, const float *x, uint32_t cols,
                             uint32_t rows, const float *norm_w, float eps, float *x_normed,
                             float *gate, float *up, float *hidden) {
    if ((norm_w != NULL) != (x_normed != NULL)) return 0;
#ifdef MOCK_DECLINE_GROUPS
    return 2;
#endif
    if (t != 12 && t != 14) return 2;
    if (norm_w) {
        vbs_oracle_rms_norm(x, norm_w, x_normed, cols, eps);
        x = x_normed;
    }
    if (!vbs_oracle_linear_tile(t, (const uint8_t *)wg, x, gate, cols, rows, 0, 0, 0) ||
        !vbs_oracle_linear_tile(t, (const uint8_t *)wu, x, up, cols, rows, 0, 0, 0))
        return 0;
    vbs_oracle_silu_mul(gate, up, hidden, rows);
    g_fused[6]++;
    return 1;
}
