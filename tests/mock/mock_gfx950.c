/* mock_gfx950.c -- TEST-ONLY stand-in for libvbs_gfx950.so.
 *
 * Implements the device library's C ABI (include/vbs_gfx950.h) on host memory
 * with the CPU oracle, so the C11 backend shim and its calling conventions can
 * be exercised without a GPU. It is built by tests/test_backend_contract.py
 * into a temporary directory and loaded only through VBS_GFX950_LIB; the
 * product never loads it. MOCK_ABI / MOCK_DROP let a test build variants with
 * a wrong ABI version or a missing entry point.
 */
#include <math.h>
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
/* The fused neighbours of a linear (vbs_gfx950_linear_fused) and the grouped
 * q/k/v and gate/up launches, composed of the oracle's ops; like the device
 * library, only for Q4_K and Q6_K and for the same combinations (else 2:
 * nothing done, the shim issues the ops itself). A GPU launch's workgroups
 * read and write in no fixed order, so these entries take the orders that
 * expose aliasing: the per-row inputs (acc, gate, k_row: read by the thread
 * that writes the row) are read first, then every output is overwritten
 * with NaN (0xFFFF in the caches), then the inputs every workgroup reads
 * (x, the norm weights) are read and the results computed into private
 * copies, and the outputs are written in the reverse of the ops' order.
 * Whenever an output aliases an input or another output of the launch, the
 * result then differs from the ops one by one, which is what the shim's
 * aliasing checks must prevent. Built with
 * MOCK_DECLINE_GROUPS the grouped entries decline every shape, with
 * MOCK_DECLINE_FUSED every entry here does (the shim's fallbacks run). */
static unsigned g_fused[7]; /* launches joined with a NORMALIZE, ROTARY, add, ACTIVATION, CACHE;
                               grouped q/k/v and gate/up launches */
unsigned mock_fused_count(int which) { return which >= 0 && which < 7 ? g_fused[which] : 0u; }

static float *fcopy(const float *src, uint32_t n) {
    float *d = (float *)malloc(sizeof(float) * (n ? n : 1u));
    if (d && src) memcpy(d, src, sizeof(float) * n);
    return d;
}

static void poison(float *p, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) p[i] = NAN;
}

static void poison16(uint16_t *p, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) p[i] = 0xFFFFu;
}

/* xn = rms_norm(x) when norm_w is given (into a fresh copy; x otherwise) */
static float *normed_copy(const float *x, const float *norm_w, uint32_t cols, float eps) {
    float *xn = fcopy(x, cols);
    if (xn && norm_w) vbs_oracle_rms_norm(x, norm_w, xn, cols, eps);
    return xn;
}

int vbs_gfx950_linear_fused(int t, const void *w, const float *x, float *y, uint32_t cols,
                            uint32_t rows, const vbs_gfx950_linear_join_t *j) {
    if (!j) return 0;
    if ((j->norm_w != NULL) != (j->x_normed != NULL) || (j->gate != NULL) != (j->hidden != NULL) ||
        (j->k_row != NULL) != (j->kc != NULL) || (j->k_row != NULL) != (j->vc != NULL))
        return 0;
#ifdef MOCK_DECLINE_FUSED
    return 2;
#endif
    if (t != 12 && t != 14) return 2;
    const int after = (j->acc != NULL) + (j->rope != 0) + (j->gate != NULL) + (j->k_row != NULL);
    if (after > 1 || (!after && !j->norm_w) || (j->norm_w && after && !j->rope)) return 2;
    /* per-row reads, then the outputs clobbered, then the shared reads */
    float *acc = j->acc ? fcopy(j->acc, rows) : NULL, *gate = j->gate ? fcopy(j->gate, rows) : NULL;
    float *krow = j->k_row ? fcopy(j->k_row, rows) : NULL;
    if (j->x_normed) poison(j->x_normed, cols);
    poison(y, rows);
    if (j->acc) poison(j->acc, rows);
    if (j->hidden) poison(j->hidden, rows);
    if (j->k_row) {
        poison16(j->kc + j->kv_off, rows);
        poison16(j->vc + j->kv_off, rows);
    }
    float *xn = normed_copy(x, j->norm_w, cols, j->norm_eps), *yt = fcopy(NULL, rows);
    float *hid = j->gate ? fcopy(NULL, rows) : NULL;
    uint16_t *kr = j->k_row ? (uint16_t *)malloc(2u * rows) : NULL;
    uint16_t *vr = j->k_row ? (uint16_t *)malloc(2u * rows) : NULL;
    int ok = xn && yt && vbs_oracle_linear_tile(t, (const uint8_t *)w, xn, yt, cols, rows, 0, 0, 0);
    if (ok && j->rope) vbs_oracle_rope(yt, j->pos, j->head_dim, rows / j->head_dim, j->theta);
    if (ok && acc) vbs_oracle_add(acc, yt, acc, rows);
    if (ok && hid) vbs_oracle_silu_mul(gate, yt, hid, rows);
    if (ok && kr && vr) vbs_oracle_cache_store(krow, yt, kr, vr, 0, 0, 1, rows);
    /* writes, last op first */
    if (ok) {
        if (kr && vr) {
            memcpy(j->vc + j->kv_off, vr, 2u * rows);
            memcpy(j->kc + j->kv_off, kr, 2u * rows);
        }
        if (hid) memcpy(j->hidden, hid, 4u * rows);
        if (acc) memcpy(j->acc, acc, 4u * rows);
        memcpy(y, yt, 4u * rows);
        if (j->norm_w) memcpy(j->x_normed, xn, 4u * cols);
        g_fused[0] += j->norm_w != NULL;
        g_fused[1] += j->rope != 0;
        g_fused[2] += j->acc != NULL;
        g_fused[3] += j->gate != NULL;
        g_fused[4] += j->k_row != NULL;
    }
    free(xn); free(yt); free(acc); free(gate); free(krow); free(hid); free(kr); free(vr);
    return ok ? 1 : 0;
}

int vbs_gfx950_qkv_fused(int t, const void *wq, const void *wk, const void *wv, const float *x,
                         uint32_t cols, uint32_t q_rows, uint32_t kv_rows, const float *norm_w,
                         float eps, float *x_normed, float *q, float *k, float *v, uint32_t pos,
                         uint32_t hd, float theta, uint16_t *kc, uint16_t *vc, uint32_t layer,
                         uint32_t max_ctx) {
    if ((norm_w != NULL) != (x_normed != NULL) || pos >= max_ctx) return 0;
#if defined(MOCK_DECLINE_GROUPS) || defined(MOCK_DECLINE_FUSED)
    return 2;
#endif
    if (t != 12 && t != 14) return 2;
    const uint64_t off = ((uint64_t)layer * max_ctx + pos) * kv_rows;
    if (x_normed) poison(x_normed, cols);
    poison(q, q_rows);
    poison(k, kv_rows);
    poison(v, kv_rows);
    poison16(kc + off, kv_rows);
    poison16(vc + off, kv_rows);
    float *xn = normed_copy(x, norm_w, cols, eps), *qt = fcopy(NULL, q_rows);
    float *kt = fcopy(NULL, kv_rows), *vt = fcopy(NULL, kv_rows);
    uint16_t *kr = (uint16_t *)malloc(2u * kv_rows), *vr = (uint16_t *)malloc(2u * kv_rows);
    int ok = xn && qt && kt && vt && kr && vr &&
             vbs_oracle_linear_tile(t, (const uint8_t *)wq, xn, qt, cols, q_rows, 0, 0, 0) &&
             vbs_oracle_linear_tile(t, (const uint8_t *)wk, xn, kt, cols, kv_rows, 0, 0, 0) &&
             vbs_oracle_linear_tile(t, (const uint8_t *)wv, xn, vt, cols, kv_rows, 0, 0, 0);
    if (ok) {
        vbs_oracle_rope(qt, pos, hd, q_rows / hd, theta);
        vbs_oracle_rope(kt, pos, hd, kv_rows / hd, theta);
        vbs_oracle_cache_store(kt, vt, kr, vr, 0, 0, 1, kv_rows);
        memcpy(vc + off, vr, 2u * kv_rows);
        memcpy(kc + off, kr, 2u * kv_rows);
        memcpy(v, vt, 4u * kv_rows);
        memcpy(k, kt, 4u * kv_rows);
        memcpy(q, qt, 4u * q_rows);
        if (norm_w) memcpy(x_normed, xn, 4u * cols);
        g_fused[5]++;
    }
    free(xn); free(qt); free(kt); free(vt); free(kr); free(vr);
    return ok ? 1 : 0;
}

int vbs_gfx950_gate_up_fused(int t, const void *wg, const void *wu, const float *x, uint32_t cols,
                             uint32_t rows, const float *norm_w, float eps, float *x_normed,
                             float *gate, float *up, float *hidden) {
    if ((norm_w != NULL) != (x_normed != NULL)) return 0;
#if defined(MOCK_DECLINE_GROUPS) || defined(MOCK_DECLINE_FUSED)
    return 2;
#endif
    if (t != 12 && t != 14) return 2;
    if (x_normed) poison(x_normed, cols);
    poison(gate, rows);
    poison(up, rows);
    poison(hidden, rows);
    float *xn = normed_copy(x, norm_w, cols, eps), *gt = fcopy(NULL, rows);
    float *ut = fcopy(NULL, rows), *ht = fcopy(NULL, rows);
    int ok = xn && gt && ut && ht &&
             vbs_oracle_linear_tile(t, (const uint8_t *)wg, xn, gt, cols, rows, 0, 0, 0) &&
             vbs_oracle_linear_tile(t, (const uint8_t *)wu, xn, ut, cols, rows, 0, 0, 0);
    if (ok) {
        vbs_oracle_silu_mul(gt, ut, ht, rows);
        memcpy(hidden, ht, 4u * rows);
        memcpy(up, ut, 4u * rows);
        memcpy(gate, gt, 4u * rows);
        if (norm_w) memcpy(x_normed, xn, 4u * cols);
        g_fused[6]++;
    }
    free(xn); free(gt); free(ut); free(ht);
    return ok ? 1 : 0;
}
