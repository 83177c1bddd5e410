/* vbs_oracle.c — CPU oracle for the quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker; never linked into the product).
 * A clean-room restatement of the reference's CPU semantics. Each function
 * cites the reference lines whose arithmetic it reproduces; expression order
 * is kept because the dequantised values must be bit-identical. Build with
 * -ffp-contract=off so no multiply-add pair is fused (the reference's x86-64
 * build has no FMA).
 */
#include "vbs_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

enum {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14,
    T_LNS8 = 40
};

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ------------------------------------------------------------------ */
/* half precision                                                      */
/* ------------------------------------------------------------------ */

/* src/vbs_dequant.c:21-44. Zero, normal and inf/nan are bit assembly;
 * a subnormal half is man * 2^-24, which is exactly representable as a
 * normal float, so it is computed arithmetically here. */
float vbs_oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u, man = h & 1023u;
    if (e == 31u) return u2f(sign | 0x7F800000u | (man << 13));
    if (e != 0u) return u2f(sign | ((e + 112u) << 23) | (man << 13));
    float mag = (float)man * 5.9604644775390625e-08f; /* 2^-24, exact */
    return u2f(sign | f2u(mag));
}

/* src/vbs_dequant.c:46-74. Normal results round to nearest even; results
 * below the smallest normal are formed from the 24-bit significand with
 * round-half-UP; values under 2^-25 flush to signed zero; overflow gives
 * inf; NaN keeps only a "payload nonzero" bit (0x7C01). */
uint16_t vbs_oracle_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    int be = (int)((u >> 23) & 255u);
    uint32_t frac = u & 0x7FFFFFu;
    if (be == 255) return (uint16_t)(sign | 0x7C00u | (frac != 0u));
    int he = be - 112; /* half biased exponent */
    if (he >= 31) return (uint16_t)(sign | 0x7C00u);
    if (he <= 0) {
        if (he < -10) return sign;
        unsigned sh = (unsigned)(14 - he);                 /* 14..24 */
        uint32_t sig = frac | 0x800000u;
        uint32_t q = (sig + (1u << (sh - 1u))) >> sh;      /* half up */
        return (uint16_t)(sign | (q >= 1024u ? 1024u : q));
    }
    uint32_t lsb = (frac >> 13) & 1u;
    uint32_t r = frac + 4095u + lsb;                       /* nearest even */
    if (r >> 23) { r = 0; he++; }
    if (he >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)he << 10) | (r >> 13));
}

typedef struct {
    uint16_t (*fn)(float);
    uint32_t first_range, n_ranges;
    uint64_t *out;
} digest_job_t;

#define DIGEST_RANGES 256u
static void *digest_worker(void *arg) {
    digest_job_t *j = (digest_job_t *)arg;
    for (uint32_t r = j->first_range; r < j->first_range + j->n_ranges; r++) {
        uint64_t h = 1469598103934665603ull; /* FNV-1a 64 */
        uint64_t base = (uint64_t)r << 24;
        for (uint64_t i = 0; i < (1ull << 24); i++) {
            uint16_t v = j->fn(u2f((uint32_t)(base + i)));
            h = (h ^ (v & 255u)) * 1099511628211ull;
            h = (h ^ (v >> 8)) * 1099511628211ull;
        }
        j->out[r] = h;
    }
    return NULL;
}

uint64_t vbs_oracle_digest_f32_to_f16(uint16_t (*fn)(float), int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    uint64_t parts[DIGEST_RANGES];
    pthread_t th[64];
    digest_job_t jobs[64];
    uint32_t per = (DIGEST_RANGES + (uint32_t)nthreads - 1u) / (uint32_t)nthreads;
    int launched = 0;
    for (int t = 0; t < nthreads; t++) {
        uint32_t first = (uint32_t)t * per;
        if (first >= DIGEST_RANGES) break;
        uint32_t n = first + per > DIGEST_RANGES ? DIGEST_RANGES - first : per;
        jobs[t] = (digest_job_t){fn, first, n, parts};
        pthread_create(&th[t], NULL, digest_worker, &jobs[t]);
        launched++;
    }
    for (int t = 0; t < launched; t++) pthread_join(th[t], NULL);
    uint64_t h = 1469598103934665603ull;
    for (uint32_t r = 0; r < DIGEST_RANGES; r++)
        for (int b = 0; b < 8; b++) h = (h ^ ((parts[r] >> (8 * b)) & 255u)) * 1099511628211ull;
    return h;
}

/* ------------------------------------------------------------------ */
/* geometry                                                            */
/* ------------------------------------------------------------------ */

/* src/vbs_gguf.c:12-40, restricted to the hot-path types. */
int vbs_oracle_geometry(int type, uint32_t *epb, uint32_t *bpb) {
    uint32_t e, b;
    switch (type) {
        case T_F32: e = 1; b = 4; break;
        case T_F16: e = 1; b = 2; break;
        case T_Q4_0: e = 32; b = 18; break;
        case T_Q4_1: e = 32; b = 20; break;
        case T_Q8_0: e = 32; b = 34; break;
        case T_Q4_K: e = 256; b = 144; break;
        case T_Q6_K: e = 256; b = 210; break;
        case T_LNS8: e = 32; b = 36; break;
        default: return 0;
    }
    if (epb) *epb = e;
    if (bpb) *bpb = b;
    return 1;
}

uint64_t vbs_oracle_row_bytes(int type, uint32_t cols) {
    uint32_t e, b;
    if (!vbs_oracle_geometry(type, &e, &b)) return 0;
    return (uint64_t)(cols / e) * b;
}

/* ------------------------------------------------------------------ */
/* block dequantisation                                                */
/* ------------------------------------------------------------------ */

/* src/vbs_dequant.c:123-132: value = ((float)nib - 8) * d; element i < 16
 * is the low nibble of qs[i], element i >= 16 the high nibble of qs[i-16]. */
static void dq_q4_0(const uint8_t *b, float *y) {
    float d = vbs_oracle_f16_to_f32(rd16(b));
    for (int e = 0; e < 32; e++) {
        uint8_t byte = b[2 + (e & 15)];
        int nib = e < 16 ? (byte & 15) : (byte >> 4);
        y[e] = ((float)nib - 8.0f) * d;
    }
}

/* src/vbs_dequant.c:134-143: value = d * nib + m (two roundings). */
static void dq_q4_1(const uint8_t *b, float *y) {
    float d = vbs_oracle_f16_to_f32(rd16(b));
    float m = vbs_oracle_f16_to_f32(rd16(b + 2));
    for (int e = 0; e < 32; e++) {
        uint8_t byte = b[4 + (e & 15)];
        int nib = e < 16 ? (byte & 15) : (byte >> 4);
        float t = d * (float)nib;
        y[e] = t + m;
    }
}

/* src/vbs_dequant.c:174-179: value = d * q, q signed. */
static void dq_q8_0(const uint8_t *b, float *y) {
    float d = vbs_oracle_f16_to_f32(rd16(b));
    for (int e = 0; e < 32; e++) y[e] = d * (float)(int8_t)b[2 + e];
}

/* Sub-block j (0..7) 6-bit scale and min of a Q4_K super-block,
 * src/vbs_dequant.c:225-233: j < 4 take the low 6 bits of bytes j / j+4;
 * j >= 4 combine the nibbles of byte j+4 with the top two bits of bytes
 * j-4 (scale) and j (min). */
static void q4k_scale_min(const uint8_t *s, int j, int *sc, int *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
        return;
    }
    int top_sc = s[j - 4] >> 6, top_mn = s[j] >> 6;
    *sc = (s[j + 4] & 15) | (top_sc << 4);
    *mn = (s[j + 4] >> 4) | (top_mn << 4);
}

/* src/vbs_dequant.c:258-277: d and dmin first, scales[12] at 4, qs[128] at
 * 16; element e lives in qs[32*(e/64) + e%32], low nibble when e%64 < 32.
 * value = ((d * sc) * nib) - (dmin * m). */
static void dq_q4_k(const uint8_t *b, float *y) {
    float d = vbs_oracle_f16_to_f32(rd16(b));
    float dmin = vbs_oracle_f16_to_f32(rd16(b + 2));
    const uint8_t *s = b + 4, *qs = b + 16;
    for (int j = 0; j < 8; j++) {
        int sc, mn;
        q4k_scale_min(s, j, &sc, &mn);
        const uint8_t *grp = qs + 32 * (j >> 1);
        int hi = j & 1;
        for (int l = 0; l < 32; l++) {
            int nib = hi ? (grp[l] >> 4) : (grp[l] & 15);
            float a = d * (float)sc;
            float p = a * (float)nib;
            float c = dmin * (float)mn;
            y[32 * j + l] = p - c;
        }
    }
}

/* src/vbs_dequant.c:316-333: ql[128] @0, qh[64] @128, int8 scales[16] @192,
 * d @208. Element e: half h = e/128, quarter q = (e%128)/32, lane l = e%32;
 * low 4 bits from ql[64h + 32(q&1) + l] (shifted by 4 for q >= 2), high 2
 * bits from qh[32h + l] >> 2q; scale index 8h + 2q + l/16.
 * value = ((d * sc) * (q6 - 32)). */
/* quarter q (0..3) of half h: constant shifts, so the 32-element loop
 * vectorises; element l takes scale 8h + 2q + l/16, formed as d * scale once
 * per 16 elements (the same product the reference forms per element) */
#define DQ_Q6K_QUARTER(Q)                                                          \
    do {                                                                           \
        const uint8_t *lq = ql + 64 * h + 32 * ((Q) & 1);                          \
        const uint8_t *hq = qh + 32 * h;                                           \
        float *yq = y + 128 * h + 32 * (Q);                                        \
        float a0 = d * (float)sc[8 * h + 2 * (Q)], a1 = d * (float)sc[8 * h + 2 * (Q) + 1]; \
        for (int l = 0; l < 32; l++) {                                             \
            int lo = (lq[l] >> ((Q) >= 2 ? 4 : 0)) & 15;                           \
            int hi2 = (hq[l] >> (2 * (Q))) & 3;                                    \
            int v = (lo | (hi2 << 4)) - 32;                                        \
            yq[l] = (l < 16 ? a0 : a1) * (float)v;                                 \
        }                                                                          \
    } while (0)

static void dq_q6_k(const uint8_t *b, float *y) {
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    float d = vbs_oracle_f16_to_f32(rd16(b + 208));
    for (int h = 0; h < 2; h++) {
        DQ_Q6K_QUARTER(0);
        DQ_Q6K_QUARTER(1);
        DQ_Q6K_QUARTER(2);
        DQ_Q6K_QUARTER(3);
    }
}

/* LNS8, src/vbs_host_math.h:111-121 and 250-255 (the reference keeps it in
 * the host math, not in vbs_dequant_block): 32 codes, f32 scale at byte 32,
 * value = exp2f(code) * scale. */
static void dq_lns8(const uint8_t *b, float *y) {
    float scale;
    memcpy(&scale, b + 32, 4);
    for (int i = 0; i < 32; i++) y[i] = exp2f((float)b[i]) * scale;
}

/* src/vbs_dequant.c:339-356 (hot-path types; LNS8 added for the bridge). */
int vbs_oracle_dequant_block(int type, const uint8_t *blk, float *out) {
    if (!blk || !out) return 0;
    switch (type) {
        case T_Q4_0: dq_q4_0(blk, out); return 32;
        case T_Q4_1: dq_q4_1(blk, out); return 32;
        case T_Q8_0: dq_q8_0(blk, out); return 32;
        case T_Q4_K: dq_q4_k(blk, out); return 256;
        case T_Q6_K: dq_q6_k(blk, out); return 256;
        case T_LNS8: dq_lns8(blk, out); return 32;
        default: return 0;
    }
}

/* src/vbs_host_math.h:94-129 (F32 copy, F16 per element, blocks in order). */
int vbs_oracle_dequant_row(int type, const uint8_t *row, uint32_t cols, float *out) {
    uint32_t epb, bpb;
    if (!vbs_oracle_geometry(type, &epb, &bpb)) return 0;
    if (type == T_F32) { memcpy(out, row, (size_t)cols * 4); return 1; }
    if (type == T_F16) {
        for (uint32_t i = 0; i < cols; i++) out[i] = vbs_oracle_f16_to_f32(rd16(row + 2 * (size_t)i));
        return 1;
    }
    for (uint32_t b = 0; b < cols / epb; b++)
        if (vbs_oracle_dequant_block(type, row + (size_t)b * bpb, out + (size_t)b * epb) != (int)epb)
            return 0;
    return 1;
}

/* ------------------------------------------------------------------ */
/* linear tile                                                         */
/* ------------------------------------------------------------------ */

/* src/vbs_host_math.h:223-267: per row, dequantise block by block and
 * accumulate (double)w * x in double in element order; the float result
 * replaces y[row_off + r] or is added to it. cols must be a whole number
 * of blocks. */
static int linear_rows(int type, const uint8_t *w, const float *x, float *y, uint32_t cols,
                       uint32_t r0, uint32_t r1, uint32_t col_off, uint32_t row_off,
                       int accumulate) {
    uint32_t epb, bpb;
    if (!vbs_oracle_geometry(type, &epb, &bpb) || cols % epb) return 0;
    uint64_t rb = (uint64_t)(cols / epb) * bpb;
    float vals[4][256];
    const float *xs = x + col_off;
    /* four rows at a time: each keeps its own double sum over its elements in
     * order (the rows' sums are independent chains, so they overlap in the
     * pipeline; no row's arithmetic changes) */
    uint32_t r = r0;
    if (type != T_F32 && type != T_F16) {
        for (; r + 4 <= r1; r += 4) {
            double acc[4] = {0.0, 0.0, 0.0, 0.0};
            for (uint32_t b = 0; b < cols / epb; b++) {
                const float *xb = xs + (size_t)b * epb;
                for (int k = 0; k < 4; k++) {
                    const uint8_t *blk = w + (uint64_t)(r + k) * rb + (uint64_t)b * bpb;
                    if (vbs_oracle_dequant_block(type, blk, vals[k]) != (int)epb) return 0;
                }
                for (uint32_t i = 0; i < epb; i++) {
                    double xi = xb[i];
                    acc[0] += (double)vals[0][i] * xi;
                    acc[1] += (double)vals[1][i] * xi;
                    acc[2] += (double)vals[2][i] * xi;
                    acc[3] += (double)vals[3][i] * xi;
                }
            }
            for (int k = 0; k < 4; k++) {
                float *dst = y + row_off + r + k;
                *dst = accumulate ? *dst + (float)acc[k] : (float)acc[k];
            }
        }
    }
    for (; r < r1; r++) {
        const uint8_t *row = w + (uint64_t)r * rb;
        double acc = 0.0;
        for (uint32_t b = 0; b < cols / epb; b++) {
            const uint8_t *blk = row + (uint64_t)b * bpb;
            const float *xb = xs + (size_t)b * epb;
            if (type == T_F32) {
                float wf;
                memcpy(&wf, blk, 4);
                acc += (double)wf * xb[0];
            } else if (type == T_F16) {
                acc += (double)vbs_oracle_f16_to_f32(rd16(blk)) * xb[0];
            } else {
                if (vbs_oracle_dequant_block(type, blk, vals[0]) != (int)epb) return 0;
                for (uint32_t i = 0; i < epb; i++) acc += (double)vals[0][i] * xb[i];
            }
        }
        float *dst = y + row_off + r;
        *dst = accumulate ? *dst + (float)acc : (float)acc;
    }
    return 1;
}

int vbs_oracle_linear_tile(int type, const uint8_t *w, const float *x, float *y,
                           uint32_t cols, uint32_t rows, uint32_t col_off,
                           uint32_t row_off, int accumulate) {
    return linear_rows(type, w, x, y, cols, 0, rows, col_off, row_off, accumulate);
}

typedef struct {
    int type; const uint8_t *w; const float *x; float *y;
    uint32_t cols, r0, r1, col_off, row_off; int acc; int ok;
} lin_job_t;

static void *lin_worker(void *a) {
    lin_job_t *j = (lin_job_t *)a;
    j->ok = linear_rows(j->type, j->w, j->x, j->y, j->cols, j->r0, j->r1, j->col_off, j->row_off, j->acc);
    return NULL;
}

int vbs_oracle_linear_tile_mt(int type, const uint8_t *w, const float *x, float *y,
                              uint32_t cols, uint32_t rows, uint32_t col_off,
                              uint32_t row_off, int accumulate, int nthreads) {
    if (nthreads <= 1 || rows < 64)
        return linear_rows(type, w, x, y, cols, 0, rows, col_off, row_off, accumulate);
    if (nthreads > 64) nthreads = 64;
    pthread_t th[64];
    lin_job_t jobs[64];
    uint32_t per = (rows + (uint32_t)nthreads - 1) / (uint32_t)nthreads;
    int n = 0;
    for (int t = 0; t < nthreads; t++) {
        uint32_t r0 = (uint32_t)t * per;
        if (r0 >= rows) break;
        uint32_t r1 = r0 + per > rows ? rows : r0 + per;
        jobs[n] = (lin_job_t){type, w, x, y, cols, r0, r1, col_off, row_off, accumulate, 0};
        pthread_create(&th[n], NULL, lin_worker, &jobs[n]);
        n++;
    }
    int ok = 1;
    for (int t = 0; t < n; t++) { pthread_join(th[t], NULL); ok &= jobs[t].ok; }
    return ok;
}

/* ------------------------------------------------------------------ */
/* primitives                                                          */
/* ------------------------------------------------------------------ */

/* src/vbs_host_math.h:136-142: dequantised row `token`; the row stride is
 * (dim / elements_per_block) * bytes_per_block. */
int vbs_oracle_embed_row(int type, const uint8_t *table, uint32_t token, float *out, uint32_t dim) {
    uint64_t rb = vbs_oracle_row_bytes(type, dim);
    if (!rb) return 0;
    return vbs_oracle_dequant_row(type, table + (uint64_t)token * rb, dim, out);
}

/* src/vbs_host_math.h:28-36: ss = sum of (double)x^2; scale =
 * 1 / sqrtf((float)(ss / n) + eps); out = (x * scale) * w. */
void vbs_oracle_rms_norm(const float *in, const float *w, float *out, uint32_t n, float eps) {
    double ss = 0.0;
    for (uint32_t i = 0; i < n; i++) {
        double v = in[i];
        ss += v * v;
    }
    float mean = (float)(ss / (double)n);
    float scale = 1.0f / sqrtf(mean + eps);
    for (uint32_t i = 0; i < n; i++) {
        float t = in[i] * scale;
        out[i] = t * w[i];
    }
}

/* src/vbs_host_math.h:38-51: pairs (i, i+1), i even, of every head rotate
 * by angle = (float)pos * powf(theta, -(float)i / head_dim). */
void vbs_oracle_rope(float *x, uint32_t pos, uint32_t head_dim, uint32_t n_heads, float theta) {
    for (uint32_t i = 0; i + 1 < head_dim; i += 2) {
        float expo = -(float)i / (float)head_dim;
        float ang = (float)pos * powf(theta, expo);
        float c = cosf(ang), s = sinf(ang);
        for (uint32_t h = 0; h < n_heads; h++) {
            float *p = x + (size_t)h * head_dim + i;
            float a = p[0], b = p[1];
            float ac = a * c, bs = b * s, as = a * s, bc = b * c;
            p[0] = ac - bs;
            p[1] = as + bc;
        }
    }
}

/* src/vbs_host_math.h:53-57: out = (g / (1 + expf(-g))) * u. */
void vbs_oracle_silu_mul(const float *gate, const float *up, float *out, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        float den = 1.0f + expf(-gate[i]);
        float s = gate[i] / den;
        out[i] = s * up[i];
    }
}

/* src/vbs_host_math.h:59-62. */
void vbs_oracle_add(const float *a, const float *b, float *out, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) out[i] = a[i] + b[i];
}

/* src/vbs_host_math.h:150-159: f16 store at ((layer*max_ctx + pos)*kv_dim + i). */
void vbs_oracle_cache_store(const float *k, const float *v, uint16_t *kc, uint16_t *vc,
                            uint32_t pos, uint32_t layer, uint32_t max_ctx, uint32_t kv_dim) {
    uint64_t base = ((uint64_t)layer * max_ctx + pos) * kv_dim;
    for (uint32_t i = 0; i < kv_dim; i++) {
        kc[base + i] = vbs_oracle_f32_to_f16(k[i]);
        vc[base + i] = vbs_oracle_f32_to_f16(v[i]);
    }
}

/* Every half as a float, built once by vbs_oracle_f16_to_f32 itself: the
 * attention below reads keys and values through it (the same values, without
 * a call and its branches per cached element). */
static float g_half_table[65536];
static pthread_once_t g_half_once = PTHREAD_ONCE_INIT;
static void half_table_init(void) {
    for (uint32_t h = 0; h < 65536u; h++) g_half_table[h] = vbs_oracle_f16_to_f32((uint16_t)h);
}

/* src/vbs_host_math.h:170-209 for q heads [h0, h1): for each q head h (kv
 * head h / group): sequential online softmax over s < seq_len with score =
 * (float)(double dot) * scale, m starting at -FLT_MAX, r = expf(m - m'),
 * e = expf(score - m'), l = l*r + e, acc = acc*r + e*v; out = acc * (1 / l).
 * Heads are independent, so splitting them over threads changes no result. */
static void attention_heads(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                            uint32_t seq_len, uint64_t lbase, uint32_t nkh, uint32_t hd,
                            uint32_t group, float scale, uint32_t h0, uint32_t h1) {
    const float *f16 = g_half_table;
    for (uint32_t h = h0; h < h1; h++) {
        const float *qh = q + (size_t)h * hd;
        float *acc = out + (size_t)h * hd;
        uint32_t kvh = h / group;
        float m = -3.4028235e38f, l = 0.0f;
        for (uint32_t d = 0; d < hd; d++) acc[d] = 0.0f;
        for (uint32_t s = 0; s < seq_len; s++) {
            uint64_t at = lbase + ((uint64_t)s * nkh + kvh) * hd;
            double dot = 0.0;
            for (uint32_t d = 0; d < hd; d++) dot += (double)qh[d] * (double)f16[kc[at + d]];
            float score = (float)dot * scale;
            float mn = score > m ? score : m;
            float r = expf(m - mn);
            float e = expf(score - mn);
            float lr = l * r;
            l = lr + e;
            m = mn;
            for (uint32_t d = 0; d < hd; d++) {
                float vv = f16[vc[at + d]];
                float ar = acc[d] * r, ev = e * vv;
                acc[d] = ar + ev;
            }
        }
        float inv = 1.0f / l;
        for (uint32_t d = 0; d < hd; d++) acc[d] *= inv;
    }
}

typedef struct {
    const float *q; const uint16_t *kc, *vc; float *out;
    uint32_t seq_len; uint64_t lbase; uint32_t nkh, hd, group; float scale; uint32_t h0, h1;
} attn_job_t;

static void *attn_worker(void *a) {
    attn_job_t *j = (attn_job_t *)a;
    attention_heads(j->q, j->kc, j->vc, j->out, j->seq_len, j->lbase, j->nkh, j->hd, j->group,
                    j->scale, j->h0, j->h1);
    return NULL;
}

void vbs_oracle_attention_mt(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                             uint32_t seq_len, uint32_t layer, uint32_t max_ctx, uint32_t nqh,
                             uint32_t nkh, uint32_t hd, float scale, int nthreads) {
    if (!nkh || !nqh || !hd) return;
    pthread_once(&g_half_once, half_table_init);
    uint32_t group = nqh / nkh ? nqh / nkh : 1;
    uint64_t lbase = (uint64_t)layer * max_ctx * nkh * hd;
    if (nthreads > 64) nthreads = 64;
    if (nthreads > (int)nqh) nthreads = (int)nqh;
    if (nthreads <= 1) {
        attention_heads(q, kc, vc, out, seq_len, lbase, nkh, hd, group, scale, 0, nqh);
        return;
    }
    pthread_t th[64];
    attn_job_t jobs[64];
    uint32_t per = (nqh + (uint32_t)nthreads - 1) / (uint32_t)nthreads;
    int n = 0;
    for (int t = 0; t < nthreads; t++) {
        uint32_t h0 = (uint32_t)t * per, h1 = h0 + per < nqh ? h0 + per : nqh;
        if (h0 >= h1) break;
        jobs[n] = (attn_job_t){q, kc, vc, out, seq_len, lbase, nkh, hd, group, scale, h0, h1};
        if (pthread_create(&th[n], NULL, attn_worker, &jobs[n]) != 0) {
            attention_heads(q, kc, vc, out, seq_len, lbase, nkh, hd, group, scale, h0, h1);
            continue;
        }
        n++;
    }
    for (int t = 0; t < n; t++) pthread_join(th[t], NULL);
}

void vbs_oracle_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                          uint32_t seq_len, uint32_t layer, uint32_t max_ctx, uint32_t nqh,
                          uint32_t nkh, uint32_t hd, float scale) {
    vbs_oracle_attention_mt(q, kc, vc, out, seq_len, layer, max_ctx, nqh, nkh, hd, scale, 1);
}

/* ------------------------------------------------------------------ */
/* one decode step                                                     */
/* ------------------------------------------------------------------ */

/* src/vbs_specializer.c:231-349 with the bridge arguments of
 * src/vbs_specializer_bridge.c:148-183 (eps, theta, seq_len = pos + 1,
 * scale = 1/sqrtf(head_dim)). */
int vbs_oracle_forward_token(const vbs_oracle_model_t *m, uint32_t token, uint32_t pos,
                             float *logits, int nt) {
    uint32_t H = m->hidden, F = m->ffn, hd = m->head_dim;
    uint32_t qd = m->n_heads * hd, kvd = m->n_kv_heads * hd;
    float *buf = (float *)calloc((size_t)4 * H + 2 * qd + 2 * kvd + 3 * F, sizeof(float));
    if (!buf) return 0;
    float *stream = buf, *normed = stream + H, *tmp = normed + H, *qb = tmp + H;
    float *kb = qb + qd, *vb = kb + kvd, *ab = vb + kvd, *gate = ab + qd, *up = gate + F;
    float *hid = up + F;
    int ok = vbs_oracle_embed_row(m->embd_type, m->tok_embd, token, stream, H);
    float scale = 1.0f / sqrtf((float)hd);
    for (uint32_t L = 0; ok && L < m->n_layers; L++) {
        const int *t = m->wtype + 7 * L;
        const uint8_t *const *w = m->wdata + 7 * L;
        vbs_oracle_rms_norm(stream, m->attn_norm[L], normed, H, m->rms_eps);
        ok &= vbs_oracle_linear_tile_mt(t[0], w[0], normed, qb, H, qd, 0, 0, 0, nt);
        vbs_oracle_rope(qb, pos, hd, m->n_heads, m->rope_theta);
        ok &= vbs_oracle_linear_tile_mt(t[1], w[1], normed, kb, H, kvd, 0, 0, 0, nt);
        vbs_oracle_rope(kb, pos, hd, m->n_kv_heads, m->rope_theta);
        ok &= vbs_oracle_linear_tile_mt(t[2], w[2], normed, vb, H, kvd, 0, 0, 0, nt);
        vbs_oracle_cache_store(kb, vb, m->kc, m->vc, pos, L, m->max_ctx, kvd);
        vbs_oracle_attention_mt(qb, m->kc, m->vc, ab, pos + 1, L, m->max_ctx, m->n_heads,
                                m->n_kv_heads, hd, scale, nt);
        ok &= vbs_oracle_linear_tile_mt(t[3], w[3], ab, tmp, qd, H, 0, 0, 0, nt);
        vbs_oracle_add(stream, tmp, stream, H);
        vbs_oracle_rms_norm(stream, m->ffn_norm[L], normed, H, m->rms_eps);
        ok &= vbs_oracle_linear_tile_mt(t[4], w[4], normed, gate, H, F, 0, 0, 0, nt);
        ok &= vbs_oracle_linear_tile_mt(t[5], w[5], normed, up, H, F, 0, 0, 0, nt);
        vbs_oracle_silu_mul(gate, up, hid, F);
        ok &= vbs_oracle_linear_tile_mt(t[6], w[6], hid, tmp, F, H, 0, 0, 0, nt);
        vbs_oracle_add(stream, tmp, stream, H);
    }
    if (ok) {
        vbs_oracle_rms_norm(stream, m->out_norm, normed, H, m->rms_eps);
        ok = vbs_oracle_linear_tile_mt(m->head_type, m->lm_head, normed, logits, H, m->vocab,
                                       0, 0, 0, nt);
    }
    free(buf);
    return ok;
}

/* ------------------------------------------------------------------ */
/* CPU hot-kernel table (ABI v1) and its activation quantiser          */
/* ------------------------------------------------------------------ */

/* src/vbs_cpu.c:74-93: round to nearest even in the normal and the
 * subnormal range; exponent above 15 (inf, NaN included) -> infinity;
 * exponent below -25 -> zero. */
uint16_t vbs_oracle_f32_to_f16_rne(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    int e = (int)((u >> 23) & 255u) - 127;
    uint32_t man = u & 0x7FFFFFu;
    if (e > 15) return (uint16_t)(sign | 0x7C00u);
    if (e >= -14) {
        uint32_t h = (uint32_t)(e + 15) << 10 | man >> 13;
        uint32_t low = man & 0x1FFFu;
        if (low > 0x1000u || (low == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (e < -25) return sign;
    man |= 0x800000u;
    int sh = -e - 1;
    uint32_t h = man >> sh, low = man & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (low > half || (low == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* src/vbs_cpu.c:166-182. Per 32-element block: d = amax/127, q =
 * roundf(x * (1/d)) clamped to +-127 (all zero when d == 0), qd = f16(d),
 * qsum = f16(sum(q) * d), both through the RNE conversion above. */
void vbs_oracle_quantize_q8(const float *x, uint32_t cols, int8_t *xq, float *qd, float *qsum) {
    for (uint32_t b = 0; b < cols / 32; b++) {
        const float *xb = x + (size_t)b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++)
            if (fabsf(xb[i]) > amax) amax = fabsf(xb[i]);
        float d = amax / 127.0f;
        float inv = d != 0.0f ? 1.0f / d : 0.0f;
        int total = 0;
        for (int i = 0; i < 32; i++) {
            int q = (int)roundf(xb[i] * inv);
            if (q < -127) q = -127;
            if (q > 127) q = 127;
            xq[(size_t)b * 32 + i] = (int8_t)q;
            total += q;
        }
        qd[b] = vbs_oracle_f16_to_f32(vbs_oracle_f32_to_f16_rne(d));
        qsum[b] = vbs_oracle_f16_to_f32(vbs_oracle_f32_to_f16_rne((float)total * d));
    }
}

/* src/hotkernels/vbs_hot_ref_impl.h:49-129. Quantised rows: one float sum
 * per row, per block `sum += f16(d) * qd[b] * (float)dot` with an exact
 * int dot (Q4_0 nibbles - 8, Q4_1 nibbles plus `sum += f16(m) * qsum[b]`).
 * F32 / F16 rows: `sum += w[i] * x[i]` element by element. */
int vbs_oracle_hot_matvec(int type, const void *wv, uint32_t rows, uint32_t cols,
                          const int8_t *xq, const float *qd, const float *qsum, const float *x,
                          float *y) {
    const uint8_t *w = (const uint8_t *)wv;
    size_t nb = cols / 32;
    for (uint32_t r = 0; r < rows; r++) {
        float sum = 0.0f;
        switch (type) {
            case T_Q8_0:
                for (size_t b = 0; b < nb; b++) {
                    const uint8_t *blk = w + ((size_t)r * nb + b) * 34;
                    int dot = 0;
                    for (int i = 0; i < 32; i++) dot += (int)(int8_t)blk[2 + i] * (int)xq[b * 32 + i];
                    sum += vbs_oracle_f16_to_f32(rd16(blk)) * qd[b] * (float)dot;
                }
                break;
            case T_Q4_0:
            case T_Q4_1: {
                size_t bs = type == T_Q4_0 ? 18 : 20, qo = type == T_Q4_0 ? 2 : 4;
                int off = type == T_Q4_0 ? 8 : 0;
                for (size_t b = 0; b < nb; b++) {
                    const uint8_t *blk = w + ((size_t)r * nb + b) * bs;
                    int dot = 0;
                    for (int i = 0; i < 16; i++) {
                        dot += ((int)(blk[qo + i] & 15u) - off) * (int)xq[b * 32 + i];
                        dot += ((int)(blk[qo + i] >> 4) - off) * (int)xq[b * 32 + 16 + i];
                    }
                    sum += vbs_oracle_f16_to_f32(rd16(blk)) * qd[b] * (float)dot;
                    if (type == T_Q4_1) sum += vbs_oracle_f16_to_f32(rd16(blk + 2)) * qsum[b];
                }
                break;
            }
            case T_F32:
                for (size_t i = 0; i < cols; i++) {
                    float wi;
                    memcpy(&wi, w + ((size_t)r * cols + i) * 4, 4);
                    sum += wi * x[i];
                }
                break;
            case T_F16:
                for (size_t i = 0; i < cols; i++)
                    sum += vbs_oracle_f16_to_f32(rd16(w + ((size_t)r * cols + i) * 2)) * x[i];
                break;
            default:
                return 0;
        }
        y[r] = sum;
    }
    return 1;
}
