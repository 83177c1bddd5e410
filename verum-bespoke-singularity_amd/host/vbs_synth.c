/* vbs_synth.c — deterministic synthetic GGUF blocks (see vbs_synth.h). */
#include "vbs_synth.h"
#include "vbs_half.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct { uint64_t s; } rng_t;

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* splitmix64 stream keyed by (seed, stream, index). */
static rng_t rng_at(uint64_t seed, uint64_t stream, uint64_t index) {
    rng_t r;
    r.s = mix64(seed ^ mix64(stream * 0x9E3779B97F4A7C15ull + 0x632BE59BD9B4E019ull)) ^
          mix64(index + 0x8CB92BA72F3D8DD7ull);
    return r;
}

static uint64_t next64(rng_t *r) {
    r->s += 0x9E3779B97F4A7C15ull;
    return mix64(r->s);
}

/* uniform integer in [0, n) */
static uint32_t below(rng_t *r, uint32_t n) {
    return (uint32_t)(((next64(r) >> 32) * (uint64_t)n) >> 32);
}

/* standard normal, Box-Muller in double */
static double normal(rng_t *r) {
    double u1 = ((double)(next64(r) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    double u2 = (double)(next64(r) >> 11) * (1.0 / 9007199254740992.0);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

static void fill_nibbles(rng_t *r, uint8_t *qs, int nbytes) {
    for (int i = 0; i < nbytes; i += 8) {
        uint64_t v = next64(r);
        for (int k = 0; k < 8 && i + k < nbytes; k++) qs[i + k] = (uint8_t)(v >> (8 * k));
    }
}

static void gen_block(int type, rng_t *r, uint8_t *b) {
    switch (type) {
        case 2: /* Q4_0 */
            put16(b, vbs_f2h((float)fabs(normal(r)) * 0.02f));
            fill_nibbles(r, b + 2, 16);
            break;
        case 3: /* Q4_1 */
            put16(b, vbs_f2h((float)fabs(normal(r)) * 0.01f));
            put16(b + 2, vbs_f2h((float)normal(r) * 0.01f));
            fill_nibbles(r, b + 4, 16);
            break;
        case 8: /* Q8_0 */
            put16(b, vbs_f2h((float)fabs(normal(r)) * 0.01f));
            for (int i = 0; i < 32; i++) b[2 + i] = (uint8_t)(int8_t)((int)below(r, 255) - 127);
            break;
        case 12: { /* Q4_K */
            put16(b, vbs_f2h((float)fabs(normal(r)) * 0.01f));
            put16(b + 2, vbs_f2h((float)fabs(normal(r)) * 0.01f));
            int sc[8], mn[8];
            for (int j = 0; j < 8; j++) { sc[j] = (int)below(r, 64); mn[j] = (int)below(r, 64); }
            uint8_t *s = b + 4;
            for (int j = 0; j < 4; j++) {
                s[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
                s[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
                s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
            }
            fill_nibbles(r, b + 16, 128);
            break;
        }
        case 14: { /* Q6_K */
            uint8_t *ql = b, *qh = b + 128;
            memset(b, 0, 192);
            put16(b + 208, vbs_f2h((float)fabs(normal(r)) * 0.01f));
            for (int i = 0; i < 16; i++) b[192 + i] = (uint8_t)(int8_t)((int)below(r, 64) - 32);
            for (int e = 0; e < 256; e++) {
                int q6 = (int)below(r, 64);
                int h = e >> 7, q = (e >> 5) & 3, l = e & 31;
                int qi = 64 * h + 32 * (q & 1) + l;
                ql[qi] |= (uint8_t)((q6 & 15) << (q >= 2 ? 4 : 0));
                qh[32 * h + l] |= (uint8_t)((q6 >> 4) << (2 * q));
            }
            break;
        }
        case 0: { /* F32 */
            float f = (float)normal(r);
            memcpy(b, &f, 4);
            break;
        }
        case 1: /* F16 */
            put16(b, vbs_f2h((float)normal(r)));
            break;
        default: break;
    }
}

static int block_bytes(int type) {
    switch (type) {
        case 0: return 4;
        case 1: return 2;
        case 2: return 18;
        case 3: return 20;
        case 8: return 34;
        case 12: return 144;
        case 14: return 210;
        default: return 0;
    }
}

typedef struct {
    int type; uint64_t seed, stream, first, n; uint8_t *out;
    float scale, offset; int kind; /* 0 blocks, 1 f32 normal, 2 f16 normal */
} job_t;

static void *worker(void *a) {
    job_t *j = (job_t *)a;
    if (j->kind == 0) {
        int bb = block_bytes(j->type);
        for (uint64_t i = 0; i < j->n; i++) {
            rng_t r = rng_at(j->seed, j->stream, j->first + i);
            gen_block(j->type, &r, j->out + i * (uint64_t)bb);
        }
        return NULL;
    }
    /* Normals come in chunks of 256 elements per counter so any element
     * range regenerates identically. */
    uint64_t i = 0;
    while (i < j->n) {
        uint64_t g = j->first + i, chunk = g >> 8;
        rng_t r = rng_at(j->seed, j->stream, chunk);
        for (uint64_t k = 0; k < (g & 255u); k++) (void)normal(&r);
        for (uint64_t k = g & 255u; k < 256 && i < j->n; k++, i++) {
            float v = (float)normal(&r);
            if (j->kind == 1) ((float *)j->out)[i] = j->offset + j->scale * v;
            else ((uint16_t *)j->out)[i] = vbs_f2h(j->scale * v);
        }
    }
    return NULL;
}

static void run_jobs(job_t proto, int elem_bytes, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    if (proto.n < 4096) nthreads = 1;
    pthread_t th[64];
    job_t jobs[64];
    uint64_t per = (proto.n + (uint64_t)nthreads - 1) / (uint64_t)nthreads;
    int launched = 0;
    for (int t = 0; t < nthreads; t++) {
        uint64_t s = (uint64_t)t * per;
        if (s >= proto.n) break;
        jobs[t] = proto;
        jobs[t].first = proto.first + s;
        jobs[t].n = s + per > proto.n ? proto.n - s : per;
        jobs[t].out = proto.out + s * (uint64_t)elem_bytes;
        if (nthreads == 1) { worker(&jobs[t]); continue; }
        pthread_create(&th[t], NULL, worker, &jobs[t]);
        launched++;
    }
    for (int t = 0; t < launched; t++) pthread_join(th[t], NULL);
}

int vbs_synth_blocks(int type, uint64_t seed, uint64_t stream, uint64_t first_block,
                     uint64_t n_blocks, void *out, int nthreads) {
    int bb = block_bytes(type);
    if (!bb || !out) return 0;
    job_t p = {type, seed, stream, first_block, n_blocks, (uint8_t *)out, 0.f, 0.f, 0};
    run_jobs(p, bb, nthreads);
    return 1;
}

void vbs_synth_normal_f32(uint64_t seed, uint64_t stream, uint64_t first, size_t n,
                          float scale, float offset, float *out, int nthreads) {
    job_t p = {0, seed, stream, first, n, (uint8_t *)out, scale, offset, 1};
    run_jobs(p, 4, nthreads);
}

void vbs_synth_normal_f16(uint64_t seed, uint64_t stream, uint64_t first, size_t n,
                          float scale, uint16_t *out, int nthreads) {
    job_t p = {0, seed, stream, first, n, (uint8_t *)out, scale, 0.f, 2};
    run_jobs(p, 2, nthreads);
}

void vbs_synth_tokens(uint64_t seed, uint64_t stream, uint32_t vocab, size_t n, uint32_t *out) {
    for (size_t i = 0; i < n; i++) {
        rng_t r = rng_at(seed, stream, i);
        out[i] = below(&r, vocab);
    }
}


/* ---- GGUF v3 writer ---------------------------------------------------------
 * Layout (as src/vbs_gguf.c reads it): "GGUF", u32 version 3, u64 tensor
 * count, u64 metadata count; metadata records (string key, u32 type, value);
 * tensor records (string name, u32 n_dims, u64 dims innermost first, u32
 * type, u64 offset into the data section); zero padding to the alignment;
 * tensor data, each tensor starting at a multiple of the alignment. */
enum { GG_UINT32 = 4, GG_FLOAT32 = 6, GG_STRING = 8 };
enum { GG_ALIGN = 32 };

typedef struct {
    FILE *f;
    int ok;
} gw_t;

static void gw_bytes(gw_t *w, const void *p, size_t n) {
    if (w->ok && n && fwrite(p, 1, n, w->f) != n) w->ok = 0;
}
static void gw_u32(gw_t *w, uint32_t v) { gw_bytes(w, &v, 4); }
static void gw_u64(gw_t *w, uint64_t v) { gw_bytes(w, &v, 8); }
static void gw_str(gw_t *w, const char *s) {
    const uint64_t n = strlen(s);
    gw_u64(w, n);
    gw_bytes(w, s, n);
}
static void gw_kv_u32(gw_t *w, const char *k, uint32_t v) {
    gw_str(w, k);
    gw_u32(w, GG_UINT32);
    gw_u32(w, v);
}
static void gw_kv_f32(gw_t *w, const char *k, float v) {
    gw_str(w, k);
    gw_u32(w, GG_FLOAT32);
    gw_bytes(w, &v, 4);
}
static void gw_kv_str(gw_t *w, const char *k, const char *v) {
    gw_str(w, k);
    gw_u32(w, GG_STRING);
    gw_str(w, v);
}
static void gw_pad(gw_t *w, uint64_t *pos) {
    static const uint8_t zero[GG_ALIGN] = {0};
    const uint64_t r = *pos % GG_ALIGN;
    if (r) {
        gw_bytes(w, zero, GG_ALIGN - r);
        *pos += GG_ALIGN - r;
    }
}

typedef struct {
    char name[64];
    int type;            /* ggml type; 0 (F32) for the norms */
    uint64_t rows, cols; /* cols innermost */
    uint64_t stream;
    int is_norm;         /* f32 N(0,1)*0.1 + 1 */
    uint64_t offset;     /* into the data section */
    uint64_t bytes;
} gt_t;

static int geometry(int type, uint32_t *e, uint32_t *b) {
    switch (type) {
        case 0: *e = 1; *b = 4; return 1;
        case 1: *e = 1; *b = 2; return 1;
        case 2: *e = 32; *b = 18; return 1;
        case 3: *e = 32; *b = 20; return 1;
        case 8: *e = 32; *b = 34; return 1;
        case 12: *e = 256; *b = 144; return 1;
        case 14: *e = 256; *b = 210; return 1;
        default: return 0;
    }
}

int vbs_synth_write_gguf(const char *path, const vbs_synth_gguf_cfg_t *c, char *err, size_t cap) {
    if (!path || !c) { snprintf(err, cap, "null argument"); return 0; }
    if (!c->n_layers || !c->hidden || !c->ffn || !c->n_heads || !c->n_kv_heads || !c->head_dim ||
        !c->vocab || !c->context_length) {
        snprintf(err, cap, "empty model dimension");
        return 0;
    }
    const uint64_t H = c->hidden, F = c->ffn, qd = (uint64_t)c->n_heads * c->head_dim;
    const uint64_t kvd = (uint64_t)c->n_kv_heads * c->head_dim;
    const size_t nt = 3 + 9 * (size_t)c->n_layers;
    gt_t *t = (gt_t *)calloc(nt, sizeof(gt_t));
    if (!t) { snprintf(err, cap, "out of memory"); return 0; }
    size_t k = 0;
    const uint64_t roles_rc[7][2] = {{qd, H}, {kvd, H}, {kvd, H}, {H, qd}, {F, H}, {F, H}, {H, F}};
    static const char *role_names[7] = {"attn_q", "attn_k", "attn_v", "attn_output",
                                        "ffn_gate", "ffn_up", "ffn_down"};
    snprintf(t[k].name, sizeof t[k].name, "token_embd.weight");
    t[k].type = c->embd_type; t[k].rows = c->vocab; t[k].cols = H; t[k].stream = 1; k++;
    for (uint32_t L = 0; L < c->n_layers; L++) {
        /* attn_norm, q, k, v, o, ffn_norm, gate, up, down */
        static const int order[9] = {-1, 0, 1, 2, 3, -2, 4, 5, 6};
        for (int i = 0; i < 9; i++) {
            gt_t *x = &t[k++];
            const int m = order[i];
            if (m < 0) {
                snprintf(x->name, sizeof x->name, "blk.%u.%s.weight", L,
                         m == -1 ? "attn_norm" : "ffn_norm");
                x->type = 0; x->rows = 1; x->cols = H; x->is_norm = 1;
                x->stream = 100 + 16ull * L + (m == -1 ? 8 : 9);
            } else {
                snprintf(x->name, sizeof x->name, "blk.%u.%s.weight", L, role_names[m]);
                x->type = c->wtype[m]; x->rows = roles_rc[m][0]; x->cols = roles_rc[m][1];
                x->stream = 100 + 16ull * L + (uint64_t)m;
            }
        }
    }
    snprintf(t[k].name, sizeof t[k].name, "output_norm.weight");
    t[k].type = 0; t[k].rows = 1; t[k].cols = H; t[k].is_norm = 1; t[k].stream = 3; k++;
    snprintf(t[k].name, sizeof t[k].name, "output.weight");
    t[k].type = c->head_type; t[k].rows = c->vocab; t[k].cols = H; t[k].stream = 2; k++;
    if (k != nt) { free(t); snprintf(err, cap, "internal: %zu tensors, expected %zu", k, nt); return 0; }
    uint64_t off = 0;
    for (size_t i = 0; i < nt; i++) {
        uint32_t e, b;
        if (!geometry(t[i].type, &e, &b) || t[i].cols % e) {
            snprintf(err, cap, "tensor %s: type %d does not fit %llu columns", t[i].name, t[i].type,
                     (unsigned long long)t[i].cols);
            free(t);
            return 0;
        }
        t[i].bytes = t[i].rows * (t[i].cols / e) * b;
        t[i].offset = off;
        off = (off + t[i].bytes + GG_ALIGN - 1) / GG_ALIGN * GG_ALIGN;
    }
    gw_t w = {fopen(path, "wb"), 1};
    if (!w.f) { free(t); snprintf(err, cap, "cannot create %s", path); return 0; }
    gw_bytes(&w, "GGUF", 4);
    gw_u32(&w, 3);
    gw_u64(&w, nt);
    gw_u64(&w, 12);
    gw_kv_str(&w, "general.architecture", "llama");
    gw_kv_u32(&w, "general.alignment", GG_ALIGN);
    gw_kv_u32(&w, "llama.block_count", c->n_layers);
    gw_kv_u32(&w, "llama.context_length", c->context_length);
    gw_kv_u32(&w, "llama.embedding_length", c->hidden);
    gw_kv_u32(&w, "llama.feed_forward_length", c->ffn);
    gw_kv_u32(&w, "llama.attention.head_count", c->n_heads);
    gw_kv_u32(&w, "llama.attention.head_count_kv", c->n_kv_heads);
    gw_kv_u32(&w, "llama.rope.dimension_count", c->head_dim);
    gw_kv_f32(&w, "llama.rope.freq_base", c->rope_theta);
    gw_kv_f32(&w, "llama.attention.layer_norm_rms_epsilon", c->rms_eps);
    gw_kv_u32(&w, "llama.vocab_size", c->vocab);
    for (size_t i = 0; i < nt; i++) {
        gw_str(&w, t[i].name);
        const int two = !t[i].is_norm;
        gw_u32(&w, two ? 2 : 1);
        gw_u64(&w, t[i].cols);
        if (two) gw_u64(&w, t[i].rows);
        gw_u32(&w, (uint32_t)t[i].type);
        gw_u64(&w, t[i].offset);
    }
    long hdr = ftell(w.f);
    uint64_t pos = hdr < 0 ? 0 : (uint64_t)hdr;
    gw_pad(&w, &pos);
    /* data: each tensor in chunks of at most 32 MiB of generated blocks */
    const size_t chunk = (size_t)32 << 20;
    uint8_t *buf = (uint8_t *)malloc(chunk);
    if (!buf) w.ok = 0;
    uint64_t data_pos = 0;
    for (size_t i = 0; i < nt && w.ok; i++) {
        static const uint8_t zero[GG_ALIGN] = {0};
        if (data_pos < t[i].offset) {
            gw_bytes(&w, zero, (size_t)(t[i].offset - data_pos));
            data_pos = t[i].offset;
        }
        uint32_t e = 1, b = 4;
        (void)geometry(t[i].type, &e, &b);
        if (t[i].is_norm) {
            vbs_synth_normal_f32(c->seed, t[i].stream, 0, (size_t)t[i].cols, 0.1f, 1.0f, (float *)buf,
                                 c->nthreads);
            gw_bytes(&w, buf, (size_t)t[i].bytes);
        } else {  /* the matrix generators of the test models (F32/F16: N(0,1) elements) */
            const uint64_t nblk = t[i].bytes / b, per = chunk / b;
            for (uint64_t b0 = 0; b0 < nblk && w.ok; b0 += per) {
                const uint64_t n = nblk - b0 < per ? nblk - b0 : per;
                if (t[i].type == 0)
                    vbs_synth_normal_f32(c->seed, t[i].stream, b0, (size_t)n, 1.0f, 0.0f, (float *)buf,
                                         c->nthreads);
                else if (t[i].type == 1)
                    vbs_synth_normal_f16(c->seed, t[i].stream, b0, (size_t)n, 1.0f, (uint16_t *)buf,
                                         c->nthreads);
                else if (!vbs_synth_blocks(t[i].type, c->seed, t[i].stream, b0, n, buf, c->nthreads)) {
                    w.ok = 0;
                    break;
                }
                gw_bytes(&w, buf, (size_t)(n * b));
            }
        }
        data_pos += t[i].bytes;
    }
    free(buf);
    free(t);
    if (fclose(w.f) != 0) w.ok = 0;
    if (!w.ok) { snprintf(err, cap, "write failed: %s", path); return 0; }
    return 1;
}
