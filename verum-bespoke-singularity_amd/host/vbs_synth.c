/* vbs_synth.c — deterministic synthetic GGUF blocks (see vbs_synth.h). */
#include "vbs_synth.h"
#include "vbs_half.h"

#include <math.h>
#include <pthread.h>
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
