/* vbs_decode.c — decode-step driver over a vbs_backend_ops_t table (see
 * vbs_decode.h). The dispatch helpers restate the bridge's contract
 * (src/vbs_specializer_bridge.c:83-206): resident weights use calling
 * convention A (weight_stage == NULL, zero offsets, no accumulate), and
 * primitives pass the canonical argument order with the same scalars. */
#include "vbs_decode.h"
#include "vbs_gfx950.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { SC_Q, SC_K, SC_V, SC_ATTN, SC_GATE, SC_UP, SC_HIDDEN, SC_NORMED, SC_QN, SC_KN, SC_COUNT };

struct vbs_decode {
    const vbs_backend_ops_t *ops;
    vbs_device_t *dev;
    vbs_decode_model_t m;
    vbs_buffer_t *stream, *tmp, *logits, *kc, *vc;
    vbs_buffer_t *scratch[SC_COUNT];
    vbs_buffer_t *tok_embd, *out_norm, *lm_head;
    vbs_buffer_t **attn_norm, **ffn_norm, **w; /* w: n_layers x 7 */
    void *lin_pipe[64];
    void *embed_pipe[64];
    void *prim_pipe[VBS_OP_PROJECTION + 1];
    uint32_t dispatches;
    uint64_t weight_bytes;
    float *host_logits;
    int ok;
    /* device-pointer view for the graph decoder */
    const float **view_attn_norm, **view_ffn_norm;
    const void **view_w;
    int *view_wtype;
};

static uint64_t row_bytes(int type, uint32_t cols) {
    switch (type) {
        case VBS_GGML_TYPE_F32: return 4ull * cols;
        case VBS_GGML_TYPE_F16: return 2ull * cols;
        case VBS_GGML_TYPE_Q4_0: return 18ull * (cols / 32u);
        case VBS_GGML_TYPE_Q4_1: return 20ull * (cols / 32u);
        case VBS_GGML_TYPE_Q8_0: return 34ull * (cols / 32u);
        case VBS_GGML_TYPE_Q4_K: return 144ull * (cols / 256u);
        case VBS_GGML_TYPE_Q6_K: return 210ull * (cols / 256u);
        case VBS_GGML_TYPE_LNS8: return 36ull * (cols / 32u);
        default: return 0;
    }
}

static vbs_buffer_t *upload(vbs_decode_t *d, const void *src, size_t bytes, char *err, size_t cap,
                            const char *what) {
    vbs_buffer_t *b = d->ops->alloc_buffer(d->dev, bytes, false);
    if (!b) {
        snprintf(err, cap, "alloc %s (%zu B) failed", what, bytes);
        return NULL;
    }
    if (src && !d->ops->copy_to_device(b, src, bytes)) {
        snprintf(err, cap, "upload %s (%zu B) failed", what, bytes);
        d->ops->free_buffer(b);
        return NULL;
    }
    d->weight_bytes += bytes;
    return b;
}

/* Matrix shapes of the seven per-layer weights: rows, cols. */
static void mat_shape(const vbs_decode_model_t *m, int k, uint32_t *rows, uint32_t *cols) {
    uint32_t qd = m->n_heads * m->head_dim, kvd = m->n_kv_heads * m->head_dim;
    static const int in_is_q[7] = {0, 0, 0, 1, 0, 0, 0};
    switch (k) {
        case 0: *rows = qd; break;
        case 1: case 2: *rows = kvd; break;
        case 3: *rows = m->hidden; break;
        case 4: case 5: *rows = m->ffn; break;
        default: *rows = m->hidden; break;
    }
    *cols = k == 6 ? m->ffn : (in_is_q[k] ? qd : m->hidden);
}

void vbs_decode_destroy(vbs_decode_t *d) {
    if (!d) return;
    const vbs_backend_ops_t *o = d->ops;
    vbs_buffer_t *single[] = {d->stream, d->tmp, d->logits, d->kc, d->vc,
                              d->tok_embd, d->out_norm, d->lm_head};
    for (size_t i = 0; i < sizeof(single) / sizeof(single[0]); i++)
        if (single[i]) o->free_buffer(single[i]);
    for (int i = 0; i < SC_COUNT; i++)
        if (d->scratch[i]) o->free_buffer(d->scratch[i]);
    for (uint32_t L = 0; L < d->m.n_layers; L++) {
        if (d->attn_norm && d->attn_norm[L]) o->free_buffer(d->attn_norm[L]);
        if (d->ffn_norm && d->ffn_norm[L]) o->free_buffer(d->ffn_norm[L]);
        for (int k = 0; k < 7; k++)
            if (d->w && d->w[7 * L + k]) o->free_buffer(d->w[7 * L + k]);
    }
    free(d->attn_norm);
    free(d->ffn_norm);
    free(d->w);
    free(d->view_attn_norm);
    free(d->view_ffn_norm);
    free(d->view_w);
    free(d->view_wtype);
    free(d->host_logits);
    free(d);
}

vbs_decode_t *vbs_decode_create(const vbs_backend_ops_t *ops, const vbs_decode_model_t *m,
                                char *err, size_t cap) {
    if (!ops || !m || !ops->get_device_count || ops->get_device_count() < 1) {
        snprintf(err, cap, "backend has no device (was init() called?)");
        return NULL;
    }
    vbs_decode_t *d = (vbs_decode_t *)calloc(1, sizeof(*d));
    if (!d) return NULL;
    d->ops = ops;
    d->dev = ops->get_device(0);
    d->m = *m;
    uint32_t H = m->hidden, F = m->ffn, qd = m->n_heads * m->head_dim;
    uint32_t kvd = m->n_kv_heads * m->head_dim;
    /* Runtime buffers, sized as src/vbs_engine.c:84-164 sizes them. */
    size_t sc_elems[SC_COUNT] = {qd, kvd, kvd, qd, F, F, F, H, qd, kvd};
    d->stream = ops->alloc_buffer(d->dev, (size_t)H * 4, false);
    d->tmp = ops->alloc_buffer(d->dev, (size_t)H * 4, false);
    d->logits = ops->alloc_buffer(d->dev, (size_t)m->vocab * 4, false);
    size_t kv_bytes = (size_t)m->n_layers * m->max_ctx * kvd * 2;
    d->kc = ops->alloc_buffer(d->dev, kv_bytes, false);
    d->vc = ops->alloc_buffer(d->dev, kv_bytes, false);
    int ok = d->stream && d->tmp && d->logits && d->kc && d->vc;
    for (int i = 0; ok && i < SC_COUNT; i++) {
        d->scratch[i] = ops->alloc_buffer(d->dev, sc_elems[i] * 4, false);
        ok = d->scratch[i] != NULL;
    }
    d->host_logits = (float *)malloc((size_t)m->vocab * 4);
    if (!ok || !d->host_logits) {
        snprintf(err, cap, "runtime buffer allocation failed");
        vbs_decode_destroy(d);
        return NULL;
    }
    d->attn_norm = (vbs_buffer_t **)calloc(m->n_layers, sizeof(void *));
    d->ffn_norm = (vbs_buffer_t **)calloc(m->n_layers, sizeof(void *));
    d->w = (vbs_buffer_t **)calloc((size_t)m->n_layers * 7, sizeof(void *));
    if (!d->attn_norm || !d->ffn_norm || !d->w) {
        vbs_decode_destroy(d);
        return NULL;
    }
    d->tok_embd = upload(d, m->tok_embd, row_bytes(m->embd_type, H) * m->vocab, err, cap, "token_embd");
    d->out_norm = d->tok_embd ? upload(d, m->out_norm, (size_t)H * 4, err, cap, "output_norm") : NULL;
    d->lm_head = d->out_norm ? upload(d, m->lm_head, row_bytes(m->head_type, H) * m->vocab, err, cap, "output") : NULL;
    ok = d->lm_head != NULL;
    for (uint32_t L = 0; ok && L < m->n_layers; L++) {
        d->attn_norm[L] = upload(d, m->attn_norm[L], (size_t)H * 4, err, cap, "attn_norm");
        d->ffn_norm[L] = d->attn_norm[L] ? upload(d, m->ffn_norm[L], (size_t)H * 4, err, cap, "ffn_norm") : NULL;
        ok = d->ffn_norm[L] != NULL;
        for (int k = 0; ok && k < 7; k++) {
            uint32_t r, c;
            mat_shape(m, k, &r, &c);
            uint64_t bytes = row_bytes(m->wtype[7 * L + k], c) * r;
            if (!bytes) {
                snprintf(err, cap, "layer %u matrix %d: unsupported type %d", L, k, m->wtype[7 * L + k]);
                ok = 0;
                break;
            }
            d->w[7 * L + k] = upload(d, m->wdata[7 * L + k], bytes, err, cap, "layer weight");
            ok = d->w[7 * L + k] != NULL;
        }
    }
    if (!ok) {
        vbs_decode_destroy(d);
        return NULL;
    }
    d->ok = 1;
    return d;
}

uint64_t vbs_decode_weight_bytes(const vbs_decode_t *d) { return d ? d->weight_bytes : 0; }
uint32_t vbs_decode_dispatch_count(const vbs_decode_t *d) { return d ? d->dispatches : 0; }

static int kv_xfer(vbs_decode_t *d, uint16_t *kc, uint16_t *vc, uint32_t n_pos, int to_dev) {
    const vbs_decode_model_t *m = &d->m;
    if (n_pos > m->max_ctx) return 0;
    size_t kvd = (size_t)m->n_kv_heads * m->head_dim;
    size_t lbytes = (size_t)m->max_ctx * kvd * 2, nbytes = (size_t)n_pos * kvd * 2;
    for (uint32_t L = 0; L < m->n_layers; L++) {
        for (int which = 0; which < 2; which++) {
            vbs_buffer_t *b = which ? d->vc : d->kc;
            uint16_t *h = (which ? vc : kc) + (size_t)L * n_pos * kvd;
            /* A sub-range view; on a host-memory backend (host_ptr ==
             * internal_handle, src/vbs_backend_cpu.c:78-79) it is both. */
            uint8_t *at = (uint8_t *)b->internal_handle + L * lbytes;
            vbs_buffer_t view = {at, b->host_ptr == b->internal_handle ? at : NULL, nbytes, d->dev};
            int ok = to_dev ? d->ops->copy_to_device(&view, h, nbytes)
                            : d->ops->copy_to_host(h, &view, nbytes);
            if (!ok) return 0;
        }
    }
    return 1;
}

int vbs_decode_load_kv(vbs_decode_t *d, const uint16_t *kc, const uint16_t *vc, uint32_t n_pos) {
    return d && kv_xfer(d, (uint16_t *)kc, (uint16_t *)vc, n_pos, 1);
}

int vbs_decode_read_kv(vbs_decode_t *d, uint16_t *kc, uint16_t *vc, uint32_t n_pos) {
    return d && kv_xfer(d, kc, vc, n_pos, 0);
}

/* ---- bridge-equivalent dispatch helpers ---------------------------------- */

static void *lin_pipe(vbs_decode_t *d, int type) {
    if ((unsigned)type >= 64) return NULL;
    if (!d->lin_pipe[type]) {
        char e[256];
        d->lin_pipe[type] = d->ops->compile_linear_pipeline(d->dev, (vbs_ggml_type_t)type, e, sizeof(e));
    }
    return d->lin_pipe[type];
}

static void *emb_pipe(vbs_decode_t *d, int type) {
    if ((unsigned)type >= 64) return NULL;
    if (!d->embed_pipe[type]) {
        char e[256];
        d->embed_pipe[type] = d->ops->compile_embed_pipeline(d->dev, (vbs_ggml_type_t)type, e, sizeof(e));
    }
    return d->embed_pipe[type];
}

static void *prim(vbs_decode_t *d, vbs_op_kind_t k) {
    if (!d->prim_pipe[k]) {
        char e[256];
        d->prim_pipe[k] = d->ops->compile_primitive_pipeline(d->dev, k, e, sizeof(e));
    }
    return d->prim_pipe[k];
}

static vbs_arg_t ab(const void *h) { vbs_arg_t a = {VBS_ARG_BUFFER, h, 0}; return a; }
static vbs_arg_t au(const uint32_t *v) { vbs_arg_t a = {VBS_ARG_SCALAR, v, 4}; return a; }
static vbs_arg_t af(const float *v) { vbs_arg_t a = {VBS_ARG_SCALAR, v, 4}; return a; }
#define H_(b) ((b)->internal_handle)

/* src/vbs_specializer_bridge.c:83-90 */
static void linear(vbs_decode_t *d, int type, vbs_buffer_t *w, vbs_buffer_t *in, vbs_buffer_t *out,
                   uint32_t rows, uint32_t cols) {
    void *p = lin_pipe(d, type);
    d->dispatches++;
    if (!p || !d->ops->dispatch_linear_tile(d->dev, p, w, NULL, 0, in, out, cols, rows, 0, 0, false))
        d->ok = 0;
}

static void primitive(vbs_decode_t *d, vbs_op_kind_t k, void *pipe, const vbs_arg_t *a, size_t n,
                      size_t grid, size_t block) {
    d->dispatches++;
    if (!pipe || !d->ops->dispatch_primitive(d->dev, pipe, a, n, grid, block)) d->ok = 0;
    (void)k;
}

int vbs_decode_step(vbs_decode_t *d, uint32_t token, uint32_t pos, float *logits) {
    if (!d) return 0;
    const vbs_decode_model_t *m = &d->m;
    if (token >= m->vocab || pos >= m->max_ctx) return 0;
    d->ok = 1;
    d->dispatches = 0;
    uint32_t H = m->hidden, F = m->ffn, hd = m->head_dim, nq = m->n_heads, nkv = m->n_kv_heads;
    uint32_t qd = nq * hd, kvd = nkv * hd, maxc = m->max_ctx, V = m->vocab;
    float eps = m->rms_eps, theta = m->rope_theta, scale = 1.0f / sqrtf((float)hd);
    uint32_t seq = pos + 1;
    vbs_buffer_t *S = d->stream, *T = d->tmp, **sc = d->scratch;

    { /* embed: B w, S token, B out, S dim (bridge.c:130-146) */
        vbs_arg_t a[] = {ab(H_(d->tok_embd)), au(&token), ab(H_(S)), au(&H)};
        primitive(d, VBS_OP_EMBEDDING, emb_pipe(d, m->embd_type), a, 4, (H + 255) / 256, 256);
    }
    for (uint32_t L = 0; L < m->n_layers; L++) {
        vbs_buffer_t **w = d->w + 7 * L;
        const int *t = m->wtype + 7 * L;
        uint32_t layer = L;
        { /* norm: B in, B w, B out, S dim, S eps (bridge.c:148-155) */
            vbs_arg_t a[] = {ab(H_(S)), ab(H_(d->attn_norm[L])), ab(H_(sc[SC_NORMED])), au(&H), af(&eps)};
            primitive(d, VBS_OP_NORMALIZE, prim(d, VBS_OP_NORMALIZE), a, 5, (H + 255) / 256, 256);
        }
        linear(d, t[0], w[0], sc[SC_NORMED], sc[SC_Q], qd, H);
        { /* rope: B x, S pos, S hd, S nh, S theta (bridge.c:157-165) */
            vbs_arg_t a[] = {ab(H_(sc[SC_Q])), au(&pos), au(&hd), au(&nq), af(&theta)};
            primitive(d, VBS_OP_ROTARY, prim(d, VBS_OP_ROTARY), a, 5, ((hd / 2) * nq + 255) / 256, 256);
        }
        linear(d, t[1], w[1], sc[SC_NORMED], sc[SC_K], kvd, H);
        {
            vbs_arg_t a[] = {ab(H_(sc[SC_K])), au(&pos), au(&hd), au(&nkv), af(&theta)};
            primitive(d, VBS_OP_ROTARY, prim(d, VBS_OP_ROTARY), a, 5, ((hd / 2) * nkv + 255) / 256, 256);
        }
        linear(d, t[2], w[2], sc[SC_NORMED], sc[SC_V], kvd, H);
        { /* cache: B k, B v, B kc, B vc, S pos, S layer, S max_ctx, S kv_dim (bridge.c:167-173) */
            vbs_arg_t a[] = {ab(H_(sc[SC_K])), ab(H_(sc[SC_V])), ab(H_(d->kc)), ab(H_(d->vc)),
                             au(&pos), au(&layer), au(&maxc), au(&kvd)};
            primitive(d, VBS_OP_CACHE, prim(d, VBS_OP_CACHE), a, 8, (kvd + 255) / 256, 256);
        }
        { /* attn (bridge.c:175-183): seq_len = pos + 1, scale = 1/sqrtf(hd) */
            vbs_arg_t a[] = {ab(H_(sc[SC_Q])), ab(H_(d->kc)), ab(H_(d->vc)), ab(H_(sc[SC_ATTN])),
                             au(&seq), au(&layer), au(&maxc), au(&nq), au(&nkv), au(&hd), af(&scale)};
            primitive(d, VBS_OP_ATTENTION, prim(d, VBS_OP_ATTENTION), a, 11, nq, hd > 32 ? hd : 32);
        }
        linear(d, t[3], w[3], sc[SC_ATTN], T, H, qd);
        { /* add: B a, B b, B out, S n (bridge.c:193-199), STREAM += TMP */
            vbs_arg_t a[] = {ab(H_(S)), ab(H_(T)), ab(H_(S)), au(&H)};
            primitive(d, VBS_OP_ELEMENTWISE, prim(d, VBS_OP_ELEMENTWISE), a, 4, (H + 255) / 256, 256);
        }
        {
            vbs_arg_t a[] = {ab(H_(S)), ab(H_(d->ffn_norm[L])), ab(H_(sc[SC_NORMED])), au(&H), af(&eps)};
            primitive(d, VBS_OP_NORMALIZE, prim(d, VBS_OP_NORMALIZE), a, 5, (H + 255) / 256, 256);
        }
        linear(d, t[4], w[4], sc[SC_NORMED], sc[SC_GATE], F, H);
        linear(d, t[5], w[5], sc[SC_NORMED], sc[SC_UP], F, H);
        { /* silu: B gate, B up, B out, S n (bridge.c:185-191) */
            vbs_arg_t a[] = {ab(H_(sc[SC_GATE])), ab(H_(sc[SC_UP])), ab(H_(sc[SC_HIDDEN])), au(&F)};
            primitive(d, VBS_OP_ACTIVATION, prim(d, VBS_OP_ACTIVATION), a, 4, (F + 255) / 256, 256);
        }
        linear(d, t[6], w[6], sc[SC_HIDDEN], T, H, F);
        {
            vbs_arg_t a[] = {ab(H_(S)), ab(H_(T)), ab(H_(S)), au(&H)};
            primitive(d, VBS_OP_ELEMENTWISE, prim(d, VBS_OP_ELEMENTWISE), a, 4, (H + 255) / 256, 256);
        }
    }
    {
        vbs_arg_t a[] = {ab(H_(S)), ab(H_(d->out_norm)), ab(H_(sc[SC_NORMED])), au(&H), af(&eps)};
        primitive(d, VBS_OP_NORMALIZE, prim(d, VBS_OP_NORMALIZE), a, 5, (H + 255) / 256, 256);
    }
    linear(d, m->head_type, d->lm_head, sc[SC_NORMED], d->logits, V, H);
    if (logits && d->ok) {
        /* vbs_gpu_readback_logits (bridge.c:201-206): copy_to_host, no sync first */
        vbs_buffer_t view = {H_(d->logits), NULL, (size_t)V * 4, d->dev};
        if (!d->ops->copy_to_host(logits, &view, (size_t)V * 4)) d->ok = 0;
    }
    return d->ok;
}

int vbs_decode_greedy(vbs_decode_t *d, uint32_t token, uint32_t pos, uint32_t n,
                      uint32_t *tokens_out, float *margins_out) {
    if (!d) return 0;
    for (uint32_t i = 0; i < n; i++) {
        if (!vbs_decode_step(d, token, pos + i, d->host_logits)) return 0;
        uint32_t best = 0;
        float bv = d->host_logits[0], second = -INFINITY;
        for (uint32_t v = 1; v < d->m.vocab; v++) { /* strict '>' keeps the first max */
            float x = d->host_logits[v];
            if (x > bv) { second = bv; bv = x; best = v; }
            else if (x > second) second = x;
        }
        tokens_out[i] = best;
        if (margins_out) margins_out[i] = bv - second;
        token = best;
    }
    return 1;
}

int vbs_decode_device_model(vbs_decode_t *d, void *out) {
    if (!d || !out) return 0;
    vbs_gfx950_model_t *v = (vbs_gfx950_model_t *)out;
    const vbs_decode_model_t *m = &d->m;
    uint32_t L = m->n_layers;
    if (!d->view_w) {
        d->view_attn_norm = (const float **)calloc(L, sizeof(void *));
        d->view_ffn_norm = (const float **)calloc(L, sizeof(void *));
        d->view_w = (const void **)calloc((size_t)7 * L, sizeof(void *));
        d->view_wtype = (int *)calloc((size_t)7 * L, sizeof(int));
        if (!d->view_attn_norm || !d->view_ffn_norm || !d->view_w || !d->view_wtype) return 0;
        for (uint32_t i = 0; i < L; i++) {
            d->view_attn_norm[i] = (const float *)d->attn_norm[i]->internal_handle;
            d->view_ffn_norm[i] = (const float *)d->ffn_norm[i]->internal_handle;
        }
        for (uint32_t i = 0; i < 7 * L; i++) {
            d->view_w[i] = d->w[i]->internal_handle;
            d->view_wtype[i] = m->wtype[i];
        }
    }
    memset(v, 0, sizeof(*v));
    v->n_layers = L;
    v->hidden = m->hidden;
    v->ffn = m->ffn;
    v->n_heads = m->n_heads;
    v->n_kv_heads = m->n_kv_heads;
    v->head_dim = m->head_dim;
    v->vocab = m->vocab;
    v->max_ctx = m->max_ctx;
    v->rope_theta = m->rope_theta;
    v->rms_eps = m->rms_eps;
    v->embd_type = m->embd_type;
    v->tok_embd = d->tok_embd->internal_handle;
    v->out_norm = (const float *)d->out_norm->internal_handle;
    v->head_type = m->head_type;
    v->lm_head = d->lm_head->internal_handle;
    v->attn_norm = d->view_attn_norm;
    v->ffn_norm = d->view_ffn_norm;
    v->wtype = d->view_wtype;
    v->wdata = d->view_w;
    v->kc = (uint16_t *)d->kc->internal_handle;
    v->vc = (uint16_t *)d->vc->internal_handle;
    return 1;
}
