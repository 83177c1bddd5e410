// vbs_decoder.hip — one decode token as a replayable HIP graph.
//
// The step is the specializer's forward_token (src/vbs_specializer.c:270-349)
// with the bridge's scalars (src/vbs_specializer_bridge.c:148-183): embed ->
// per layer [attn_norm, Q, rope(Q), K, rope(K), V, cache, attention, O, add,
// ffn_norm, gate, up, silu, down, add] -> output_norm -> lm_head, followed by
// a greedy argmax. Neighbouring ops run as one launch where the matrix-core
// matvec can carry them (same arithmetic, one kernel): attn_norm + Q/K/V +
// RoPE + cache store; O + residual add; ffn_norm + gate/up + SiLU*up; down +
// residual add; output_norm + lm_head: six launches per layer with attention's
// two. At the 7B shape (Q4_K O over 32 heads of 128) the attention merge
// moves into the O launch (k_mvl_attn): five. Other weight types run the
// per-op kernels of the C ABI. The
// position-dependent kernels read the position from device memory, so one
// captured graph serves every token:
//   * RoPE reads cos/sin of each pair from a [max_ctx][head_dim/2] table that
//     the host fills with the reference's own expressions and libm;
//   * the KV store and attention compute their offsets / sequence length from
//     the device position;
//   * the argmax kernel writes the next token, records it, advances the
//     position and gathers the next token's embedding into the residual
//     stream, so the graph starts at the first layer (the host gathers the
//     first token's embedding before the first replay).
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "vbs_dev_common.h"
#include "vbs_gfx950.h"
#include "vbs_internal.h"
#include "vbs_lds_dma.h"

namespace vbs {

// ---- position-dependent kernels ---------------------------------------------

__global__ __launch_bounds__(256) void k_rope_table(float *__restrict__ x,
                                                    const uint32_t *__restrict__ pos_dev,
                                                    const float2 *__restrict__ tab, uint32_t hd,
                                                    uint32_t nh) {
    const uint32_t pairs = hd / 2u;
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= pairs * nh) return;
    const uint32_t h = idx / pairs, p = idx % pairs;
    const float2 cs = tab[(uint64_t)pos_dev[0] * pairs + p];
    float *v = x + (uint64_t)h * hd + 2u * p;
    const float x0 = v[0], x1 = v[1];
    v[0] = __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y));
    v[1] = __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
}

__global__ __launch_bounds__(256) void k_cache_store_pos(const float *__restrict__ k,
                                                         const float *__restrict__ v,
                                                         uint16_t *__restrict__ kc,
                                                         uint16_t *__restrict__ vc,
                                                         const uint32_t *__restrict__ pos_dev,
                                                         uint32_t layer, uint32_t max_ctx,
                                                         uint32_t kv_dim) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= kv_dim) return;
    const uint64_t base = ((uint64_t)layer * max_ctx + pos_dev[0]) * kv_dim;
    kc[base + i] = vbs_f2h(k[i]);
    vc[base + i] = vbs_f2h(v[i]);
}

// Greedy pick: the first index of the maximum (strict '>' scan order, as
// main.c:929-932), and the runner-up value for the margin report. Writes the
// token for the next replay, records it at tokens[step], advances pos and step.
struct Top2 {
    float v1;
    uint32_t i1;
    float v2;
};

__device__ __forceinline__ Top2 top2_merge(Top2 a, Top2 b) {
    // Symmetric in a and b (any reduction tree gives the same result): the
    // larger value wins, the lower index on ties, so the first maximum wins;
    // a NaN can only sit at index 0 (the scan never takes one elsewhere), and
    // there it wins, as the reference's strict '>' scan from index 0 keeps it.
    const bool a_nan = a.v1 != a.v1, b_nan = b.v1 != b.v1;
    const bool b_wins = b_nan || (!a_nan && (b.v1 > a.v1 || (b.v1 == a.v1 && b.i1 < a.i1)));
    Top2 r;
    r.v1 = b_wins ? b.v1 : a.v1;
    r.i1 = b_wins ? b.i1 : a.i1;
    const float loser = b_wins ? a.v1 : b.v1;
    r.v2 = fmaxf(loser, fmaxf(a.v2, b.v2));
    return r;
}

// One workgroup per sequence b of a batch (gridDim.x sequences): logits row b,
// state token_dev[b], pos_dev[b], step_dev[b], outputs tokens[step * nb + b].
// It then writes the next step's input, row `token` of the embedding table
// (type T, src/vbs_host_math.h:94-142, as k_dequant_rows computes it), to
// x + b * dim: the gather that would otherwise open the next step's graph.
constexpr uint32_t kArgVec = 8, kArgScalar = 16;  // loads per thread in flight per pass

template <int T>
__global__ __launch_bounds__(1024) void k_argmax_advance(const float *__restrict__ logits,
                                                         uint32_t n, uint32_t *token_dev,
                                                         uint32_t *pos_dev, uint32_t *step_dev,
                                                         uint32_t *tokens, float *margins,
                                                         uint32_t max_steps,
                                                         const uint8_t *__restrict__ embd,
                                                         uint64_t embd_rb, uint32_t dim,
                                                         float *__restrict__ x) {
    __shared__ Top2 red[16];
    const uint32_t sb = blockIdx.x, nb = gridDim.x;
    logits += (uint64_t)sb * n;
    token_dev += sb;
    pos_dev += sb;
    step_dev += sb;
    x += (uint64_t)sb * dim;
    Top2 t{-INFINITY, 0xFFFFFFFFu, -INFINITY};
    auto consider = [&](float v, uint32_t i) {
        if (v != v && i != 0u) return;  // a NaN never beats anything after index 0
        if (t.i1 == 0xFFFFFFFFu || v > t.v1) {
            if (t.i1 != 0xFFFFFFFFu) t.v2 = fmaxf(t.v2, t.v1);
            t.v1 = v;
            t.i1 = i;
        } else {
            t.v2 = fmaxf(t.v2, v);
        }
    };
    // each thread scans its indices in increasing order: 16-byte chunks
    // c, c + 1024, ... when the logits allow it, single floats otherwise; a
    // pass requests all of its loads before it looks at any value
    if ((n % 4u) == 0 && ((uintptr_t)logits & 15u) == 0) {
        const float4 *l4 = reinterpret_cast<const float4 *>(logits);
        const uint32_t n4 = n / 4u;
        for (uint32_t c0 = threadIdx.x; c0 < n4; c0 += 1024u * kArgVec) {
            float4 f[kArgVec];
#pragma unroll
            for (uint32_t k = 0; k < kArgVec; k++) {
                const uint32_t c = c0 + 1024u * k;
                f[k] = c < n4 ? l4[c] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (uint32_t k = 0; k < kArgVec; k++) {
                const uint32_t c = c0 + 1024u * k;
                if (c < n4) {
                    consider(f[k].x, 4u * c);
                    consider(f[k].y, 4u * c + 1u);
                    consider(f[k].z, 4u * c + 2u);
                    consider(f[k].w, 4u * c + 3u);
                }
            }
        }
    } else {
        for (uint32_t i0 = threadIdx.x; i0 < n; i0 += 1024u * kArgScalar) {
            float f[kArgScalar];
#pragma unroll
            for (uint32_t k = 0; k < kArgScalar; k++) {
                const uint32_t i = i0 + 1024u * k;
                f[k] = i < n ? logits[i] : 0.f;
            }
#pragma unroll
            for (uint32_t k = 0; k < kArgScalar; k++) {
                const uint32_t i = i0 + 1024u * k;
                if (i < n) consider(f[k], i);
            }
        }
    }
    // wave butterflies, then the 16 wave results in one wave
    auto wave_merge = [](Top2 v, uint32_t width) {
        for (uint32_t off = width / 2u; off > 0; off >>= 1) {
            Top2 o;
            o.v1 = __shfl_xor(v.v1, (int)off, 64);
            o.i1 = (uint32_t)__shfl_xor((int)v.i1, (int)off, 64);
            o.v2 = __shfl_xor(v.v2, (int)off, 64);
            v = top2_merge(v, o);
        }
        return v;
    };
    t = wave_merge(t, 64u);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = t;
    __syncthreads();
    if (wave == 0) {
        Top2 w = lane < 16u ? red[lane] : Top2{-INFINITY, 0xFFFFFFFFu, -INFINITY};
        w = wave_merge(w, 16u);
        if (lane == 0) red[0] = w;
    }
    __syncthreads();
    const uint32_t tok = red[0].i1;
    if (threadIdx.x == 0) {
        const uint32_t step = step_dev[0];
        if (step < max_steps) {
            tokens[step * nb + sb] = tok;
            margins[step * nb + sb] = red[0].v1 - red[0].v2;
        }
        token_dev[0] = tok;
        pos_dev[0] = pos_dev[0] + 1u;
        step_dev[0] = step + 1u;
    }
    if (tok < n) {  // (always: index 0 is taken even when every logit is NaN)
        const uint8_t *row = embd + (uint64_t)tok * embd_rb;
        for (uint32_t e = threadIdx.x; e < dim; e += 1024u)
            x[e] = deq_elem<T>(row + (uint64_t)(e / Geo<T>::E) * Geo<T>::B, e % Geo<T>::E);
    }
}

// The argmax of `nb` logit rows of n (the vocabulary) and, for each, the
// embedding of the chosen token into x + b * dim (table of type `type`).
static hipError_t launch_argmax_embed(int type, const float *logits, uint32_t n, uint32_t nb,
                                      uint32_t *token_dev, uint32_t *pos_dev, uint32_t *step_dev,
                                      uint32_t *tokens, float *margins, uint32_t max_steps,
                                      const void *embd, uint32_t dim, float *x, hipStream_t s) {
    const uint64_t rb = row_bytes(type, dim);
    const uint8_t *e = (const uint8_t *)embd;
#define VBS_ARGMAX(TT)                                                                             \
    k_argmax_advance<TT><<<nb, 1024, 0, s>>>(logits, n, token_dev, pos_dev, step_dev, tokens,      \
                                             margins, max_steps, e, rb, dim, x)
    switch (type) {
        case kF32: VBS_ARGMAX(kF32); break;
        case kF16: VBS_ARGMAX(kF16); break;
        case kQ4_0: VBS_ARGMAX(kQ4_0); break;
        case kQ4_1: VBS_ARGMAX(kQ4_1); break;
        case kQ8_0: VBS_ARGMAX(kQ8_0); break;
        case kQ4_K: VBS_ARGMAX(kQ4_K); break;
        case kQ6_K: VBS_ARGMAX(kQ6_K); break;
        case kLNS8: VBS_ARGMAX(kLNS8); break;
        default: return hipErrorInvalidValue;
    }
#undef VBS_ARGMAX
    return hipGetLastError();
}

// ---- decoder -------------------------------------------------------------------

struct Decoder {
    vbs_gfx950_model_t m;
    std::vector<const float *> attn_norm, ffn_norm;
    std::vector<int> wtype;
    std::vector<const void *> wdata;
    float *stream = nullptr, *tmp, *normed, *q, *k, *v, *attn, *gate, *up, *hid, *logits;
    uint32_t *state = nullptr;  // [token, pos, step]
    uint32_t *tokens = nullptr;
    float *margins = nullptr;
    float *part = nullptr;
    float2 *rope = nullptr;
    // attention merged inside the O launch (attn_o_fits): the XCDs' copies of
    // the merged vector, their flags, the count of workgroups that merged
    // every head themselves, and the bound on each workgroup's wait
    float *mbuf = nullptr;
    uint32_t *mflag = nullptr, *fallbacks = nullptr;
    uint32_t ao_spin = 0;
    uint32_t max_steps = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    void *arena = nullptr;
};

// Polls of a workgroup's bounded wait for its XCD's merged heads in the O launch:
// a poll is an L2 round trip and a short sleep, so the bound is ~1 ms, far
// past the few microseconds the other workgroups take to publish.
constexpr uint32_t kAttnOSpin = 2048;

// The O launch takes the attention merge (launch_q4k_mvl_attn) when every
// layer's O is Q4_K of the 7B shape: q dimension 4096 (32 heads of 128, 16
// blocks), at most 16 rows per each of the 256 workgroups, group <= 8, the
// weights and caches 16-byte aligned -- and when the device has a CU for each
// of those workgroups (one fits a CU), so that they all run at once: a
// workgroup's wait for the others' heads is bounded, but on fewer CUs it
// would run out in every launch.
static bool attn_o_fits(const vbs_gfx950_model_t &m) {
    const uint32_t qd = m.n_heads * m.head_dim, wgs = 8u * m.n_heads;
    if (device_cus() < wgs) return false;
    if (m.head_dim != 128u || qd != 4096u || m.n_kv_heads == 0 || m.n_heads % m.n_kv_heads ||
        m.n_heads / m.n_kv_heads > 8u || (m.hidden + wgs - 1u) / wgs > 16u ||
        ((uintptr_t)m.kc & 15u) || ((uintptr_t)m.vc & 15u))
        return false;
    for (uint32_t L = 0; L < m.n_layers; L++)
        if (m.wtype[7 * L + 3] != kQ4_K || ((uintptr_t)m.wdata[7 * L + 3] & 15u)) return false;
    return true;
}

static hipError_t enqueue_step(const Decoder &d, hipStream_t s) {
    const vbs_gfx950_model_t &m = d.m;
    const uint32_t H = m.hidden, F = m.ffn, hd = m.head_dim, nq = m.n_heads, nkv = m.n_kv_heads;
    const uint32_t qd = nq * hd, kvd = nkv * hd;
    const float scale = 1.0f / sqrtf((float)hd);
    uint32_t *token_dev = d.state, *pos_dev = d.state + 1, *step_dev = d.state + 2;
    const uint32_t pairs = hd / 2u;
#define VBS_TRY(expr)                     \
    do {                                  \
        hipError_t e_ = (expr);           \
        if (e_ != hipSuccess) return e_;  \
    } while (0)
    // the stream holds the token's embedding already (written by the previous
    // step's argmax, or by decoder_start for the first step)
    for (uint32_t L = 0; L < m.n_layers; L++) {
        const int *t = d.wtype.data() + 7 * L;
        const uint8_t *const *w = (const uint8_t *const *)d.wdata.data() + 7 * L;
        const uint64_t layer_off = (uint64_t)L * m.max_ctx * kvd;
        // attn_norm, Q, K, V, RoPE and the cache store: one matrix-core launch
        // when q, k and v share a K-quant type
        hipError_t e = hipErrorNotSupported;
        if (t[0] == t[1] && t[1] == t[2]) {
            const uint32_t rows[3] = {qd, kvd, kvd};
            e = launch_kq_qkv(t[0], w, 3, 0, d.stream, d.attn_norm[L], m.rms_eps, H, rows, d.q,
                              m.kc, m.vc, layer_off, kvd, d.rope, pos_dev, hd, s);
        }
        if (e == hipErrorNotSupported) {
            VBS_TRY(launch_rms_norm(d.stream, d.attn_norm[L], d.normed, H, m.rms_eps, s));
            VBS_TRY(launch_linear(t[0], w[0], d.normed, d.q, H, qd, 0, s));
            k_rope_table<<<(pairs * nq + 255u) / 256u, 256, 0, s>>>(d.q, pos_dev, d.rope, hd, nq);
            VBS_TRY(hipGetLastError());
            VBS_TRY(launch_linear(t[1], w[1], d.normed, d.k, H, kvd, 0, s));
            k_rope_table<<<(pairs * nkv + 255u) / 256u, 256, 0, s>>>(d.k, pos_dev, d.rope, hd, nkv);
            VBS_TRY(hipGetLastError());
            VBS_TRY(launch_linear(t[2], w[2], d.normed, d.v, H, kvd, 0, s));
            k_cache_store_pos<<<(kvd + 255u) / 256u, 256, 0, s>>>(d.k, d.v, m.kc, m.vc, pos_dev,
                                                                    L, m.max_ctx, kvd);
            VBS_TRY(hipGetLastError());
        } else {
            VBS_TRY(e);
        }
        if (d.mbuf) {
            // attention chunks, then O with the merge in front and the residual
            // add folded in: two launches, the results of the three below
            VBS_TRY(launch_attention_chunks(d.q, m.kc, m.vc, m.max_ctx, pos_dev, d.part, layer_off, nq,
                                            nkv, hd, scale, d.mflag, attn_o_flags(qd), kAttnOFlagStride, s));
            AttnOArgs ao{};
            ao.w = w[3];
            ao.y = d.stream;
            ao.rows = H;
            ao.cols = qd;
            ao.rpw = (H + 8u * nq - 1u) / (8u * nq);
            ao.part = d.part;
            ao.stride_chunks = attention_chunk_stride(m.max_ctx, nkv);
            ao.nkh = nkv;
            ao.pos = pos_dev;
            ao.attn = nullptr;  // (nothing in the step reads the merged vector itself)
            ao.mbuf = d.mbuf;
            ao.mflag = d.mflag;
            ao.spin = d.ao_spin;
            ao.fallbacks = d.fallbacks;
            VBS_TRY(launch_q4k_mvl_attn(ao, s));
            e = hipSuccess;
        } else {
            VBS_TRY(launch_attention(d.q, m.kc, m.vc, d.attn, m.max_ctx, pos_dev, d.part, layer_off,
                                     nq, nkv, hd, scale, s));
            // O with the residual add folded in (stream + O*attn, as the add computes it)
            e = launch_kq_linear(t[3], w[3], d.attn, d.stream, qd, H, 1, s);
        }
        if (e == hipErrorNotSupported) {
            VBS_TRY(launch_linear(t[3], w[3], d.attn, d.tmp, qd, H, 0, s));
            VBS_TRY(launch_add(d.stream, d.tmp, d.stream, H, s));
        } else {
            VBS_TRY(e);
        }
        // ffn_norm, gate, up and SiLU*up: one launch when gate and up share a type
        e = t[4] == t[5] ? launch_kq_silu(t[4], w[4], w[5], d.stream, d.ffn_norm[L], m.rms_eps, H,
                                          F, d.hid, s)
                         : hipErrorNotSupported;
        if (e == hipErrorNotSupported) {
            VBS_TRY(launch_rms_norm(d.stream, d.ffn_norm[L], d.normed, H, m.rms_eps, s));
            VBS_TRY(launch_linear(t[4], w[4], d.normed, d.gate, H, F, 0, s));
            VBS_TRY(launch_linear(t[5], w[5], d.normed, d.up, H, F, 0, s));
            VBS_TRY(launch_silu_mul(d.gate, d.up, d.hid, F, s));
        } else {
            VBS_TRY(e);
        }
        // down with the residual add folded in
        e = launch_kq_linear(t[6], w[6], d.hid, d.stream, F, H, 1, s);
        if (e == hipErrorNotSupported) {
            VBS_TRY(launch_linear(t[6], w[6], d.hid, d.tmp, F, H, 0, s));
            VBS_TRY(launch_add(d.stream, d.tmp, d.stream, H, s));
        } else {
            VBS_TRY(e);
        }
    }
    // output_norm and lm_head
    hipError_t e = launch_kq_norm_linear(m.head_type, (const uint8_t *)m.lm_head, d.stream,
                                         m.out_norm, m.rms_eps, d.logits, H, m.vocab, s);
    if (e == hipErrorNotSupported) {
        VBS_TRY(launch_rms_norm(d.stream, m.out_norm, d.normed, H, m.rms_eps, s));
        VBS_TRY(launch_linear(m.head_type, (const uint8_t *)m.lm_head, d.normed, d.logits, H,
                              m.vocab, 0, s));
    } else {
        VBS_TRY(e);
    }
    VBS_TRY(launch_argmax_embed(m.embd_type, d.logits, m.vocab, 1, token_dev, pos_dev, step_dev,
                                d.tokens, d.margins, d.max_steps, m.tok_embd, H, d.stream, s));
#undef VBS_TRY
    return hipSuccess;
}

static void decoder_free(Decoder *d) {
    if (!d) return;
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    if (d->arena) {
        (void)hipStreamSynchronize(rt_stream());
        (void)hipFree(d->arena);
    }
    delete d;
}

}  // namespace vbs

using namespace vbs;

extern "C" {

int vbs_gfx950_decoder_create(const vbs_gfx950_model_t *m, uint32_t max_steps, void **handle) {
    if (!rt_ready()) return 0;
    if (!m || !handle) return rt_fail("decoder_create: null argument");
    *handle = nullptr;
    if (!m->n_layers || !m->hidden || !m->ffn || !m->n_heads || !m->n_kv_heads || !m->head_dim ||
        !m->vocab || !m->max_ctx)
        return rt_fail("decoder_create: empty model dimension");
    if (m->n_heads % m->n_kv_heads || m->n_heads / m->n_kv_heads > 16 || m->head_dim > 256 ||
        (m->head_dim & 1u))
        return rt_fail("decoder_create: unsupported head geometry");
    if (!m->tok_embd || !m->out_norm || !m->lm_head || !m->attn_norm || !m->ffn_norm ||
        !m->wtype || !m->wdata || !m->kc || !m->vc)
        return rt_fail("decoder_create: null model pointer");
    if (!block_elems(m->embd_type) || !block_elems(m->head_type))
        return rt_fail("decoder_create: unsupported embedding/head type");
    for (uint32_t i = 0; i < 7 * m->n_layers; i++) {
        if (!block_elems(m->wtype[i]) || !m->wdata[i])
            return rt_fail("decoder_create: layer %u matrix %u unsupported or null", i / 7, i % 7);
    }
    Decoder *d = new Decoder();
    d->m = *m;
    d->attn_norm.assign(m->attn_norm, m->attn_norm + m->n_layers);
    d->ffn_norm.assign(m->ffn_norm, m->ffn_norm + m->n_layers);
    d->wtype.assign(m->wtype, m->wtype + 7 * m->n_layers);
    d->wdata.assign(m->wdata, m->wdata + 7 * m->n_layers);
    d->max_steps = max_steps ? max_steps : 1;
    const uint32_t H = m->hidden, F = m->ffn, qd = m->n_heads * m->head_dim;
    const uint32_t kvd = m->n_kv_heads * m->head_dim, pairs = m->head_dim / 2u;
    // one arena: activations, state, outputs, attention partials, RoPE table
    const size_t n_f32 = 3ull * H + 2ull * qd + 2ull * kvd + 3ull * F + m->vocab;
    const size_t part = attention_partial_bytes(m->max_ctx, m->n_heads, m->n_kv_heads, m->head_dim);
    const size_t rope = (size_t)m->max_ctx * pairs * sizeof(float2);
    auto up256 = [](size_t b) { return (b + 255u) & ~(size_t)255u; };
    const size_t sz_f = up256(n_f32 * 4), sz_st = 256, sz_tok = up256(d->max_steps * 4ull);
    const bool ao = attn_o_fits(*m);
    const size_t sz_ao = ao ? up256(attn_o_exchange_bytes(qd)) + 256u : 0u;
    const size_t total = sz_f + sz_st + 2 * sz_tok + up256(part) + up256(rope) + sz_ao;
    if (hipMalloc(&d->arena, total) != hipSuccess) {
        delete d;
        return rt_fail("decoder_create: hipMalloc(%zu) failed", total);
    }
    uint8_t *p = (uint8_t *)d->arena;
    float *f = (float *)p;
    d->stream = f; f += H;
    d->tmp = f; f += H;
    d->normed = f; f += H;
    d->q = f; f += qd;
    d->attn = f; f += qd;
    d->k = f; f += kvd;
    d->v = f; f += kvd;
    d->gate = f; f += F;
    d->up = f; f += F;
    d->hid = f; f += F;
    d->logits = f;
    p += sz_f;
    d->state = (uint32_t *)p; p += sz_st;
    d->tokens = (uint32_t *)p; p += sz_tok;
    d->margins = (float *)p; p += sz_tok;
    d->part = (float *)p; p += up256(part);
    d->rope = (float2 *)p; p += up256(rope);
    if (ao) {
        d->mbuf = (float *)p;
        d->mflag = (uint32_t *)(p + (size_t)kAttnOXcds * qd * sizeof(float));
        p += up256(attn_o_exchange_bytes(qd));
        d->fallbacks = (uint32_t *)p;
        const char *sp = getenv("VBS_ATTN_O_SPIN");  // (tests force the fallback with 0)
        d->ao_spin = sp ? (uint32_t)strtoul(sp, nullptr, 10) : kAttnOSpin;
    }
    // RoPE table with the reference's expressions (src/vbs_host_math.h:43-44)
    std::vector<float2> tab((size_t)m->max_ctx * pairs);
    for (uint32_t pos = 0; pos < m->max_ctx; pos++)
        for (uint32_t pr = 0; pr < pairs; pr++) {
            const uint32_t i = 2u * pr;
            const float angle = (float)pos * powf(m->rope_theta, -(float)i / (float)m->head_dim);
            tab[(size_t)pos * pairs + pr] = make_float2(cosf(angle), sinf(angle));
        }
    hipStream_t s = rt_stream();
    if (!rt_hip_ok(hipMemcpyAsync(d->rope, tab.data(), rope, hipMemcpyHostToDevice, s),
                   "decoder_create: rope table") ||
        !rt_hip_ok(hipMemsetAsync(d->state, 0, sz_st, s), "decoder_create: state") ||
        (ao && !rt_hip_ok(hipMemsetAsync(d->mbuf, 0, sz_ao, s), "decoder_create: exchange")) ||
        !rt_hip_ok(hipStreamSynchronize(s), "decoder_create")) {
        decoder_free(d);
        return 0;
    }
    // capture one token step
    if (!rt_hip_ok(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture")) {
        decoder_free(d);
        return 0;
    }
    hipError_t e = enqueue_step(*d, s);
    hipGraph_t g = nullptr;
    hipError_t e2 = hipStreamEndCapture(s, &g);
    if (e != hipSuccess || e2 != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        decoder_free(d);
        return rt_fail("decoder_create: capture failed (%s)",
                       hipGetErrorString(e != hipSuccess ? e : e2));
    }
    d->graph = g;
    if (!rt_hip_ok(hipGraphInstantiate(&d->exec, g, nullptr, nullptr, 0), "graph instantiate")) {
        decoder_free(d);
        return 0;
    }
    *handle = d;
    return 1;
}

static int set_state(Decoder *d, uint32_t token, uint32_t pos) {
    if (token >= d->m.vocab) return rt_fail("decoder: token %u >= vocab %u", token, d->m.vocab);
    if (pos >= d->m.max_ctx) return rt_fail("decoder: pos %u >= max_ctx %u", pos, d->m.max_ctx);
    const uint32_t st[3] = {token, pos, 0};
    hipStream_t s = rt_stream();
    return rt_hip_ok(hipMemcpyAsync(d->state, st, sizeof(st), hipMemcpyHostToDevice, s),
                     "decoder: state") &&
           rt_hip_ok(launch_dequant_rows(d->m.embd_type, (const uint8_t *)d->m.tok_embd, d->state,
                                         0, 1, d->m.hidden, d->stream, s),
                     "decoder: first embedding") &&
           rt_hip_ok(hipStreamSynchronize(s), "decoder: state");
}

int vbs_gfx950_decoder_step(void *handle, uint32_t token, uint32_t pos, float *logits) {
    if (!rt_ready()) return 0;
    Decoder *d = (Decoder *)handle;
    if (!d) return rt_fail("decoder_step: null handle");
    if (!set_state(d, token, pos)) return 0;
    hipStream_t s = rt_stream();
    if (!rt_hip_ok(hipGraphLaunch(d->exec, s), "decoder_step: graph launch")) return 0;
    if (logits &&
        !rt_hip_ok(hipMemcpyAsync(logits, d->logits, (size_t)d->m.vocab * 4, hipMemcpyDeviceToHost, s),
                   "decoder_step: logits"))
        return 0;
    return rt_hip_ok(hipStreamSynchronize(s), "decoder_step");
}

int vbs_gfx950_decoder_greedy(void *handle, uint32_t token, uint32_t pos, uint32_t n,
                              uint32_t *tokens, float *margins) {
    if (!rt_ready()) return 0;
    Decoder *d = (Decoder *)handle;
    if (!d || !tokens) return rt_fail("decoder_greedy: null argument");
    if (n > d->max_steps) return rt_fail("decoder_greedy: %u steps > max_steps %u", n, d->max_steps);
    if ((uint64_t)pos + n > d->m.max_ctx) return rt_fail("decoder_greedy: context exhausted");
    if (!set_state(d, token, pos)) return 0;
    hipStream_t s = rt_stream();
    for (uint32_t i = 0; i < n; i++)
        if (!rt_hip_ok(hipGraphLaunch(d->exec, s), "decoder_greedy: graph launch")) return 0;
    if (!rt_hip_ok(hipMemcpyAsync(tokens, d->tokens, (size_t)n * 4, hipMemcpyDeviceToHost, s),
                   "decoder_greedy: tokens"))
        return 0;
    if (margins &&
        !rt_hip_ok(hipMemcpyAsync(margins, d->margins, (size_t)n * 4, hipMemcpyDeviceToHost, s),
                   "decoder_greedy: margins"))
        return 0;
    return rt_hip_ok(hipStreamSynchronize(s), "decoder_greedy");
}

int vbs_gfx950_decoder_greedy_eager(void *handle, uint32_t token, uint32_t pos, uint32_t n,
                                    uint32_t *tokens, float *margins) {
    if (!rt_ready()) return 0;
    Decoder *d = (Decoder *)handle;
    if (!d || !tokens) return rt_fail("decoder_greedy_eager: null argument");
    if (n > d->max_steps)
        return rt_fail("decoder_greedy_eager: %u steps > max_steps %u", n, d->max_steps);
    if ((uint64_t)pos + n > d->m.max_ctx) return rt_fail("decoder_greedy_eager: context exhausted");
    if (!set_state(d, token, pos)) return 0;
    hipStream_t s = rt_stream();
    for (uint32_t i = 0; i < n; i++)
        if (!rt_hip_ok(enqueue_step(*d, s), "decoder_greedy_eager: step")) return 0;
    if (!rt_hip_ok(hipMemcpyAsync(tokens, d->tokens, (size_t)n * 4, hipMemcpyDeviceToHost, s),
                   "decoder_greedy_eager: tokens"))
        return 0;
    if (margins &&
        !rt_hip_ok(hipMemcpyAsync(margins, d->margins, (size_t)n * 4, hipMemcpyDeviceToHost, s),
                   "decoder_greedy_eager: margins"))
        return 0;
    return rt_hip_ok(hipStreamSynchronize(s), "decoder_greedy_eager");
}

int vbs_gfx950_decoder_attn_o_fallbacks(void *handle, uint32_t *count) {
    Decoder *d = (Decoder *)handle;
    if (!d) return rt_fail("decoder: NULL handle");
    uint32_t c = 0;
    if (d->fallbacks && !rt_hip_ok(hipMemcpy(&c, d->fallbacks, sizeof(c), hipMemcpyDeviceToHost),
                                   "decoder: fallbacks"))
        return -1;
    if (count) *count = c;
    return d->fallbacks ? 1 : 0;
}

int vbs_gfx950_decoder_destroy(void *handle) {
    decoder_free((Decoder *)handle);
    return 1;
}

}  // extern "C"

// ---- batched decode step (up to 8 sequences) ---------------------------------
//
// The same token step for `batch` independent sequences, each with its own
// KV cache (sequence b's caches at + b kv_seq elements) and position, over
// one copy of the weights: every matrix is one batched matrix-core launch
// (x prepared once per launch: attn_norm / ffn_norm / output_norm and
// SiLU*up are folded into the preparation), Q, K, V share a launch, as do
// gate and up; O and down add into the residual stream; RoPE and the cache
// store of every sequence are one launch and attention one pair of launches
// over all sequences. 11 launches per layer. The reference has no batched
// decode (src/vbs_specializer.c:353-357 loops tokens one by one): each
// sequence computes the single-sequence step, with the batched matvec's
// arithmetic.
namespace vbs {

__global__ __launch_bounds__(256) void k_rope_store_b(float *__restrict__ q, const float *__restrict__ k,
                                                      const float *__restrict__ v, uint32_t qd,
                                                      uint32_t kvd, uint32_t hd,
                                                      const float2 *__restrict__ tab,
                                                      const uint32_t *__restrict__ pos_dev,
                                                      uint16_t *__restrict__ kc,
                                                      uint16_t *__restrict__ vc, uint64_t kv_seq,
                                                      uint64_t layer_off, uint32_t max_ctx) {
    const uint32_t b = blockIdx.y, u = blockIdx.x * 256u + threadIdx.x;
    const uint32_t pairs = hd / 2u, nqp = qd / 2u, nkp = kvd / 2u;
    if (u >= nqp + 2u * nkp) return;
    const uint32_t pos = pos_dev[b];
    if (pos >= max_ctx) return;  // (the host bounds every greedy run by max_ctx)
    const uint64_t row = (uint64_t)b * kv_seq + layer_off + (uint64_t)pos * kvd;
    auto rope = [&](float &x0, float &x1, uint32_t p) {
        const float2 cs = tab[(uint64_t)pos * pairs + p];
        const float a = x0, c = x1;
        x0 = __fsub_rn(__fmul_rn(a, cs.x), __fmul_rn(c, cs.y));
        x1 = __fadd_rn(__fmul_rn(a, cs.y), __fmul_rn(c, cs.x));
    };
    if (u < nqp) {  // q pair, in place (src/vbs_host_math.h:38-51)
        float *x = q + (uint64_t)b * qd + 2u * u;
        float x0 = x[0], x1 = x[1];
        rope(x0, x1, u % pairs);
        x[0] = x0;
        x[1] = x1;
    } else if (u < nqp + nkp) {  // k pair: RoPE, then the f16 store (src/vbs_host_math.h:150-159)
        const uint32_t i = 2u * (u - nqp);
        float x0 = k[(uint64_t)b * kvd + i], x1 = k[(uint64_t)b * kvd + i + 1u];
        rope(x0, x1, (u - nqp) % pairs);
        kc[row + i] = vbs_f2h(x0);
        kc[row + i + 1u] = vbs_f2h(x1);
    } else {  // v pair: the f16 store
        const uint32_t i = 2u * (u - nqp - nkp);
        vc[row + i] = vbs_f2h(v[(uint64_t)b * kvd + i]);
        vc[row + i + 1u] = vbs_f2h(v[(uint64_t)b * kvd + i + 1u]);
    }
}

struct BDecoder {
    vbs_gfx950_model_t m;
    uint32_t batch = 0;
    uint64_t kv_seq = 0;
    std::vector<const float *> attn_norm, ffn_norm;
    std::vector<int> wtype;
    std::vector<const void *> wdata;
    float *x = nullptr, *q, *k, *v, *attn, *gate, *up, *logits, *part;
    uint8_t *xp = nullptr;
    float2 *rope = nullptr;
    uint32_t *state = nullptr;  // token[batch], pos[batch], step[batch]
    uint32_t *tokens = nullptr;
    float *margins = nullptr;
    uint32_t max_steps = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    void *arena = nullptr;
};

static hipError_t enqueue_step_batch(const BDecoder &d, hipStream_t s) {
    const vbs_gfx950_model_t &m = d.m;
    const uint32_t B = d.batch, H = m.hidden, F = m.ffn, hd = m.head_dim;
    const uint32_t nq = m.n_heads, nkv = m.n_kv_heads, qd = nq * hd, kvd = nkv * hd, V = m.vocab;
    const float scale = 1.0f / sqrtf((float)hd);
    uint32_t *token_dev = d.state, *pos_dev = d.state + B, *step_dev = d.state + 2u * B;
#define VBS_TRY(expr)                     \
    do {                                  \
        hipError_t e_ = (expr);           \
        if (e_ != hipSuccess) return e_;  \
    } while (0)
    // x holds every sequence's token embedding already (the previous step's
    // argmax, or bdecoder_run for the first step)
    const uint32_t units = qd / 2u + kvd;
    for (uint32_t L = 0; L < m.n_layers; L++) {
        const int *t = d.wtype.data() + 7 * L;
        const uint8_t *const *w = (const uint8_t *const *)d.wdata.data() + 7 * L;
        const uint64_t layer_off = (uint64_t)L * m.max_ctx * kvd;
        {  // attn_norm, Q, K, V, RoPE and the cache stores: one launch after the
           // preparation when q, k and v are Q4_K, else the store kernel after them
            VBS_TRY(launch_xprep(XP_NORM, d.x, nullptr, H, d.attn_norm[L], m.rms_eps, H, B, d.xp, s));
            const uint32_t rows[3] = {qd, kvd, kvd}, ys[3] = {qd, kvd, kvd};
            hipError_t e = t[0] == t[1] && t[1] == t[2]
                               ? launch_mvb_qkv(t[0], w, rows, d.q, qd, d.xp, H, B, d.rope, pos_dev, m.kc,
                                                m.vc, d.kv_seq, layer_off, hd, kvd, m.max_ctx, s)
                               : hipErrorNotSupported;
            if (e == hipErrorNotSupported) {
                float *const y[3] = {d.q, d.k, d.v};
                VBS_TRY(launch_mvb(t[0], 3, w, rows, y, ys, 0, d.xp, H, B, s));
                k_rope_store_b<<<dim3((units + 255u) / 256u, B), 256, 0, s>>>(
                    d.q, d.k, d.v, qd, kvd, hd, d.rope, pos_dev, m.kc, m.vc, d.kv_seq, layer_off,
                    m.max_ctx);
                e = hipGetLastError();
            }
            VBS_TRY(e);
        }
        // attention; its merge writes O's prepared x when the matrix-core
        // chunk kernel runs (else the merge, then the preparation)
        hipError_t ea = launch_attention_batch(d.q, m.kc, m.vc, nullptr, m.max_ctx, pos_dev, d.part,
                                               layer_off, nq, nkv, hd, scale, B, qd, d.kv_seq, s);
        if (ea == hipSuccess) {
            ea = launch_attn_merge_prep(d.part, d.xp, attention_chunk_stride(m.max_ctx, nkv), pos_dev,
                                        nq, nkv,
                                        attention_partial_bytes(m.max_ctx, nq, nkv, hd) / sizeof(float),
                                        B, s);
        } else if (ea == hipErrorNotSupported) {
            ea = launch_attention_batch(d.q, m.kc, m.vc, d.attn, m.max_ctx, pos_dev, d.part, layer_off,
                                        nq, nkv, hd, scale, B, qd, d.kv_seq, s);
            if (ea == hipSuccess)
                ea = launch_xprep(XP_PLAIN, d.attn, nullptr, qd, nullptr, 0.f, qd, B, d.xp, s);
        }
        VBS_TRY(ea);
        {  // O, added into the residual stream
            const uint32_t rows[1] = {H}, ys[1] = {H};
            float *const y[1] = {d.x};
            VBS_TRY(launch_mvb(t[3], 1, w + 3, rows, y, ys, 1, d.xp, qd, B, s));
        }
        {  // ffn_norm, gate and up
            VBS_TRY(launch_xprep(XP_NORM, d.x, nullptr, H, d.ffn_norm[L], m.rms_eps, H, B, d.xp, s));
            const uint32_t rows[2] = {F, F}, ys[2] = {F, F};
            float *const y[2] = {d.gate, d.up};
            VBS_TRY(launch_mvb(t[4], 2, w + 4, rows, y, ys, 0, d.xp, H, B, s));
        }
        {  // SiLU*up, down, added into the residual stream
            VBS_TRY(launch_xprep(XP_SILU, d.gate, d.up, F, nullptr, 0.f, F, B, d.xp, s));
            const uint32_t rows[1] = {H}, ys[1] = {H};
            float *const y[1] = {d.x};
            VBS_TRY(launch_mvb(t[6], 1, w + 6, rows, y, ys, 1, d.xp, F, B, s));
        }
    }
    {  // output_norm and lm_head
        VBS_TRY(launch_xprep(XP_NORM, d.x, nullptr, H, m.out_norm, m.rms_eps, H, B, d.xp, s));
        const uint8_t *wh[1] = {(const uint8_t *)m.lm_head};
        const uint32_t rows[1] = {V}, ys[1] = {V};
        float *const y[1] = {d.logits};
        VBS_TRY(launch_mvb(m.head_type, 1, wh, rows, y, ys, 0, d.xp, H, B, s));
    }
    VBS_TRY(launch_argmax_embed(m.embd_type, d.logits, V, B, token_dev, pos_dev, step_dev,
                                d.tokens, d.margins, d.max_steps, m.tok_embd, H, d.x, s));
#undef VBS_TRY
    return hipSuccess;
}

static void bdecoder_free(BDecoder *d) {
    if (!d) return;
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    if (d->arena) {
        (void)hipStreamSynchronize(rt_stream());
        (void)hipFree(d->arena);
    }
    delete d;
}

static bool kq_type(int t) { return t == kQ4_K || t == kQ6_K; }
static bool kq_cols(uint32_t c) { return c && c % 256u == 0 && c / 256u <= 128u; }

}  // namespace vbs

extern "C" {

int vbs_gfx950_bdecoder_create(const vbs_gfx950_model_t *m, uint32_t batch, uint64_t kv_seq_stride,
                               uint32_t max_steps, void **handle) {
    if (!rt_ready()) return 0;
    if (!m || !handle) return rt_fail("bdecoder_create: null argument");
    *handle = nullptr;
    if (batch == 0 || batch > 8u) return rt_fail("bdecoder_create: batch %u outside 1..8", batch);
    if (!m->n_layers || !m->hidden || !m->ffn || !m->n_heads || !m->n_kv_heads || !m->head_dim ||
        !m->vocab || !m->max_ctx)
        return rt_fail("bdecoder_create: empty model dimension");
    if (m->n_heads % m->n_kv_heads || m->n_heads / m->n_kv_heads > 16 || m->head_dim > 256 ||
        (m->head_dim & 1u))
        return rt_fail("bdecoder_create: unsupported head geometry");
    if (!m->tok_embd || !m->out_norm || !m->lm_head || !m->attn_norm || !m->ffn_norm ||
        !m->wtype || !m->wdata || !m->kc || !m->vc)
        return rt_fail("bdecoder_create: null model pointer");
    const uint32_t H = m->hidden, F = m->ffn, qd = m->n_heads * m->head_dim;
    const uint32_t kvd = m->n_kv_heads * m->head_dim, pairs = m->head_dim / 2u;
    if (kv_seq_stride < (uint64_t)m->n_layers * m->max_ctx * kvd)
        return rt_fail("bdecoder_create: kv_seq_stride below one sequence's cache");
    if (!block_elems(m->embd_type)) return rt_fail("bdecoder_create: unsupported embedding type");
    // every matrix on the batched matrix-core path
    if (!kq_type(m->head_type) || !kq_cols(H) || !kq_cols(F) || !kq_cols(qd))
        return rt_fail("bdecoder_create: lm_head and the layer shapes must suit the K-quant "
                       "matrix-core kernels (Q4_K/Q6_K, widths a multiple of 256 up to 32768)");
    for (uint32_t L = 0; L < m->n_layers; L++) {
        const int *t = m->wtype + 7 * L;
        for (uint32_t i = 0; i < 7; i++)
            if (!kq_type(t[i]) || !m->wdata[7 * L + i])
                return rt_fail("bdecoder_create: layer %u matrix %u is not Q4_K/Q6_K", L, i);
        if (t[0] != t[1] || t[1] != t[2] || t[4] != t[5])
            return rt_fail("bdecoder_create: layer %u: q/k/v and gate/up must share a type", L);
    }
    BDecoder *d = new BDecoder();
    d->m = *m;
    d->batch = batch;
    d->kv_seq = kv_seq_stride;
    d->attn_norm.assign(m->attn_norm, m->attn_norm + m->n_layers);
    d->ffn_norm.assign(m->ffn_norm, m->ffn_norm + m->n_layers);
    d->wtype.assign(m->wtype, m->wtype + 7 * m->n_layers);
    d->wdata.assign(m->wdata, m->wdata + 7 * m->n_layers);
    d->max_steps = max_steps ? max_steps : 1;
    const uint64_t B = batch;
    const size_t n_f32 = B * (H + 2ull * qd + 2ull * kvd + 2ull * F + m->vocab);
    const size_t part1 = attention_partial_bytes(m->max_ctx, m->n_heads, m->n_kv_heads, m->head_dim);
    const size_t xpb = xprep_bytes(H > F ? (H > qd ? H : qd) : (F > qd ? F : qd));
    const size_t rope = (size_t)m->max_ctx * pairs * sizeof(float2);
    auto up256 = [](size_t b) { return (b + 255u) & ~(size_t)255u; };
    const size_t sz_f = up256(n_f32 * 4), sz_st = up256(3 * B * 4);
    const size_t sz_tok = up256((size_t)d->max_steps * B * 4);
    const size_t total = sz_f + sz_st + 2 * sz_tok + up256(B * part1) + up256(xpb) + up256(rope);
    if (hipMalloc(&d->arena, total) != hipSuccess) {
        delete d;
        return rt_fail("bdecoder_create: hipMalloc(%zu) failed", total);
    }
    uint8_t *p = (uint8_t *)d->arena;
    float *f = (float *)p;
    d->x = f; f += B * H;
    d->q = f; f += B * qd;
    d->attn = f; f += B * qd;
    d->k = f; f += B * kvd;
    d->v = f; f += B * kvd;
    d->gate = f; f += B * F;
    d->up = f; f += B * F;
    d->logits = f;
    p += sz_f;
    d->state = (uint32_t *)p; p += sz_st;
    d->tokens = (uint32_t *)p; p += sz_tok;
    d->margins = (float *)p; p += sz_tok;
    d->part = (float *)p; p += up256(B * part1);
    d->xp = p; p += up256(xpb);
    d->rope = (float2 *)p;
    std::vector<float2> tab((size_t)m->max_ctx * pairs);
    for (uint32_t pos = 0; pos < m->max_ctx; pos++)
        for (uint32_t pr = 0; pr < pairs; pr++) {
            const uint32_t i = 2u * pr;
            const float angle = (float)pos * powf(m->rope_theta, -(float)i / (float)m->head_dim);
            tab[(size_t)pos * pairs + pr] = make_float2(cosf(angle), sinf(angle));
        }
    hipStream_t s = rt_stream();
    if (!rt_hip_ok(hipMemcpyAsync(d->rope, tab.data(), rope, hipMemcpyHostToDevice, s),
                   "bdecoder_create: rope table") ||
        !rt_hip_ok(hipMemsetAsync(d->state, 0, sz_st, s), "bdecoder_create: state") ||
        !rt_hip_ok(hipStreamSynchronize(s), "bdecoder_create")) {
        bdecoder_free(d);
        return 0;
    }
    if (!rt_hip_ok(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture")) {
        bdecoder_free(d);
        return 0;
    }
    hipError_t e = enqueue_step_batch(*d, s);
    hipGraph_t g = nullptr;
    hipError_t e2 = hipStreamEndCapture(s, &g);
    if (e != hipSuccess || e2 != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        bdecoder_free(d);
        return rt_fail("bdecoder_create: capture failed (%s)",
                       hipGetErrorString(e != hipSuccess ? e : e2));
    }
    d->graph = g;
    if (!rt_hip_ok(hipGraphInstantiate(&d->exec, g, nullptr, nullptr, 0), "graph instantiate")) {
        bdecoder_free(d);
        return 0;
    }
    *handle = d;
    return 1;
}

static int bdecoder_run(void *handle, const uint32_t *tokens0, const uint32_t *pos0, uint32_t n,
                        uint32_t *tokens, float *margins, bool eager, float *logits = nullptr) {
    if (!rt_ready()) return 0;
    BDecoder *d = (BDecoder *)handle;
    if (!d || !tokens0 || !pos0 || !tokens) return rt_fail("bdecoder_greedy: null argument");
    if (n > d->max_steps) return rt_fail("bdecoder_greedy: %u steps > max_steps %u", n, d->max_steps);
    const uint32_t B = d->batch;
    std::vector<uint32_t> st(3 * B, 0u);
    for (uint32_t b = 0; b < B; b++) {
        if (tokens0[b] >= d->m.vocab)
            return rt_fail("bdecoder_greedy: token %u >= vocab %u", tokens0[b], d->m.vocab);
        if ((uint64_t)pos0[b] + n > d->m.max_ctx)
            return rt_fail("bdecoder_greedy: sequence %u: context exhausted", b);
        st[b] = tokens0[b];
        st[B + b] = pos0[b];
    }
    hipStream_t s = rt_stream();
    if (!rt_hip_ok(hipMemcpyAsync(d->state, st.data(), st.size() * 4, hipMemcpyHostToDevice, s),
                   "bdecoder_greedy: state") ||
        !rt_hip_ok(launch_dequant_rows(d->m.embd_type, (const uint8_t *)d->m.tok_embd, d->state, 0,
                                       B, d->m.hidden, d->x, s),
                   "bdecoder_greedy: first embeddings"))
        return 0;
    for (uint32_t i = 0; i < n; i++) {
        if (!rt_hip_ok(eager ? enqueue_step_batch(*d, s) : hipGraphLaunch(d->exec, s),
                       "bdecoder_greedy: step"))
            return 0;
    }
    if (!rt_hip_ok(hipMemcpyAsync(tokens, d->tokens, (size_t)n * B * 4, hipMemcpyDeviceToHost, s),
                   "bdecoder_greedy: tokens"))
        return 0;
    if (margins &&
        !rt_hip_ok(hipMemcpyAsync(margins, d->margins, (size_t)n * B * 4, hipMemcpyDeviceToHost, s),
                   "bdecoder_greedy: margins"))
        return 0;
    if (logits &&
        !rt_hip_ok(hipMemcpyAsync(logits, d->logits, (size_t)B * d->m.vocab * 4, hipMemcpyDeviceToHost,
                                  s),
                   "bdecoder_step: logits"))
        return 0;
    return rt_hip_ok(hipStreamSynchronize(s), "bdecoder_greedy");
}

int vbs_gfx950_bdecoder_greedy(void *handle, const uint32_t *tokens0, const uint32_t *pos0,
                               uint32_t n, uint32_t *tokens, float *margins) {
    return bdecoder_run(handle, tokens0, pos0, n, tokens, margins, false);
}

int vbs_gfx950_bdecoder_greedy_eager(void *handle, const uint32_t *tokens0, const uint32_t *pos0,
                                     uint32_t n, uint32_t *tokens, float *margins) {
    return bdecoder_run(handle, tokens0, pos0, n, tokens, margins, true);
}

int vbs_gfx950_bdecoder_step(void *handle, const uint32_t *tokens, const uint32_t *pos,
                             float *logits) {
    BDecoder *d = (BDecoder *)handle;
    if (!d) return rt_fail("bdecoder_step: null argument");
    std::vector<uint32_t> next(d->batch);
    return bdecoder_run(handle, tokens, pos, 1, next.data(), nullptr, false, logits);
}

int vbs_gfx950_bdecoder_destroy(void *handle) {
    bdecoder_free((BDecoder *)handle);
    return 1;
}

}  // extern "C"
