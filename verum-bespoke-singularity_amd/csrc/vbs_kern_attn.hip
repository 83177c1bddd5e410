// vbs_kern_attn.hip — single-query GQA attention over the f16 KV cache,
// split along the sequence ("flash decoding").
//
// Reference: vbs_host_attention (src/vbs_host_math.h:170-209): for every q
// head h (kv head h / group), score_s = (float)(double dot(q_h, k_s)) * scale,
// then a sequential online softmax over s < seq_len and out = acc * (1/l).
//
// Here: phase 1 gives each workgroup one kv head and a chunk of 64 positions;
// it computes the scores of all q heads of that kv head (the dot in double, as
// the reference does), the chunk maximum m, l = sum exp(score - m) and
// acc = sum exp(score - m) * v. Phase 2 merges the chunks with the usual
// log-sum-exp rescaling. The result equals the reference's up to fp32
// rounding order (the reference's own backend test allows 1e-4).
#include "vbs_dev_common.h"
#include "vbs_internal.h"

namespace vbs {

constexpr uint32_t kChunk = 64;  // positions per workgroup
constexpr uint32_t kMaxGroup = 16;

__global__ __launch_bounds__(256) void k_attn_partial(const float *__restrict__ q,
                                                      const uint16_t *__restrict__ kc,
                                                      const uint16_t *__restrict__ vc,
                                                      float *__restrict__ part,
                                                      uint32_t seq_len, const uint32_t *pos_dev,
                                                      uint64_t layer_off, uint32_t nkh, uint32_t hd,
                                                      uint32_t group, float scale,
                                                      uint32_t n_chunks) {
    extern __shared__ float lds[];
    float *qs = lds;                       // [group][hd]
    float *ps = qs + group * hd;           // [group][kChunk]
    float *red = ps + group * kChunk;      // [256 / hd][group][hd] partial acc

    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, t = threadIdx.x;
    // graph replays take the position from device memory: seq_len = pos + 1
    if (pos_dev) seq_len = pos_dev[0] + 1u;
    const uint32_t s0 = chunk * kChunk;
    if (s0 >= seq_len) return;  // chunk past the current sequence (grid sized for the maximum)
    const uint32_t valid = min(kChunk, seq_len - s0);

    for (uint32_t i = t; i < group * hd; i += 256u) qs[i] = q[(uint64_t)kvh * group * hd + i];
    __syncthreads();

    // Scores: four threads per position, each a quarter of the head dim.
    {
        const uint32_t sl = t >> 2, quarter = t & 3u;
        double dot[kMaxGroup];
#pragma unroll
        for (uint32_t g = 0; g < kMaxGroup; g++) dot[g] = 0.0;
        if (sl < valid) {
            const uint16_t *kr = kc + layer_off + ((uint64_t)(s0 + sl) * nkh + kvh) * hd;
            uint32_t d0 = (hd / 4u) * quarter, d1 = quarter == 3u ? hd : d0 + hd / 4u;
            for (uint32_t d = d0; d < d1; d++) {
                double kv = (double)h2f(kr[d]);
#pragma unroll
                for (uint32_t g = 0; g < kMaxGroup; g++)
                    if (g < group) dot[g] = fma((double)qs[g * hd + d], kv, dot[g]);
            }
        }
#pragma unroll
        for (uint32_t g = 0; g < kMaxGroup; g++) {
            if (g < group) {
                double v = dot[g];
                v += __shfl_xor(v, 1, 64);
                v += __shfl_xor(v, 2, 64);
                if (quarter == 0)
                    ps[g * kChunk + sl] = sl < valid ? __fmul_rn((float)v, scale) : -INFINITY;
            }
        }
    }
    __syncthreads();

    // Chunk softmax statistics, one wavefront per q head.
    const uint32_t wave = t >> 6, lane = t & 63u;
    for (uint32_t g = wave; g < group; g += 4u) {
        float sc = ps[g * kChunk + lane];
        float m = wave_max(sc);
        float e = lane < valid ? expf(sc - m) : 0.f;
        float l = wave_sum(e);
        ps[g * kChunk + lane] = e;
        if (lane == 0) {
            float *dst = part + ((uint64_t)(kvh * group + g) * n_chunks + chunk) * (hd + 2u);
            dst[0] = m;
            dst[1] = l;
        }
    }
    __syncthreads();

    // acc[g][d] = sum_s p[g][s] * v[s][d]; threads split (d, s-slice).
    const uint32_t nsl = 256u / hd, d = t % hd, sg = t / hd;
    float acc[kMaxGroup];
#pragma unroll
    for (uint32_t g = 0; g < kMaxGroup; g++) acc[g] = 0.f;
    if (sg < nsl) {
        for (uint32_t sl = sg; sl < valid; sl += nsl) {
            float v = h2f(vc[layer_off + ((uint64_t)(s0 + sl) * nkh + kvh) * hd + d]);
#pragma unroll
            for (uint32_t g = 0; g < kMaxGroup; g++)
                if (g < group) acc[g] = fmaf(ps[g * kChunk + sl], v, acc[g]);
        }
#pragma unroll
        for (uint32_t g = 0; g < kMaxGroup; g++)
            if (g < group) red[(sg * group + g) * hd + d] = acc[g];
    }
    __syncthreads();
    for (uint32_t i = t; i < group * hd; i += 256u) {
        uint32_t g = i / hd, dd = i % hd;
        float sum = 0.f;
        for (uint32_t k = 0; k < nsl; k++) sum += red[(k * group + g) * hd + dd];
        part[((uint64_t)(kvh * group + g) * n_chunks + chunk) * (hd + 2u) + 2u + dd] = sum;
    }
}

__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ part,
                                                      float *__restrict__ out, uint32_t hd,
                                                      uint32_t n_chunks, const uint32_t *pos_dev) {
    const uint32_t h = blockIdx.x;
    const uint32_t stride = n_chunks;  // partial rows are laid out for the full grid
    if (pos_dev) n_chunks = (pos_dev[0] + kChunk) / kChunk;  // chunks of seq_len = pos + 1
    const float *ph = part + (uint64_t)h * stride * (hd + 2u);
    float M = -INFINITY;
    for (uint32_t c = 0; c < n_chunks; c++) M = fmaxf(M, ph[(uint64_t)c * (hd + 2u)]);
    float l = 0.f;
    for (uint32_t c = 0; c < n_chunks; c++) {
        const float *pc = ph + (uint64_t)c * (hd + 2u);
        l = fmaf(pc[1], expf(pc[0] - M), l);
    }
    float inv = __fdiv_rn(1.0f, l);
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.f;
        for (uint32_t c = 0; c < n_chunks; c++) {
            const float *pc = ph + (uint64_t)c * (hd + 2u);
            acc = fmaf(pc[2u + d], expf(pc[0] - M), acc);
        }
        out[(uint64_t)h * hd + d] = __fmul_rn(acc, inv);
    }
}

size_t attention_partial_bytes(uint32_t max_seq, uint32_t nqh, uint32_t hd) {
    return (size_t)nqh * ((max_seq + kChunk - 1u) / kChunk) * (hd + 2u) * sizeof(float);
}

hipError_t launch_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                            uint32_t seq_len, const uint32_t *pos_dev, float *part,
                            uint64_t layer_off, uint32_t nqh, uint32_t nkh, uint32_t hd,
                            float scale, hipStream_t s) {
    if (seq_len == 0 || nkh == 0 || nqh % nkh != 0 || hd == 0 || hd > 256 || (hd & 1u))
        return hipErrorInvalidValue;
    uint32_t group = nqh / nkh;
    if (group > kMaxGroup) return hipErrorInvalidValue;
    // with pos_dev, seq_len is the largest sequence the grid must cover
    uint32_t n_chunks = (seq_len + kChunk - 1u) / kChunk;
    if (!part) part = (float *)scratch(attention_partial_bytes(seq_len, nqh, hd), s);
    if (!part) return hipErrorOutOfMemory;
    size_t lds = ((size_t)group * hd + (size_t)group * kChunk + (size_t)(256u / hd) * group * hd) *
                 sizeof(float);
    dim3 grid(n_chunks, nkh);
    k_attn_partial<<<grid, 256, lds, s>>>(q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, hd,
                                          group, scale, n_chunks);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_attn_combine<<<nqh, hd < 256u ? hd : 256u, 0, s>>>(part, out, hd, n_chunks, pos_dev);
    return hipGetLastError();
}

}  // namespace vbs
