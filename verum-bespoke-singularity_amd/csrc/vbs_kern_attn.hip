// vbs_kern_attn.hip — single-query GQA attention over the f16 KV cache,
// split along the sequence ("flash decoding").
//
// Reference: vbs_host_attention (src/vbs_host_math.h:170-209): for every q
// head h (kv head h / group), score_s = (float)(double dot(q_h, k_s)) * scale,
// then a sequential online softmax over s < seq_len and out = acc * (1/l).
//
// Each workgroup takes a chunk of positions of one kv head and produces, per
// q head of that kv head, the chunk maximum m, the sum l of exp(score - m)
// and acc[d] = sum exp(score - m) * v[d]; the chunks are merged with
// log-sum-exp rescaling: out = sum_c acc_c * e^(m_c-M) / sum_c l_c * e^(m_c-M).
// The chunk length follows the sequence (attn_split) so that about 512
// workgroups share it at any length. A second kernel merges (a hand-off
// inside one kernel, through device-scope stores, loads and an arrival
// count, measured slower than the kernel boundary on this part).
//
// Fast chunk kernel (head_dim 32/64/128, group <= 8): four waves; lanes of a
// wave split a position's head_dim into 8-element slices (16-byte K and V
// loads), so one wave step covers 64/(head_dim/8) positions ("slots") and a
// wave holds at most four steps, all loaded before any arithmetic. q lives in
// registers (the lane's slice for every q head of the group); the partial
// dot of a slice is an fp32 FMA chain and the slices are added with DPP row
// operations, which leaves every lane of a slot with its scores. Each slot
// keeps its own softmax state (max, sum, acc) over its positions, and one
// LDS pass combines the slots. Scores are fp32 dots of exactly converted f16
// keys instead of the reference's double dot: a relative difference of order
// 1e-7 in each score, far inside the 1e-4 the reference's own backend test
// allows (src/vbs_backend_test.c:617-625).
//
// Other shapes use the generic chunk kernel (double dot, one position per
// four threads).
#include "vbs_dev_common.h"
#include "vbs_internal.h"

namespace vbs {

constexpr uint32_t kChunk = 64;  // positions per workgroup of the generic kernel
constexpr uint32_t kMaxGroup = 16;
constexpr uint32_t kTargetWgs = 512;  // workgroups the sequence split aims for

// Sequence split: chunks of `len` positions (a multiple of gran, at most lmax)
// sized so that about kTargetWgs workgroups cover seq x nkh; n chunks per kv
// head. The chunk kernel, the merge and the host compute it identically.
struct AttnSplit {
    uint32_t len, n;
};
__host__ __device__ inline AttnSplit attn_split(uint32_t seq, uint32_t nkh, uint32_t gran,
                                                uint32_t lmax) {
    const uint32_t per = (uint32_t)(((uint64_t)seq * nkh + kTargetWgs - 1u) / kTargetWgs);
    uint32_t len = (per + gran - 1u) / gran * gran;
    len = len < gran ? gran : len > lmax ? lmax : len;
    return {len, (seq + len - 1u) / len};
}
// Chunks per kv head of any split of a sequence of at most max_seq (every
// len >= 64 or len >= seq * nkh / kTargetWgs).
inline uint32_t attn_max_chunks(uint32_t max_seq, uint32_t nkh) {
    const uint32_t a = (kTargetWgs + nkh - 1u) / nkh, b = (max_seq + 63u) / 64u;
    return a > b ? a : b;
}

// f16 bits -> f32 with the hardware converter (exact for every finite value).
__device__ __forceinline__ float hcvt(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// ---- generic chunk kernel ------------------------------------------------------
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


// ---- fast chunk kernel ---------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                     CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of L lanes (L = 4, 8, 16); every lane of the
// group receives the sum.
template <uint32_t L>
__device__ __forceinline__ float group_sum(float v) {
    v = dpp_add<0xB1>(v);                        // quad_perm [1,0,3,2]
    v = dpp_add<0x4E>(v);                        // quad_perm [2,3,0,1]
    if constexpr (L >= 8) v = dpp_add<0x141>(v);  // row_half_mirror
    if constexpr (L >= 16) v = dpp_add<0x140>(v); // row_mirror
    return v;
}

// e^x as 2^(x log2 e) on the hardware exponential (a few ulp; the scores
// themselves differ from the reference's double dots by ~1e-7 relative).
__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// Shape of the fast kernel: four waves; LPP lanes per position (8 head dims
// each), so a wave step covers PPW positions; a wave holds at most kSteps steps.
constexpr uint32_t kWaves = 4, kSteps = 4;
template <uint32_t HD>
struct ChunkShape {
    static constexpr uint32_t LPP = HD / 8, PPW = 64 / LPP, GRAN = kWaves * PPW,
                              LMAX = kSteps * GRAN;
};

template <uint32_t HD, uint32_t GMAX>
__global__ __launch_bounds__(64 * kWaves) void k_attn_chunk(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
    float *__restrict__ part, uint32_t seq_len, const uint32_t *__restrict__ pos_dev,
    uint64_t layer_off, uint32_t nkh, uint32_t group, float scale, uint32_t stride_chunks) {
    using S = ChunkShape<HD>;
    constexpr uint32_t LPP = S::LPP, PPW = S::PPW, NK = kWaves * PPW;  // NK position slots
    extern __shared__ __align__(16) uint8_t chunk_lds[];
    float *red = reinterpret_cast<float *>(chunk_lds);  // [NK][group][HD] acc per slot
    __shared__ float sm[NK][GMAX], sl[NK][GMAX], sf[NK][GMAX];

    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, t = threadIdx.x;
    const uint32_t wave = t >> 6, lane = t & 63u;
    const uint32_t slot = lane / LPP, c = lane % LPP, k = wave * PPW + slot;
    if (pos_dev) seq_len = pos_dev[0] + 1u;  // graph replay: the device holds the position
    const AttnSplit sp = attn_split(seq_len, nkh, S::GRAN, S::LMAX);
    if (chunk >= sp.n) return;  // past the sequence (the grid covers the longest split)
    const uint32_t s0 = chunk * sp.len;
    const uint32_t valid = min(sp.len, seq_len - s0);
    const uint32_t pw = sp.len / kWaves, ns = pw / PPW;  // positions and steps per wave
    const uint64_t rstride = (uint64_t)nkh * HD;
    const uint64_t base = layer_off + (uint64_t)s0 * rstride + (uint64_t)kvh * HD + 8u * c;

    // ---- this wave's K and V rows first (position wave*pw + b*PPW + slot;
    // positions past the chunk re-read its last row and are masked) ----------
    uint4 kr[kSteps], vr[kSteps];
#pragma unroll
    for (uint32_t b = 0; b < kSteps; b++) {
        if (b < ns) {
            const uint32_t p = min(wave * pw + b * PPW + slot, valid - 1u);
            kr[b] = *reinterpret_cast<const uint4 *>(kc + base + (uint64_t)p * rstride);
            vr[b] = *reinterpret_cast<const uint4 *>(vc + base + (uint64_t)p * rstride);
            // masked positions (re-read rows) add zeros: e = 0 and v = 0
            if (wave * pw + b * PPW + slot >= valid) vr[b] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    float qv[GMAX][8];
#pragma unroll
    for (uint32_t g = 0; g < GMAX; g++) {
        const uint32_t gg = g < group ? g : 0u;
        const float4 *qp =
            reinterpret_cast<const float4 *>(q + ((uint64_t)kvh * group + gg) * HD + 8u * c);
        const float4 a = qp[0], b4 = qp[1];
        qv[g][0] = a.x; qv[g][1] = a.y; qv[g][2] = a.z; qv[g][3] = a.w;
        qv[g][4] = b4.x; qv[g][5] = b4.y; qv[g][6] = b4.z; qv[g][7] = b4.w;
    }

    // ---- scores: every lane of a slot holds its position's scores --------------
    float sc[kSteps][GMAX];
#pragma unroll
    for (uint32_t b = 0; b < kSteps; b++) {
        const bool in = b < ns && wave * pw + b * PPW + slot < valid;
        float kf[8];
        if (b < ns) {
            const uint32_t kw[4] = {kr[b].x, kr[b].y, kr[b].z, kr[b].w};
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) kf[j] = hcvt(kw[j >> 1] >> (16u * (j & 1u)));
        }
#pragma unroll
        for (uint32_t g = 0; g < GMAX; g++) {
            float p = 0.f;
            if (b < ns) {
#pragma unroll
                for (uint32_t j = 0; j < 8; j++) p = fmaf(qv[g][j], kf[j], p);
                p = group_sum<LPP>(p);
            }
            sc[b][g] = in ? __fmul_rn(p, scale) : -INFINITY;
        }
    }

    // ---- per slot: m = max score, l = sum e^(s - m), acc = sum e^(s - m) v -----
#pragma unroll
    for (uint32_t g = 0; g < GMAX; g++) {
        float m = sc[0][g];
#pragma unroll
        for (uint32_t b = 1; b < kSteps; b++) m = fmaxf(m, sc[b][g]);
        float l = 0.f, acc[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) acc[j] = 0.f;
#pragma unroll
        for (uint32_t b = 0; b < kSteps; b++) {
            if (b < ns) {
                const float e = sc[b][g] == -INFINITY ? 0.f : fast_exp(__fsub_rn(sc[b][g], m));
                const uint32_t vw[4] = {vr[b].x, vr[b].y, vr[b].z, vr[b].w};
                l += e;
#pragma unroll
                for (uint32_t j = 0; j < 8; j++)
                    acc[j] = fmaf(e, hcvt(vw[j >> 1] >> (16u * (j & 1u))), acc[j]);
            }
        }
        if (g < group) {
            float *dst = red + ((k * group + g) * HD + 8u * c);
            reinterpret_cast<float4 *>(dst)[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
            reinterpret_cast<float4 *>(dst)[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
            if (c == 0) {
                sm[k][g] = m;
                sl[k][g] = l;
            }
        }
    }
    __syncthreads();

    // ---- combine the slots: M = max m_k, weights e^(m_k - M) (0 for empty slots)
    if (t < NK * GMAX) {
        const uint32_t kk = t / GMAX, g = t % GMAX;
        if (g < group) {
            float M = sm[0][g];
#pragma unroll
            for (uint32_t i = 1; i < NK; i++) M = fmaxf(M, sm[i][g]);
            const float mk = sm[kk][g];
            sf[kk][g] = mk == -INFINITY ? 0.f : fast_exp(__fsub_rn(mk, M));
        }
    }
    __syncthreads();
    float *const pk = part + (uint64_t)kvh * group * stride_chunks * (HD + 2u);
    for (uint32_t i = t; i < group * HD; i += 64u * kWaves) {
        const uint32_t g = i / HD, d = i % HD;
        float a = 0.f;
#pragma unroll
        for (uint32_t kk = 0; kk < NK; kk++) a = fmaf(red[(kk * group + g) * HD + d], sf[kk][g], a);
        float *dst = pk + ((uint64_t)g * stride_chunks + chunk) * (HD + 2u);
        dst[2u + d] = a;
        if (d == 0) {
            float M = sm[0][g], L = 0.f;
#pragma unroll
            for (uint32_t kk = 1; kk < NK; kk++) M = fmaxf(M, sm[kk][g]);
#pragma unroll
            for (uint32_t kk = 0; kk < NK; kk++) L = fmaf(sl[kk][g], sf[kk][g], L);
            dst[0] = M;
            dst[1] = L;
        }
    }
}

// ---- merge of the chunks -------------------------------------------------------
// One workgroup per q head; every global load is issued up front: thread
// (d, slice) loads acc_c[d] of its chunks c = slice, slice + ns, ... and
// thread t also m_t and l_t. Then M = max_c m_c (block maximum), weights
// w_c = e^(m_c - M) in LDS, L = sum_c l_c w_c, and the slices' weighted sums
// are added in LDS in a fixed order.
constexpr uint32_t kMergeBatch = 32;  // chunks per thread held in registers at once

__global__ __launch_bounds__(256) void k_attn_merge(const float *__restrict__ part,
                                                    float *__restrict__ out, uint32_t hd,
                                                    uint32_t n_chunks, uint32_t stride_chunks,
                                                    const uint32_t *__restrict__ pos_dev,
                                                    uint32_t nkh, uint32_t gran, uint32_t lmax) {
    extern __shared__ __align__(16) uint8_t merge_lds[];
    float *w = reinterpret_cast<float *>(merge_lds);  // [stride_chunks]
    float *sl = w + stride_chunks;                    // [256]
    __shared__ float red[8];
    const uint32_t h = blockIdx.x, t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    if (pos_dev) n_chunks = attn_split(pos_dev[0] + 1u, nkh, gran, lmax).n;  // seq_len = pos + 1
    const float *ph = part + (uint64_t)h * stride_chunks * (hd + 2u);
    const uint32_t ns = 256u / hd;
    const uint32_t d = t % hd, s = t / hd;
    float av[kMergeBatch];
#pragma unroll
    for (uint32_t k = 0; k < kMergeBatch; k++) {
        const uint32_t c = s + k * ns;
        av[k] = (s < ns && c < n_chunks) ? ph[(uint64_t)c * (hd + 2u) + 2u + d] : 0.f;
    }
    // this thread's chunks' (m, l): c = t, t + 256, ...
    float M = -INFINITY;
    for (uint32_t c = t; c < n_chunks; c += 256u) M = fmaxf(M, ph[(uint64_t)c * (hd + 2u)]);
    M = wave_max(M);
    if (lane == 0) red[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float L = 0.f;
    for (uint32_t c = t; c < n_chunks; c += 256u) {
        const float *pc = ph + (uint64_t)c * (hd + 2u);
        const float mc = pc[0], wc = mc == -INFINITY ? 0.f : fast_exp(__fsub_rn(mc, M));
        w[c] = wc;
        L = fmaf(pc[1], wc, L);
    }
    L = wave_sum(L);
    if (lane == 0) red[4 + wave] = L;
    __syncthreads();
    L = (red[4] + red[5]) + (red[6] + red[7]);
    float a = 0.f;
    if (s < ns) {
#pragma unroll
        for (uint32_t k = 0; k < kMergeBatch; k++) {
            const uint32_t c = s + k * ns;
            if (c < n_chunks) a = fmaf(av[k], w[c], a);
        }
        for (uint32_t c = s + kMergeBatch * ns; c < n_chunks; c += ns)
            a = fmaf(ph[(uint64_t)c * (hd + 2u) + 2u + d], w[c], a);
    }
    sl[t] = a;
    __syncthreads();
    if (t < hd) {
        float acc = 0.f;
        for (uint32_t k = 0; k < ns; k++) acc += sl[k * hd + t];
        out[(uint64_t)h * hd + t] = __fmul_rn(acc, __fdiv_rn(1.0f, L));
    }
}

size_t attention_partial_bytes(uint32_t max_seq, uint32_t nqh, uint32_t nkh, uint32_t hd) {
    return (size_t)nqh * attn_max_chunks(max_seq, nkh) * (hd + 2u) * sizeof(float);
}

template <uint32_t HD>
static hipError_t launch_chunk_hd(dim3 grid, hipStream_t s, const float *q, const uint16_t *kc,
                                  const uint16_t *vc, float *part, uint32_t seq_len,
                                  const uint32_t *pos_dev, uint64_t layer_off, uint32_t nkh,
                                  uint32_t group, float scale) {
    const size_t lds = (size_t)ChunkShape<HD>::GRAN * group * HD * sizeof(float);
#define VBS_ATTN_G(GG)                                                                          \
    do {                                                                                        \
        k_attn_chunk<HD, GG><<<grid, 64u * kWaves, lds, s>>>(q, kc, vc, part, seq_len, pos_dev,   \
                                                            layer_off, nkh, group, scale, grid.x);\
        return hipGetLastError();                                                                 \
    } while (0)
    if (group <= 1) VBS_ATTN_G(1);
    if (group <= 2) VBS_ATTN_G(2);
    if (group <= 4) VBS_ATTN_G(4);
    VBS_ATTN_G(8);
#undef VBS_ATTN_G
}

hipError_t launch_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                            uint32_t seq_len, const uint32_t *pos_dev, float *part,
                            uint64_t layer_off, uint32_t nqh, uint32_t nkh, uint32_t hd,
                            float scale, hipStream_t s) {
    if (seq_len == 0 || nkh == 0 || nqh % nkh != 0 || hd == 0 || hd > 256 || (hd & 1u))
        return hipErrorInvalidValue;
    const uint32_t group = nqh / nkh;
    if (group > kMaxGroup) return hipErrorInvalidValue;
    // with pos_dev, seq_len is the largest sequence the grid must cover
    const uint32_t stride = attn_max_chunks(seq_len, nkh);
    if (!part) part = (float *)scratch(attention_partial_bytes(seq_len, nqh, nkh, hd), s);
    if (!part) return hipErrorOutOfMemory;
    const bool fast = (hd == 32u || hd == 64u || hd == 128u) && group <= 8u &&
                      ((uintptr_t)q & 15u) == 0 && ((uintptr_t)kc & 15u) == 0 &&
                      ((uintptr_t)vc & 15u) == 0;
    hipError_t e;
    uint32_t gran = kChunk, lmax = kChunk;
    const dim3 grid(stride, nkh);
    if (fast && hd == 32u) {
        gran = ChunkShape<32>::GRAN, lmax = ChunkShape<32>::LMAX;
        e = launch_chunk_hd<32>(grid, s, q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, group,
                                scale);
    } else if (fast && hd == 64u) {
        gran = ChunkShape<64>::GRAN, lmax = ChunkShape<64>::LMAX;
        e = launch_chunk_hd<64>(grid, s, q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, group,
                                scale);
    } else if (fast) {
        gran = ChunkShape<128>::GRAN, lmax = ChunkShape<128>::LMAX;
        e = launch_chunk_hd<128>(grid, s, q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, group,
                                 scale);
    } else {
        const size_t lds = ((size_t)group * hd + (size_t)group * kChunk +
                            (size_t)(256u / hd) * group * hd) * sizeof(float);
        k_attn_partial<<<grid, 256, lds, s>>>(q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, hd,
                                              group, scale, stride);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
    const uint32_t n_chunks = attn_split(seq_len, nkh, gran, lmax).n;
    const size_t mlds = ((size_t)stride + 256u) * sizeof(float);
    k_attn_merge<<<nqh, 256, mlds, s>>>(part, out, hd, n_chunks, stride, pos_dev, nkh, gran, lmax);
    return hipGetLastError();
}

}  // namespace vbs
