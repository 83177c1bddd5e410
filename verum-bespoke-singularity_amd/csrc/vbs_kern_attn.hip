// vbs_kern_attn.hip — single-query GQA attention over the f16 KV cache,
// split along the sequence ("flash decoding").
//
// Reference: vbs_host_attention (src/vbs_host_math.h:170-209): for every q
// head h (kv head h / group), score_s = (float)(double dot(q_h, k_s)) * scale,
// then a sequential online softmax over s < seq_len and out = acc * (1/l).
//
// Two kernels. The first gives each workgroup a chunk of 64 positions of one
// kv head and writes, per q head of that kv head, the chunk maximum m, the
// sum l of exp(score - m) and acc[d] = sum exp(score - m) * v[d]. The second
// merges the chunks with log-sum-exp rescaling: out = sum_c acc_c * e^(m_c-M)
// / sum_c l_c * e^(m_c-M).
//
// Fast chunk kernel (head_dim 32/64/128, group <= 8): lanes of a wave split a
// position's head_dim into 8-element slices (16-byte K and V loads), so a
// wave covers 64/(head_dim/8) positions per load; every K and V load of the
// wave is issued before any arithmetic. q lives in registers (the lane's
// slice for every q head of the group); the partial dot of a slice is an
// fp32 FMA chain and the slices are added with DPP row operations. The
// softmax statistics and the V sums are combined across the chunk in LDS.
// Scores are fp32 dots of exactly converted f16 keys instead of the
// reference's double dot: a relative difference of order 1e-7 in each score,
// far inside the 1e-4 the reference's own backend test allows
// (src/vbs_backend_test.c:617-625).
//
// Other shapes use the generic chunk kernel (double dot, one position per
// four threads).
#include "vbs_dev_common.h"
#include "vbs_internal.h"

namespace vbs {

constexpr uint32_t kChunk = 64;  // positions per workgroup
constexpr uint32_t kMaxGroup = 16;

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

template <uint32_t HD, uint32_t GMAX, uint32_t NWV>
__global__ __launch_bounds__(64 * NWV) void k_attn_chunk(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
    float *__restrict__ part, uint32_t seq_len, const uint32_t *__restrict__ pos_dev,
    uint64_t layer_off, uint32_t nkh, uint32_t group, float scale, uint32_t stride_chunks) {
    constexpr uint32_t LPP = HD / 8;            // lanes per position
    constexpr uint32_t PPW = 64 / LPP;          // positions per wave per load
    constexpr uint32_t NB = kChunk / NWV / PPW;  // loads per wave (K and V each)
    static_assert(NB >= 1 && NB * PPW * NWV == kChunk, "chunk split");
    extern __shared__ __align__(16) uint8_t chunk_lds[];
    float *red = reinterpret_cast<float *>(chunk_lds);  // [NWV][group][HD] acc
    __shared__ float wmax[NWV][GMAX];
    __shared__ float lsum[NWV][GMAX];

    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, t = threadIdx.x;
    const uint32_t wave = t >> 6, lane = t & 63u;
    const uint32_t slot = lane / LPP, c = lane % LPP;
    if (pos_dev) seq_len = pos_dev[0] + 1u;  // graph replay: the device holds the position
    const uint32_t s0 = chunk * kChunk;
    if (s0 >= seq_len) return;  // chunk past the sequence (grid sized for the maximum)
    const uint32_t valid = min(kChunk, seq_len - s0);
    const uint64_t rstride = (uint64_t)nkh * HD;
    const uint64_t base = layer_off + (uint64_t)s0 * rstride + (uint64_t)kvh * HD + 8u * c;

    // ---- every K and V load of this wave first (positions past the sequence
    // re-read its last row and are masked below) -----------------------------
    uint4 kr[NB], vr[NB];
#pragma unroll
    for (uint32_t b = 0; b < NB; b++) {
        const uint32_t sp = min(wave * (NB * PPW) + b * PPW + slot, valid - 1u);
        kr[b] = *reinterpret_cast<const uint4 *>(kc + base + (uint64_t)sp * rstride);
    }
#pragma unroll
    for (uint32_t b = 0; b < NB; b++) {
        const uint32_t sp = min(wave * (NB * PPW) + b * PPW + slot, valid - 1u);
        vr[b] = *reinterpret_cast<const uint4 *>(vc + base + (uint64_t)sp * rstride);
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

    // ---- scores ------------------------------------------------------------
    float sc[NB][GMAX];
#pragma unroll
    for (uint32_t b = 0; b < NB; b++) {
        const uint32_t kw[4] = {kr[b].x, kr[b].y, kr[b].z, kr[b].w};
        float kf[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) kf[j] = hcvt(kw[j >> 1] >> (16u * (j & 1u)));
        const bool in = wave * (NB * PPW) + b * PPW + slot < valid;
#pragma unroll
        for (uint32_t g = 0; g < GMAX; g++) {
            float p = 0.f;
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) p = fmaf(qv[g][j], kf[j], p);
            p = group_sum<LPP>(p);
            sc[b][g] = in ? __fmul_rn(p, scale) : -INFINITY;
        }
    }

    // ---- chunk maximum per q head --------------------------------------------
#pragma unroll
    for (uint32_t g = 0; g < GMAX; g++) {
        float m = sc[0][g];
#pragma unroll
        for (uint32_t b = 1; b < NB; b++) m = fmaxf(m, sc[b][g]);
#pragma unroll
        for (uint32_t off = LPP; off < 64u; off <<= 1) m = fmaxf(m, __shfl_xor(m, (int)off, 64));
        if (lane == 0) wmax[wave][g] = m;
    }
    __syncthreads();

    // ---- e = exp(score - m); acc and l over this wave's positions ------------
    float cm[GMAX];
#pragma unroll
    for (uint32_t g = 0; g < GMAX; g++) {
        float m = wmax[0][g];
#pragma unroll
        for (uint32_t k = 1; k < NWV; k++) m = fmaxf(m, wmax[k][g]);
        cm[g] = m;
        float l = 0.f, acc[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) acc[j] = 0.f;
#pragma unroll
        for (uint32_t b = 0; b < NB; b++) {
            const float e = sc[b][g] == -INFINITY ? 0.f : expf(__fsub_rn(sc[b][g], m));
            const uint32_t vw[4] = {vr[b].x, vr[b].y, vr[b].z, vr[b].w};
            l += e;
#pragma unroll
            for (uint32_t j = 0; j < 8; j++)
                acc[j] = e == 0.f ? acc[j] : fmaf(e, hcvt(vw[j >> 1] >> (16u * (j & 1u))), acc[j]);
        }
        // add the wave's position slots (lanes LPP apart hold the same dims)
#pragma unroll
        for (uint32_t off = LPP; off < 64u; off <<= 1) {
            l += __shfl_xor(l, (int)off, 64);
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) acc[j] += __shfl_xor(acc[j], (int)off, 64);
        }
        if (g < group && slot == 0) {
            float *dst = red + ((wave * group + g) * HD + 8u * c);
            reinterpret_cast<float4 *>(dst)[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
            reinterpret_cast<float4 *>(dst)[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
            if (c == 0) lsum[wave][g] = l;
        }
    }
    __syncthreads();

    // ---- combine the waves' partials of the chunk and write (m, l, acc) ------
    for (uint32_t i = t; i < group * HD; i += 64u * NWV) {
        const uint32_t g = i / HD, d = i % HD;
        float a = 0.f;
#pragma unroll
        for (uint32_t k = 0; k < NWV; k++) a += red[(k * group + g) * HD + d];
        float *dst = part + ((uint64_t)(kvh * group + g) * stride_chunks + chunk) * (HD + 2u);
        dst[2u + d] = a;
        if (d == 0) {
            float ls = 0.f;
#pragma unroll
            for (uint32_t k = 0; k < NWV; k++) ls += lsum[k][g];
            float m = wmax[0][g];
#pragma unroll
            for (uint32_t k = 1; k < NWV; k++) m = fmaxf(m, wmax[k][g]);
            dst[0] = m;
            dst[1] = ls;
        }
    }
    (void)cm;
}

// ---- merge of the chunks -------------------------------------------------------
// One workgroup per q head. Every partial is requested up front: thread
// (d, slice) loads acc_c[d] of its chunks c = slice, slice + ns, ... while the
// chunk maxima and sums are combined (block max, weights e^(m_c - M) in LDS,
// L = sum l_c e^(m_c - M)); the slices are then added in LDS in a fixed order.
constexpr uint32_t kMergeBatch = 16;  // chunks per thread held in registers at once

__global__ __launch_bounds__(256) void k_attn_merge(const float *__restrict__ part,
                                                    float *__restrict__ out, uint32_t hd,
                                                    uint32_t n_chunks, uint32_t stride_chunks,
                                                    const uint32_t *__restrict__ pos_dev) {
    extern __shared__ __align__(16) uint8_t merge_lds[];
    float *w = reinterpret_cast<float *>(merge_lds);  // [stride_chunks]
    float *sl = w + stride_chunks;                    // [256]
    __shared__ float red[8];
    const uint32_t h = blockIdx.x, t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    if (pos_dev) n_chunks = (pos_dev[0] + kChunk) / kChunk;  // chunks of seq_len = pos + 1
    const float *ph = part + (uint64_t)h * stride_chunks * (hd + 2u);
    const uint32_t ns = 256u / hd;
    const uint32_t d = t % hd, s = t / hd;
    // this thread's first batch of acc values, requested before anything else
    float av[kMergeBatch];
#pragma unroll
    for (uint32_t k = 0; k < kMergeBatch; k++) {
        const uint32_t c = s + k * ns;
        av[k] = (s < ns && c < n_chunks) ? ph[(uint64_t)c * (hd + 2u) + 2u + d] : 0.f;
    }
    // M = max_c m_c
    float M = -INFINITY;
    for (uint32_t c = t; c < n_chunks; c += 256u) M = fmaxf(M, ph[(uint64_t)c * (hd + 2u)]);
    M = wave_max(M);
    if (lane == 0) red[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // weights and L = sum_c l_c * w_c
    float L = 0.f;
    for (uint32_t c = t; c < n_chunks; c += 256u) {
        const float *pc = ph + (uint64_t)c * (hd + 2u);
        const float wc = expf(__fsub_rn(pc[0], M));
        w[c] = wc;
        L = fmaf(pc[1], wc, L);
    }
    L = wave_sum(L);
    if (lane == 0) red[4 + wave] = L;
    __syncthreads();
    L = (red[4] + red[5]) + (red[6] + red[7]);
    // acc[d] = sum_c w_c * acc_c[d] over this thread's chunks
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

size_t attention_partial_bytes(uint32_t max_seq, uint32_t nqh, uint32_t hd) {
    return (size_t)nqh * ((max_seq + kChunk - 1u) / kChunk) * (hd + 2u) * sizeof(float);
}

template <uint32_t HD, uint32_t GMAX>
static hipError_t launch_chunk_t(dim3 grid, hipStream_t s, const float *q, const uint16_t *kc,
                                 const uint16_t *vc, float *part, uint32_t seq_len,
                                 const uint32_t *pos_dev, uint64_t layer_off, uint32_t nkh,
                                 uint32_t group, float scale) {
    // eight waves of 64 / 8 positions where a wave still covers whole loads
    constexpr uint32_t PPW = 64 / (HD / 8);
    constexpr uint32_t NWV = kChunk / PPW >= 8u ? 8u : kChunk / PPW;
    const size_t lds = (size_t)NWV * group * HD * sizeof(float);
    k_attn_chunk<HD, GMAX, NWV><<<grid, 64u * NWV, lds, s>>>(q, kc, vc, part, seq_len, pos_dev,
                                                            layer_off, nkh, group, scale, grid.x);
    return hipGetLastError();
}

template <uint32_t HD>
static hipError_t launch_chunk_hd(dim3 grid, hipStream_t s, const float *q, const uint16_t *kc,
                                  const uint16_t *vc, float *part, uint32_t seq_len,
                                  const uint32_t *pos_dev, uint64_t layer_off, uint32_t nkh,
                                  uint32_t group, float scale) {
#define VBS_ATTN_G(GG) \
    return launch_chunk_t<HD, GG>(grid, s, q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, group, scale)
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
    const uint32_t n_chunks = (seq_len + kChunk - 1u) / kChunk;
    if (!part) part = (float *)scratch(attention_partial_bytes(seq_len, nqh, hd), s);
    if (!part) return hipErrorOutOfMemory;
    const dim3 grid(n_chunks, nkh);
    const bool fast = (hd == 32u || hd == 64u || hd == 128u) && group <= 8u &&
                      ((uintptr_t)q & 15u) == 0 && ((uintptr_t)kc & 15u) == 0 &&
                      ((uintptr_t)vc & 15u) == 0;
    hipError_t e;
    if (fast) {
        switch (hd) {
            case 32: e = launch_chunk_hd<32>(grid, s, q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, group, scale); break;
            case 64: e = launch_chunk_hd<64>(grid, s, q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, group, scale); break;
            default: e = launch_chunk_hd<128>(grid, s, q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, group, scale); break;
        }
    } else {
        const size_t lds = ((size_t)group * hd + (size_t)group * kChunk +
                            (size_t)(256u / hd) * group * hd) * sizeof(float);
        k_attn_partial<<<grid, 256, lds, s>>>(q, kc, vc, part, seq_len, pos_dev, layer_off, nkh,
                                              hd, group, scale, n_chunks);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
    const size_t mlds = ((size_t)n_chunks + 256u) * sizeof(float);
    k_attn_merge<<<nqh, 256, mlds, s>>>(part, out, hd, n_chunks, n_chunks, pos_dev);
    return hipGetLastError();
}

}  // namespace vbs
