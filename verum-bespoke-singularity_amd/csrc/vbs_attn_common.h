// vbs_attn_common.h — the sequence split of split-sequence attention and the
// head_dim-128 merge of its partial results (vbs_kern_attn.hip).
//
// Partials: for q head h and chunk c, at part + (h * stride + c) * 130
// floats: m (the chunk's maximum score), l (sum of e^(s - m)) and acc[128]
// (sum of e^(s - m) v). Reference: the online softmax of vbs_host_attention
// (src/vbs_host_math.h:170-209), merged by log-sum-exp rescaling:
// out = sum_c acc_c e^(m_c - M) / sum_c l_c e^(m_c - M), M = max_c m_c.
#pragma once

#include "vbs_dev_common.h"

namespace vbs {

// One-wave workgroups the matrix-core split aims for per sequence. The chunk
// kernel holds 192 registers (157 VGPRs and the MFMA accumulators): two waves
// per SIMD, 2048 on the chip at once. At 70B, batch 8, a target of 1024 made
// 5504 of them (2.7 rounds of waves), 640 makes 4160 (2.03). Measured chunk +
// merge with 640 against 1024: 70B batch 8 51.2 against 52.3-55.7 us, 70B
// batch 1 12.9 against 13.2-13.5 us, 7B batch 1 8.3 either way.
constexpr uint32_t kMfmaTargetWgs = 640;
constexpr uint32_t kMfmaGran = 32, kMfmaTiles = 8, kMfmaLmax = kMfmaGran * kMfmaTiles;
// A batch of sequences in one chunk launch (grid z) aims for one round of the
// 2048 resident one-wave workgroups across the batch: at most 640 per
// sequence, 2048 / batch from three sequences on (70B, batch 8: 256 per
// sequence, 32 chunks of 256 positions per kv head at 8192 positions).
constexpr uint32_t kMfmaWaveSlots = 2048;
__host__ __device__ inline uint32_t attn_batch_target(uint32_t batch) {
    const uint32_t t = kMfmaWaveSlots / (batch ? batch : 1u);
    return t < kMfmaTargetWgs ? t : kMfmaTargetWgs;
}

// Sequence split: chunks of `len` positions (a multiple of gran, at most lmax)
// sized so that about `target` workgroups cover seq x nkh; n chunks per kv
// head. The chunk kernel, the merge and the host compute it identically.
struct AttnSplit {
    uint32_t len, n;
};
__host__ __device__ inline AttnSplit attn_split(uint32_t seq, uint32_t nkh, uint32_t gran,
                                                uint32_t lmax, uint32_t target) {
    const uint32_t per = (uint32_t)(((uint64_t)seq * nkh + target - 1u) / target);
    uint32_t len = (per + gran - 1u) / gran * gran;
    len = len < gran ? gran : len > lmax ? lmax : len;
    return {len, (seq + len - 1u) / len};
}
// Chunks per kv head of the matrix-core kernel's split of `seq` positions.
__host__ __device__ inline uint32_t mfma_chunks(uint32_t seq, uint32_t nkh,
                                                uint32_t target = kMfmaTargetWgs) {
    return attn_split(seq, nkh, kMfmaGran, kMfmaLmax, target).n;
}

// e^x as 2^(x log2 e) on the hardware exponential (a few ulp; the scores
// themselves differ from the reference's double dots by ~1e-7 relative).
__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// ---- head_dim-128 merge, one wave's pieces ------------------------------------------
// The merge of q head h (partials ph = part + h * stride * 130, nc chunks)
// is M and L, then four interleaved sums, residue r taking chunks r, r + 4,
// ... in order with lane l holding head dims 2l and 2l + 1, then
// out = ((a_0 + a_1) + a_2 + a_3) / L. The four-wave merge kernel gives wave
// r residue r.
constexpr uint32_t kMergeRes = 4, kMergeBatch = 32;  // residues; chunks of one held in registers
constexpr uint32_t kPartRow = 130;                   // m, l, acc[128]

struct MergeStats {
    float M, L;
    float w_lane, w_lane64;  // the weights of chunks `lane` and `lane + 64`
};

// The (m, l) of chunks lane and lane + 64, requested together.
struct MergeMl {
    float m0, l0, m1, l1;
};
__device__ __forceinline__ MergeMl merge_ml_load(const float *ph, uint32_t nc, uint32_t lane) {
    MergeMl v;
    v.m0 = lane < nc ? ph[(uint64_t)lane * kPartRow] : -INFINITY;
    v.l0 = lane < nc ? ph[(uint64_t)lane * kPartRow + 1u] : 0.f;
    v.m1 = lane + 64u < nc ? ph[(uint64_t)(lane + 64u) * kPartRow] : -INFINITY;
    v.l1 = lane + 64u < nc ? ph[(uint64_t)(lane + 64u) * kPartRow + 1u] : 0.f;
    return v;
}
// The same loads bounded by `bound` >= nc chunk rows (all inside the
// partials) instead of by nc, so that they need not wait for the chunk count;
// merge_ml_mask then drops the chunks from nc on.
__device__ __forceinline__ MergeMl merge_ml_load_bounded(const float *ph, uint32_t bound, uint32_t lane) {
    MergeMl v;
    v.m0 = lane < bound ? ph[(uint64_t)lane * kPartRow] : -INFINITY;
    v.l0 = lane < bound ? ph[(uint64_t)lane * kPartRow + 1u] : 0.f;
    v.m1 = lane + 64u < bound ? ph[(uint64_t)(lane + 64u) * kPartRow] : -INFINITY;
    v.l1 = lane + 64u < bound ? ph[(uint64_t)(lane + 64u) * kPartRow + 1u] : 0.f;
    return v;
}
__device__ __forceinline__ MergeMl merge_ml_mask(MergeMl v, uint32_t nc, uint32_t lane) {
    if (lane >= nc) v.m0 = -INFINITY, v.l0 = 0.f;
    if (lane + 64u >= nc) v.m1 = -INFINITY, v.l1 = 0.f;
    return v;
}

// Every lane of the wave gets M and L: lane l takes chunks l, l + 64, ... in
// that order (chunks from 128 on are read here).
__device__ __forceinline__ MergeStats merge_stats(const float *ph, uint32_t nc, uint32_t lane,
                                                  const MergeMl &v) {
    MergeStats st;
    float M = fmaxf(v.m0, v.m1);
    for (uint32_t c = lane + 128u; c < nc; c += 64u) M = fmaxf(M, ph[(uint64_t)c * kPartRow]);
    st.M = wave_max(M);
    const float w0 = v.m0 == -INFINITY ? 0.f : fast_exp(__fsub_rn(v.m0, st.M));
    const float w1 = v.m1 == -INFINITY ? 0.f : fast_exp(__fsub_rn(v.m1, st.M));
    float L = 0.f;
    if (lane < nc) L = fmaf(v.l0, w0, L);
    if (lane + 64u < nc) L = fmaf(v.l1, w1, L);
    for (uint32_t c = lane + 128u; c < nc; c += 64u) {
        const float mc = ph[(uint64_t)c * kPartRow];
        const float wc = mc == -INFINITY ? 0.f : fast_exp(__fsub_rn(mc, st.M));
        L = fmaf(ph[(uint64_t)c * kPartRow + 1u], wc, L);
    }
    st.L = wave_sum(L);
    st.w_lane = lane < nc ? w0 : 0.f;
    st.w_lane64 = lane + 64u < nc ? w1 : 0.f;
    return st;
}

// Residue r: the acc rows of chunks c = r + 4 k, k < kMergeBatch, requested
// at once (lane l: head dims 2l, 2l + 1; rows from nc on, when nc is a bound
// on the chunk count rather than the count, are read and not used) ...
__device__ __forceinline__ void merge_residue_load(const float *ph, uint32_t nc, uint32_t r,
                                                   uint32_t lane, float2 av[kMergeBatch]) {
#pragma unroll
    for (uint32_t k = 0; k < kMergeBatch; k++) {
        const uint32_t c = r + kMergeRes * k;
        av[k] = c < nc ? *reinterpret_cast<const float2 *>(ph + (uint64_t)c * kPartRow + 2u + 2u * lane)
                       : make_float2(0.f, 0.f);
    }
}
// ... and their sum weighted by e^(m_c - M), accumulated in chunk order (later
// chunks of the residue read here).
__device__ __forceinline__ float2 merge_residue_sum(const float *ph, uint32_t nc, const MergeStats &st,
                                                   uint32_t r, uint32_t lane,
                                                   const float2 av[kMergeBatch]) {
    float ox = 0.f, oy = 0.f;
    auto add = [&](uint32_t c, float2 a) {
        float wc;
        if (c < 128u) {  // (a lane's weight: c is wave-uniform)
            wc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                               __builtin_bit_cast(int, c < 64u ? st.w_lane : st.w_lane64),
                                               (int)(c & 63u)));
        } else {
            const float mc = ph[(uint64_t)c * kPartRow];
            wc = mc == -INFINITY ? 0.f : fast_exp(__fsub_rn(mc, st.M));
        }
        ox = fmaf(a.x, wc, ox);
        oy = fmaf(a.y, wc, oy);
    };
#pragma unroll
    for (uint32_t k = 0; k < kMergeBatch; k++) {
        const uint32_t c = r + kMergeRes * k;
        if (c < nc) add(c, av[k]);
    }
    for (uint32_t c = r + kMergeRes * kMergeBatch; c < nc; c += kMergeRes)
        add(c, *reinterpret_cast<const float2 *>(ph + (uint64_t)c * kPartRow + 2u + 2u * lane));
    return make_float2(ox, oy);
}

// The four residues in order, scaled by 1 / L.
__device__ __forceinline__ float2 merge_finish(const float2 a[kMergeRes], float L) {
    float2 s = a[0];
#pragma unroll
    for (uint32_t r = 1; r < kMergeRes; r++) {
        s.x += a[r].x;
        s.y += a[r].y;
    }
    const float inv = __fdiv_rn(1.0f, L);
    return make_float2(__fmul_rn(s.x, inv), __fmul_rn(s.y, inv));
}

// The same merge by one wave: the four residue sums accumulated side by side
// in chunk order (each residue's chunks in its own order, as the four waves
// take them), the acc rows of B chunks requested at once (B a multiple of
// kMergeRes), then merge_finish: bit-identical to the four-wave merge.
template <uint32_t B>
__device__ __forceinline__ float2 merge_one_wave(const float *ph, uint32_t nc, uint32_t lane) {
    static_assert(B % kMergeRes == 0u, "batch");
    auto load_batch = [&](uint32_t c0, float2 av[B]) {
#pragma unroll
        for (uint32_t k = 0; k < B; k++) {
            const uint32_t c = c0 + k;
            av[k] = c < nc ? *reinterpret_cast<const float2 *>(ph + (uint64_t)c * kPartRow + 2u + 2u * lane)
                           : make_float2(0.f, 0.f);
        }
    };
    float2 av[B];
    load_batch(0u, av);
    const MergeStats st = merge_stats(ph, nc, lane, merge_ml_load(ph, nc, lane));
    float ox[kMergeRes] = {0.f, 0.f, 0.f, 0.f}, oy[kMergeRes] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t c0 = 0; c0 < nc; c0 += B) {
        if (c0) load_batch(c0, av);
#pragma unroll
        for (uint32_t k = 0; k < B; k++) {
            const uint32_t c = c0 + k, r = k % kMergeRes;  // (c0 is a multiple of kMergeRes)
            if (c < nc) {
                float wc;
                if (c < 128u) {  // (as merge_residue_sum: c is wave-uniform)
                    wc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                       __builtin_bit_cast(int, c < 64u ? st.w_lane : st.w_lane64),
                                                       (int)(c & 63u)));
                } else {
                    const float mc = ph[(uint64_t)c * kPartRow];
                    wc = mc == -INFINITY ? 0.f : fast_exp(__fsub_rn(mc, st.M));
                }
                ox[r] = fmaf(av[k].x, wc, ox[r]);
                oy[r] = fmaf(av[k].y, wc, oy[r]);
            }
        }
    }
    float2 a[kMergeRes];
#pragma unroll
    for (uint32_t r = 0; r < kMergeRes; r++) a[r] = make_float2(ox[r], oy[r]);
    return merge_finish(a, st.L);
}

}  // namespace vbs
