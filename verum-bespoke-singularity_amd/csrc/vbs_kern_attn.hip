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
// The chunk length follows the sequence (attn_split) so that about
// kTargetWgs (512) workgroups of the vector-ALU kernels, or kMfmaTargetWgs
// (vbs_attn_common.h) of the matrix-core kernel, share it at any length. A second kernel merges (a hand-off
// inside one kernel, through device-scope stores, loads and an arrival
// count, measured slower than the kernel boundary on this part).
//
// Fast chunk kernel (head_dim 32/64/128, group <= 8): four waves; lanes of a
// wave split a position's head_dim into 8-element slices (16-byte K and V
// loads), so one wave step covers 64/(head_dim/8) positions ("slots"). A wave
// loads four steps at a time (up to four such batches; the next batch's K
// rows are requested once the scores are taken, its V rows once they are
// used). q lives in registers (the lane's slice for every q head of the
// group); the partial dot of a slice is an fp32 FMA chain and the slices are
// added with DPP row operations, which leaves every lane of a slot with its
// scores. Each slot keeps a running softmax state (max, sum, acc) over its
// positions; the slots of a wave are combined with lane shuffles and the four
// waves in one LDS pass. Scores are fp32 dots of exactly converted f16
// keys instead of the reference's double dot: a relative difference of order
// 1e-7 in each score, far inside the 1e-4 the reference's own backend test
// allows (src/vbs_backend_test.c:617-625).
//
// Other shapes use the generic chunk kernel (double dot, one position per
// four threads).
#include "vbs_attn_common.h"
#include "vbs_dev_common.h"
#include "vbs_internal.h"

namespace vbs {

constexpr uint32_t kChunk = 64;  // positions per workgroup of the generic kernel
constexpr uint32_t kMaxGroup = 16;
constexpr uint32_t kTargetWgs = 512;      // workgroups the vector-ALU split aims for

// (attn_split, the matrix-core split's constants and fast_exp: vbs_attn_common.h)
// Chunks per kv head of any split of a sequence of at most max_seq (every
// len >= 64 or len >= seq * nkh / target, target <= kMfmaTargetWgs).
inline uint32_t attn_max_chunks(uint32_t max_seq, uint32_t nkh) {
    const uint32_t a = (kMfmaTargetWgs + nkh - 1u) / nkh, b = (max_seq + 63u) / 64u;
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


// Shape of the fast kernel: four waves; LPP lanes per position (8 head dims
// each), so a wave step covers PPW positions ("slots"); a wave loads kSteps
// steps at a time and runs up to kBatches such batches.
constexpr uint32_t kWaves = 4, kSteps = 4, kBatches = 4;
template <uint32_t HD>
struct ChunkShape {
    static constexpr uint32_t LPP = HD / 8, PPW = 64 / LPP, GRAN = kWaves * PPW,
                              LMAX = kBatches * kSteps * GRAN;
};

template <uint32_t HD, uint32_t GMAX>
__global__ __launch_bounds__(64 * kWaves) void k_attn_chunk(
    const float *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc,
    float *__restrict__ part, uint32_t seq_len, const uint32_t *__restrict__ pos_dev,
    uint64_t layer_off, uint32_t nkh, uint32_t group, float scale, uint32_t stride_chunks) {
    using S = ChunkShape<HD>;
    constexpr uint32_t LPP = S::LPP, PPW = S::PPW;
    extern __shared__ __align__(16) uint8_t chunk_lds[];
    float *red = reinterpret_cast<float *>(chunk_lds);  // [kWaves][group][HD] acc per wave
    __shared__ float sm[kWaves][GMAX], sl[kWaves][GMAX], sf[kWaves][GMAX];

    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, t = threadIdx.x;
    const uint32_t wave = t >> 6, lane = t & 63u;
    const uint32_t slot = lane / LPP, c = lane % LPP;
    if (pos_dev) seq_len = pos_dev[0] + 1u;  // graph replay: the device holds the position
    const AttnSplit sp = attn_split(seq_len, nkh, S::GRAN, S::LMAX, kTargetWgs);
    if (chunk >= sp.n) return;  // past the sequence (the grid covers the longest split)
    const uint32_t s0 = chunk * sp.len;
    const uint32_t valid = min(sp.len, seq_len - s0);
    const uint32_t pw = sp.len / kWaves, ns = pw / PPW;  // positions and steps per wave
    const uint32_t nb = (ns + kSteps - 1u) / kSteps;     // batches of kSteps steps
    const uint64_t rstride = (uint64_t)nkh * HD;
    const uint64_t base = layer_off + (uint64_t)s0 * rstride + (uint64_t)kvh * HD + 8u * c;

    // position of step i of this lane's slot; positions past the chunk re-read
    // its last row and are masked (score -inf, v zero)
    auto pos_of = [&](uint32_t i) { return wave * pw + i * PPW + slot; };
    uint4 kr[kSteps], vr[kSteps];
    auto load_k = [&](uint32_t bi) {
#pragma unroll
        for (uint32_t b = 0; b < kSteps; b++)
            if (bi * kSteps + b < ns)
                kr[b] = *reinterpret_cast<const uint4 *>(
                    kc + base + (uint64_t)min(pos_of(bi * kSteps + b), valid - 1u) * rstride);
    };
    auto load_v = [&](uint32_t bi) {
#pragma unroll
        for (uint32_t b = 0; b < kSteps; b++) {
            const uint32_t i = bi * kSteps + b;
            if (i < ns) {
                vr[b] = *reinterpret_cast<const uint4 *>(
                    vc + base + (uint64_t)min(pos_of(i), valid - 1u) * rstride);
                if (pos_of(i) >= valid) vr[b] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
    };
    load_k(0);
    load_v(0);
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

    // per slot and q head: running max m, sum l of e^(s - m), acc of e^(s - m) v
    float m[GMAX], l[GMAX], acc[GMAX][8];
#pragma unroll
    for (uint32_t g = 0; g < GMAX; g++) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) acc[g][j] = 0.f;
    }
    for (uint32_t bi = 0; bi < nb; bi++) {
        // scores: every lane of a slot holds its position's scores
        float sc[kSteps][GMAX];
#pragma unroll
        for (uint32_t b = 0; b < kSteps; b++) {
            const uint32_t i = bi * kSteps + b;
            const bool in = i < ns && pos_of(i) < valid;
            float kf[8];
            if (i < ns) {
                const uint32_t kw[4] = {kr[b].x, kr[b].y, kr[b].z, kr[b].w};
#pragma unroll
                for (uint32_t j = 0; j < 8; j++) kf[j] = hcvt(kw[j >> 1] >> (16u * (j & 1u)));
            }
#pragma unroll
            for (uint32_t g = 0; g < GMAX; g++) {
                float p = 0.f;
                if (i < ns) {
#pragma unroll
                    for (uint32_t j = 0; j < 8; j++) p = fmaf(qv[g][j], kf[j], p);
                    p = group_sum<LPP>(p);
                }
                sc[b][g] = in ? __fmul_rn(p, scale) : -INFINITY;
            }
        }
        if (bi + 1u < nb) load_k(bi + 1u);  // the K registers are free again
#pragma unroll
        for (uint32_t g = 0; g < GMAX; g++) {
            float mb = sc[0][g];
#pragma unroll
            for (uint32_t b = 1; b < kSteps; b++) mb = fmaxf(mb, sc[b][g]);
            const float mn = fmaxf(m[g], mb);
            const float r = m[g] == -INFINITY ? 0.f : fast_exp(__fsub_rn(m[g], mn));
            l[g] *= r;
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) acc[g][j] *= r;
#pragma unroll
            for (uint32_t b = 0; b < kSteps; b++) {
                if (bi * kSteps + b < ns) {
                    const float e = sc[b][g] == -INFINITY ? 0.f : fast_exp(__fsub_rn(sc[b][g], mn));
                    const uint32_t vw[4] = {vr[b].x, vr[b].y, vr[b].z, vr[b].w};
                    l[g] += e;
#pragma unroll
                    for (uint32_t j = 0; j < 8; j++)
                        acc[g][j] = fmaf(e, hcvt(vw[j >> 1] >> (16u * (j & 1u))), acc[g][j]);
                }
            }
            m[g] = mn;
        }
        if (bi + 1u < nb) load_v(bi + 1u);
    }

    // ---- the wave's slots combined (lanes of equal c across slots): M = max m,
    // weights e^(m - M) (0 for an empty slot), then sums; every slot ends with
    // the totals and slot 0 stores them
#pragma unroll
    for (uint32_t g = 0; g < GMAX; g++) {
        float M = m[g];
#pragma unroll
        for (uint32_t off = LPP; off < 64u; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        const float f = m[g] == -INFINITY ? 0.f : fast_exp(__fsub_rn(m[g], M));
        float L = l[g] * f, a[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) a[j] = acc[g][j] * f;
#pragma unroll
        for (uint32_t off = LPP; off < 64u; off <<= 1) {
            L += __shfl_xor(L, off, 64);
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) a[j] += __shfl_xor(a[j], off, 64);
        }
        if (g < group && slot == 0) {
            float *dst = red + ((wave * group + g) * HD + 8u * c);
            reinterpret_cast<float4 *>(dst)[0] = make_float4(a[0], a[1], a[2], a[3]);
            reinterpret_cast<float4 *>(dst)[1] = make_float4(a[4], a[5], a[6], a[7]);
            if (c == 0) {
                sm[wave][g] = M;
                sl[wave][g] = L;
            }
        }
    }
    __syncthreads();

    // ---- combine the waves: M = max m_w, weights e^(m_w - M) (0 for empty waves)
    if (t < kWaves * GMAX) {
        const uint32_t w = t / GMAX, g = t % GMAX;
        if (g < group) {
            float M = sm[0][g];
#pragma unroll
            for (uint32_t i = 1; i < kWaves; i++) M = fmaxf(M, sm[i][g]);
            const float mw = sm[w][g];
            sf[w][g] = mw == -INFINITY ? 0.f : fast_exp(__fsub_rn(mw, M));
        }
    }
    __syncthreads();
    float *const pk = part + (uint64_t)kvh * group * stride_chunks * (HD + 2u);
    for (uint32_t i = t; i < group * HD; i += 64u * kWaves) {
        const uint32_t g = i / HD, d = i % HD;
        float a = 0.f;
#pragma unroll
        for (uint32_t w = 0; w < kWaves; w++) a = fmaf(red[(w * group + g) * HD + d], sf[w][g], a);
        float *dst = pk + ((uint64_t)g * stride_chunks + chunk) * (HD + 2u);
        dst[2u + d] = a;
        if (d == 0) {
            float M = sm[0][g], L = 0.f;
#pragma unroll
            for (uint32_t w = 1; w < kWaves; w++) M = fmaxf(M, sm[w][g]);
#pragma unroll
            for (uint32_t w = 0; w < kWaves; w++) L = fmaf(sl[w][g], sf[w][g], L);
            dst[0] = M;
            dst[1] = L;
        }
    }
}

// ---- matrix-core chunk kernel (head_dim 128, group <= 8) ------------------------
// One wave per chunk of up to kMfmaTiles tiles of 32 positions, on
// v_mfma_f32_16x16x32_f16:
// * scores, S = K q^T: A = 16 positions x 32 head dims of K (the cache's f16,
//   exact), B = 32 dims x 16 columns: column n holds q' of head n & 7, its
//   f16 hi part for n < 8 and lo part (q' - hi) for n >= 8, with q' = q 2^s_h
//   scaled so that the head's largest |q| lies in [2^14, 2^15). Columns n and
//   n + 8 add up (a DPP row rotation) to the fp32 dot of k with q' to ~2^-22;
//   the score is that times 2^-s_h * scale. Lane (n, g) then holds the scores
//   of head n & 7 at positions 16 hf + 4 g + r (hf, r: the two 16-position
//   halves of the tile, the four D rows).
// * online softmax per head over the tiles (running max m, sum l).
// * P V: A = P, rows n: e^(s - m) of head n & 7 (f16 hi for n < 8, lo for
//   n >= 8), k slots = exactly the lane's own eight positions; B = V with the
//   same k slots and column n of dim tile t standing for head dim 8 n + t, so
//   lane (n, g) takes its B operands from eight 16-byte V rows it loaded
//   itself (dims 8n..8n+7 of its eight positions) and no transpose is needed.
//   D rows 0-7 (hi) and 8-15 (lo) add up at the end.
// The chunk's (m, l, acc) go to the same partials as the vector-ALU kernel.
// The most chunks the matrix-core split gives any sequence of at most max_seq
// positions: the chunk count grows with the sequence while the chunk length
// stays put, so the maximum lies at the longest sequence of some chunk length
// (32 k positions for sequences of at most 32 k * target / nkh, the last
// length open-ended) or at max_seq itself. The chunk launch's grid: a graph
// replay reads the position on the device, so the grid covers every
// position up to max_seq, and workgroups beyond the current split exit at
// once (each costs dispatch time, so the grid is no larger than this).
inline uint32_t mfma_grid_chunks(uint32_t max_seq, uint32_t nkh, uint32_t target = kMfmaTargetWgs) {
    uint32_t best = 0;
    for (uint32_t k = 1; k <= kMfmaTiles; k++) {
        const uint64_t hi = k < kMfmaTiles ? (uint64_t)kMfmaGran * k * target / nkh : max_seq;
        const uint32_t s = (uint32_t)(hi < max_seq ? hi : max_seq);
        if (s == 0) continue;
        const uint32_t c = attn_split(s, nkh, kMfmaGran, kMfmaLmax, target).n;
        best = c > best ? c : best;
    }
    return best;
}

typedef _Float16 ah8 __attribute__((ext_vector_type(8)));
typedef float af4 __attribute__((ext_vector_type(4)));
typedef uint32_t au4 __attribute__((ext_vector_type(4)));

// One wave's chunk: positions [s0, s0 + valid) of kv head kvh (valid >= 1,
// nt tiles of 32) against the q heads of its group. On return every lane
// holds, for head n & 7 of its lane n = lane & 15, the chunk maximum m and
// l = sum e^(s - m); and a[dt][r] = the sum of e^(s - m) v[8 n + dt] of head
// 4 (lane >> 4) + r (rows hi + lo added; lane groups 0 and 1 carry them).
__device__ __forceinline__ void attn_mfma_wave(const float *__restrict__ q,
                                               const uint16_t *__restrict__ kc,
                                               const uint16_t *__restrict__ vc, uint64_t layer_off,
                                               uint32_t s0, uint32_t valid, uint32_t nt,
                                               uint32_t nkh, uint32_t kvh, uint32_t group,
                                               float scale, uint32_t lane, float &m_out,
                                               float &l_out, float (&a)[8][4]) {
    constexpr uint32_t HD = 128;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint64_t rstride = (uint64_t)nkh * HD;
    const uint64_t base = layer_off + (uint64_t)s0 * rstride + (uint64_t)kvh * HD;

    // ---- tile loads: K rows (A operand: position 16 hf + n, dims 32 kk + 8 g ..),
    // V rows (position p_j of this lane group, dims 8 n ..); positions past the
    // chunk re-read its last row and are masked
    auto pos_of = [&](uint32_t t, uint32_t j) { return 32u * t + 16u * (j >> 2) + 4u * g + (j & 3u); };
    au4 kr[2][4], vr[8];
    auto load_k = [&](uint32_t t) {
#pragma unroll
        for (uint32_t hf = 0; hf < 2; hf++) {
            const uint32_t p = min(32u * t + 16u * hf + n, valid - 1u);
#pragma unroll
            for (uint32_t kk = 0; kk < 4; kk++)
                kr[hf][kk] = *reinterpret_cast<const au4 *>(kc + base + (uint64_t)p * rstride +
                                                            32u * kk + 8u * g);
        }
    };
    auto load_v = [&](uint32_t t) {
#pragma unroll
        for (uint32_t j = 0; j < 8; j++)
            vr[j] = *reinterpret_cast<const au4 *>(
                vc + base + (uint64_t)min(pos_of(t, j), valid - 1u) * rstride + 8u * n);
    };
    // ---- q' of head n & 7 (heads past the group repeat head 0 and are not stored)
    const uint32_t h = n & 7u, hq = h < group ? h : 0u;
    float qv[4][8];
    {
        const float4 *qp = reinterpret_cast<const float4 *>(q + ((uint64_t)kvh * group + hq) * HD);
#pragma unroll
        for (uint32_t kk = 0; kk < 4; kk++) {
            const float4 a = qp[(32u * kk + 8u * g) / 4u], b = qp[(32u * kk + 8u * g) / 4u + 1u];
            qv[kk][0] = a.x; qv[kk][1] = a.y; qv[kk][2] = a.z; qv[kk][3] = a.w;
            qv[kk][4] = b.x; qv[kk][5] = b.y; qv[kk][6] = b.z; qv[kk][7] = b.w;
        }
    }
    // the first tile's K and V rows go out with q's loads: one memory round
    // trip before the first MMA instead of two (the scheduler may not sink
    // them below q's arithmetic)
    load_k(0);
    load_v(0);
    __builtin_amdgcn_sched_barrier(0);
    float amax = 0.f;
#pragma unroll
    for (uint32_t kk = 0; kk < 4; kk++)
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(qv[kk][j]));
    amax = fmaxf(amax, lane_xor<16>(amax));
    amax = fmaxf(amax, lane_xor<32>(amax));
    int e2 = 0;
    (void)frexpf(amax, &e2);  // amax < 2^e2
    const int sq = amax > 0.f ? 15 - e2 : 0;
    const float csc = ldexpf(scale, -sq);
    ah8 Qb[4];
#pragma unroll
    for (uint32_t kk = 0; kk < 4; kk++)
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) {
            const float x = ldexpf(qv[kk][j], sq);
            const _Float16 hi = (_Float16)x;
            Qb[kk][j] = n < 8u ? hi : (_Float16)(x - (float)hi);
        }


    float m = -INFINITY, l = 0.f;
    af4 acc[8];
#pragma unroll
    for (uint32_t t = 0; t < 8; t++) acc[t] = af4{0.f, 0.f, 0.f, 0.f};
    auto tile = [&](uint32_t t) {
        af4 S[2];
#pragma unroll
        for (uint32_t hf = 0; hf < 2; hf++) {
            S[hf] = af4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t kk = 0; kk < 4; kk++)
                S[hf] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(ah8, kr[hf][kk]),
                                                              Qb[kk], S[hf], 0, 0, 0);
        }
        if (t + 1u < nt) load_k(t + 1u);  // the K registers are free again
        // scores of positions p_j: hi + lo columns (lane n and n ^ 8), scaled, masked
        float sc[8], mt = -INFINITY;
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) {
            const float v = S[j >> 2][j & 3u];
            const float w = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                              0, __builtin_bit_cast(int, v), 0x128,
                                                              0xF, 0xF, false));  // row_ror:8
            sc[j] = pos_of(t, j) < valid ? __fmul_rn(w, csc) : -INFINITY;
            mt = fmaxf(mt, sc[j]);
        }
        mt = fmaxf(mt, lane_xor<16>(mt));
        mt = fmaxf(mt, lane_xor<32>(mt));
        const float mn = fmaxf(m, mt);
        const float rs = m == -INFINITY ? 0.f : fast_exp(__fsub_rn(m, mn));
        m = mn;
        l *= rs;
        ah8 P;
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) {
            const float e = sc[j] == -INFINITY ? 0.f : fast_exp(__fsub_rn(sc[j], mn));
            l += e;
            const _Float16 hi = (_Float16)e;
            P[j] = n < 8u ? hi : (_Float16)(e - (float)hi);
        }
        // D rows 4 g + r of the P V accumulators belong to head (4 g + r) & 7
        float rsr[4];
#pragma unroll
        for (uint32_t r = 0; r < 4; r++) rsr[r] = __shfl(rs, (4u * g + r) & 7u, 64);
#pragma unroll
        for (uint32_t dt = 0; dt < 8; dt++) {
            // B: element dt (head dim 8 n + dt) of each of the lane's eight V rows
            const uint32_t sel = (dt & 1u) ? 0x07060302u : 0x05040100u;
            au4 b;
#pragma unroll
            for (uint32_t i = 0; i < 4; i++)
                b[i] = __builtin_amdgcn_perm(vr[2 * i + 1][dt >> 1], vr[2 * i][dt >> 1], sel);
            af4 a = acc[dt];
#pragma unroll
            for (uint32_t r = 0; r < 4; r++) a[r] *= rsr[r];
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(P, __builtin_bit_cast(ah8, b), a, 0, 0, 0);
        }
        if (t + 1u < nt) load_v(t + 1u);
    };
    tile(0);  // peeled, so that its loads and uses share the entry block with q's
    for (uint32_t t = 1; t < nt; t++) tile(t);

    // ---- the chunk's partial: l summed over the lane groups of a head, rows
    // hi + lo of acc (lane groups g and g + 2), stored by lane groups 0 and 1
    l += lane_xor<16>(l);
    l += lane_xor<32>(l);
#pragma unroll
    for (uint32_t dt = 0; dt < 8; dt++)
#pragma unroll
        for (uint32_t r = 0; r < 4; r++) a[dt][r] = acc[dt][r] + lane_xor<32>(acc[dt][r]);
    m_out = m;
    l_out = l;
}

__global__ __launch_bounds__(64) void k_attn_mfma(const float *__restrict__ q,
                                                  const uint16_t *__restrict__ kc,
                                                  const uint16_t *__restrict__ vc,
                                                  float *__restrict__ part, uint32_t seq_len,
                                                  const uint32_t *__restrict__ pos_dev,
                                                  uint64_t layer_off, uint32_t nkh, uint32_t group,
                                                  float scale, uint32_t stride_chunks,
                                                  uint32_t q_bstride, uint64_t kv_bstride,
                                                  uint64_t part_bstride, uint32_t target,
                                                  uint32_t *__restrict__ clear, uint32_t nclear,
                                                  uint32_t clear_stride) {
    constexpr uint32_t HD = 128;
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, lane = threadIdx.x, bz = blockIdx.z;
    const uint32_t n = lane & 15u, g = lane >> 4;
    // the merging launch that follows (k_mvl_attn) starts from cleared flags
    if (clear && chunk == 0u && kvh == 0u && bz == 0u)
        for (uint32_t i = lane; i < nclear; i += 64u) clear[(uint64_t)i * clear_stride] = 0u;
    // sequence bz of a batch: its q, caches, position and partials
    q += (uint64_t)bz * q_bstride;
    kc += bz * kv_bstride;
    vc += bz * kv_bstride;
    part += bz * part_bstride;
    if (pos_dev) seq_len = pos_dev[bz] + 1u;  // graph replay: the device holds the position
    const AttnSplit sp = attn_split(seq_len, nkh, kMfmaGran, kMfmaLmax, target);
    if (chunk >= sp.n) return;  // past the sequence (the grid covers the longest split)
    const uint32_t s0 = chunk * sp.len, valid = min(sp.len, seq_len - s0);
    float m, l, a[8][4];
    attn_mfma_wave(q, kc, vc, layer_off, s0, valid, sp.len / kMfmaGran, nkh, kvh, group, scale,
                   lane, m, l, a);
    float *const pk = part + (uint64_t)kvh * group * stride_chunks * (HD + 2u);
    if (g < 2u) {
#pragma unroll
        for (uint32_t r = 0; r < 4; r++) {
            const uint32_t hh = 4u * g + r;
            if (hh < group) {
                float *dst = pk + ((uint64_t)hh * stride_chunks + chunk) * (HD + 2u) + 2u + 8u * n;
#pragma unroll
                for (uint32_t i = 0; i < 4; i++)
                    reinterpret_cast<float2 *>(dst)[i] = make_float2(a[2 * i][r], a[2 * i + 1][r]);
            }
        }
    }
    if (g == 0 && n < group) {
        float *dst = pk + ((uint64_t)n * stride_chunks + chunk) * (HD + 2u);
        dst[0] = m;
        dst[1] = l;
    }
}

// ---- merge of the chunks -------------------------------------------------------
// One workgroup of kMergeThreads per q head; every global load is issued up
// front: thread (d, slice) loads acc_c[d] of its chunks c = slice, slice + ns,
// ... and thread t also m_t and l_t. Then M = max_c m_c (block maximum),
// weights w_c = e^(m_c - M) in LDS, L = sum_c l_c w_c, and the slices'
// weighted sums are added in LDS in a fixed order.
constexpr uint32_t kMergeThreadBatch = 32;     // chunks per thread held in registers at once
constexpr uint32_t kMergeThreads = 512;  // (measured 2-8% faster than 1024 and than 256)

__global__ __launch_bounds__(kMergeThreads) void k_attn_merge(const float *__restrict__ part,
                                                    float *__restrict__ out, uint32_t hd,
                                                    uint32_t n_chunks, uint32_t stride_chunks,
                                                    const uint32_t *__restrict__ pos_dev,
                                                    uint32_t nkh, uint32_t gran, uint32_t lmax,
                                                    uint32_t target, uint32_t q_bstride,
                                                    uint64_t part_bstride) {
    extern __shared__ __align__(16) uint8_t merge_lds[];
    float *w = reinterpret_cast<float *>(merge_lds);  // [stride_chunks]
    float *sl = w + stride_chunks;                    // [kMergeThreads]
    constexpr uint32_t NW = kMergeThreads / 64u;
    __shared__ float red[2 * NW];
    const uint32_t h = blockIdx.x, t = threadIdx.x, lane = t & 63u, wave = t >> 6, bz = blockIdx.y;
    part += bz * part_bstride;  // sequence bz of a batch
    out += (uint64_t)bz * q_bstride;
    if (pos_dev) n_chunks = attn_split(pos_dev[bz] + 1u, nkh, gran, lmax, target).n;  // seq = pos + 1
    const float *ph = part + (uint64_t)h * stride_chunks * (hd + 2u);
    const uint32_t ns = kMergeThreads / hd;
    const uint32_t d = t % hd, s = t / hd;
    float av[kMergeThreadBatch];
#pragma unroll
    for (uint32_t k = 0; k < kMergeThreadBatch; k++) {
        const uint32_t c = s + k * ns;
        av[k] = (s < ns && c < n_chunks) ? ph[(uint64_t)c * (hd + 2u) + 2u + d] : 0.f;
    }
    // this thread's chunks' (m, l): c = t, t + kMergeThreads, ...; the first
    // pair is loaded with the acc values, before any reduction
    float m0 = -INFINITY, l0 = 0.f;
    if (t < n_chunks) {
        m0 = ph[(uint64_t)t * (hd + 2u)];
        l0 = ph[(uint64_t)t * (hd + 2u) + 1u];
    }
    float M = m0;
    for (uint32_t c = t + kMergeThreads; c < n_chunks; c += kMergeThreads)
        M = fmaxf(M, ph[(uint64_t)c * (hd + 2u)]);
    M = wave_max(M);
    if (lane == 0) red[wave] = M;
    __syncthreads();
    M = red[0];
    for (uint32_t i = 1; i < NW; i++) M = fmaxf(M, red[i]);
    float L = 0.f;
    if (t < n_chunks) {
        const float wc = m0 == -INFINITY ? 0.f : fast_exp(__fsub_rn(m0, M));
        w[t] = wc;
        L = fmaf(l0, wc, L);
    }
    for (uint32_t c = t + kMergeThreads; c < n_chunks; c += kMergeThreads) {
        const float *pc = ph + (uint64_t)c * (hd + 2u);
        const float mc = pc[0], wc = mc == -INFINITY ? 0.f : fast_exp(__fsub_rn(mc, M));
        w[c] = wc;
        L = fmaf(pc[1], wc, L);
    }
    L = wave_sum(L);
    if (lane == 0) red[NW + wave] = L;
    __syncthreads();
    L = 0.f;
    for (uint32_t i = 0; i < NW; i++) L += red[NW + i];
    float a = 0.f;
    if (s < ns) {
#pragma unroll
        for (uint32_t k = 0; k < kMergeThreadBatch; k++) {
            const uint32_t c = s + k * ns;
            if (c < n_chunks) a = fmaf(av[k], w[c], a);
        }
        for (uint32_t c = s + kMergeThreadBatch * ns; c < n_chunks; c += ns)
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

// Merge for head_dim 128 (the matrix-core chunk kernel's partials): one
// workgroup of four waves per q head (grid y: the sequences of a batch). Every
// wave forms M, L and the chunk weights itself from all chunks' (m, l); wave r
// takes residue r of the chunks (vbs_attn_common.h), its acc rows loaded at
// once, and one LDS pass adds the four sums in order. No loads wait on a
// reduction and one barrier ends it (the general merge above has four).
__global__ __launch_bounds__(64 * kMergeRes) void k_attn_merge_h128(
    const float *__restrict__ part, float *__restrict__ out, uint32_t stride_chunks,
    const uint32_t *__restrict__ pos_dev, uint32_t seq_len, uint32_t nkh, uint32_t q_bstride,
    uint64_t part_bstride, uint32_t target) {
    __shared__ float2 red[kMergeRes][64];
    const uint32_t h = blockIdx.x, bz = blockIdx.y, lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    part += bz * part_bstride;
    out += (uint64_t)bz * q_bstride;
    if (pos_dev) seq_len = pos_dev[bz] + 1u;  // seq = pos + 1
    const uint32_t nc = mfma_chunks(seq_len, nkh, target);
    const float *ph = part + (uint64_t)h * stride_chunks * kPartRow;
    float2 av[kMergeBatch];
    merge_residue_load(ph, nc, wave, lane, av);  // with the (m, l) loads: one round trip
    const MergeStats st = merge_stats(ph, nc, lane, merge_ml_load(ph, nc, lane));
    red[wave][lane] = merge_residue_sum(ph, nc, st, wave, lane, av);
    __syncthreads();
    if (wave == 0) {
        float2 a[kMergeRes];
#pragma unroll
        for (uint32_t r = 0; r < kMergeRes; r++) a[r] = red[r][lane];
        *reinterpret_cast<float2 *>(out + (uint64_t)h * 128u + 2u * lane) = merge_finish(a, st.L);
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
    const size_t lds = (size_t)kWaves * group * HD * sizeof(float);
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
    if (!part) {
        hipError_t why;
        part = (float *)rt_scratch(attention_partial_bytes(seq_len, nqh, nkh, hd), s, &why);
        if (!part) return why;
    }
    const bool fast = (hd == 32u || hd == 64u || hd == 128u) && group <= 8u &&
                      ((uintptr_t)q & 15u) == 0 && ((uintptr_t)kc & 15u) == 0 &&
                      ((uintptr_t)vc & 15u) == 0;
    hipError_t e;
    uint32_t gran = kChunk, lmax = kChunk, target = kTargetWgs;
    const dim3 grid(stride, nkh);
    if (fast && hd == 128u) {
        k_attn_mfma<<<dim3(mfma_grid_chunks(seq_len, nkh), nkh), 64, 0, s>>>(
            q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, group, scale, stride, 0u, 0ull, 0ull,
            kMfmaTargetWgs, nullptr, 0u, 0u);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        k_attn_merge_h128<<<nqh, 64 * kMergeRes, 0, s>>>(part, out, stride, pos_dev, seq_len, nkh,
                                                            0u, 0ull, kMfmaTargetWgs);
        return hipGetLastError();
    } else if (fast && hd == 32u) {
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
    const uint32_t n_chunks = attn_split(seq_len, nkh, gran, lmax, target).n;
    const size_t mlds = ((size_t)stride + kMergeThreads) * sizeof(float);
    k_attn_merge<<<nqh, kMergeThreads, mlds, s>>>(part, out, hd, n_chunks, stride, pos_dev, nkh, gran,
                                                  lmax, target, 0u, 0ull);
    return hipGetLastError();
}

uint32_t attention_chunk_stride(uint32_t max_seq, uint32_t nkh) { return attn_max_chunks(max_seq, nkh); }

// The matrix-core chunk launch alone (head_dim 128, group <= 8), for a merge
// done by the launch that follows it (k_mvl_attn): the partials at part with
// attention_chunk_stride(seq_len, nkh) chunks per q head, and the words
// clear[i stride], i < nclear, zeroed for that launch's exchange.
hipError_t launch_attention_chunks(const float *q, const uint16_t *kc, const uint16_t *vc,
                                   uint32_t seq_len, const uint32_t *pos_dev, float *part,
                                   uint64_t layer_off, uint32_t nqh, uint32_t nkh, uint32_t hd,
                                   float scale, uint32_t *clear, uint32_t nclear, uint32_t stride,
                                   hipStream_t s) {
    if (seq_len == 0 || nkh == 0 || nqh % nkh != 0 || hd != 128u || nqh / nkh > 8u || !part ||
        ((uintptr_t)q & 15u) || ((uintptr_t)kc & 15u) || ((uintptr_t)vc & 15u))
        return hipErrorNotSupported;
    k_attn_mfma<<<dim3(mfma_grid_chunks(seq_len, nkh), nkh), 64, 0, s>>>(
        q, kc, vc, part, seq_len, pos_dev, layer_off, nkh, nqh / nkh, scale, attn_max_chunks(seq_len, nkh),
        0u, 0ull, 0ull, kMfmaTargetWgs, clear, nclear, stride);
    return hipGetLastError();
}

bool attn_mfma_batch_fits(const float *q, const uint16_t *kc, const uint16_t *vc, uint32_t nqh,
                          uint32_t nkh, uint32_t hd, uint32_t q_stride, uint64_t kv_stride) {
    return nkh != 0u && nqh % nkh == 0u && hd == 128u && nqh / nkh <= 8u && ((uintptr_t)q & 15u) == 0 &&
           ((uintptr_t)kc & 15u) == 0 && ((uintptr_t)vc & 15u) == 0 && (q_stride % 4u) == 0 &&
           (kv_stride % 8u) == 0;
}

hipError_t launch_attention_batch(const float *q, const uint16_t *kc, const uint16_t *vc,
                                  float *out, uint32_t max_seq, const uint32_t *pos_dev,
                                  float *part, uint64_t layer_off, uint32_t nqh, uint32_t nkh,
                                  uint32_t hd, float scale, uint32_t batch, uint32_t q_stride,
                                  uint64_t kv_stride, hipStream_t s) {
    if (batch == 0 || !part || !pos_dev) return hipErrorInvalidValue;
    if (!out && !attn_mfma_batch_fits(q, kc, vc, nqh, nkh, hd, q_stride, kv_stride))
        return hipErrorNotSupported;
    if (max_seq == 0 || nkh == 0 || nqh % nkh != 0) return hipErrorInvalidValue;
    const uint64_t pstride = attention_partial_bytes(max_seq, nqh, nkh, hd) / sizeof(float);
    const uint32_t group = nqh / nkh;
    const bool mfma = attn_mfma_batch_fits(q, kc, vc, nqh, nkh, hd, q_stride, kv_stride);
    if (!mfma) {  // one sequence at a time through the single-sequence path
        for (uint32_t b = 0; b < batch; b++) {
            const hipError_t e = launch_attention(q + (uint64_t)b * q_stride, kc + b * kv_stride,
                                                  vc + b * kv_stride, out + (uint64_t)b * q_stride,
                                                  max_seq, pos_dev + b, part + b * pstride, layer_off,
                                                  nqh, nkh, hd, scale, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const uint32_t stride = attn_max_chunks(max_seq, nkh), target = attn_batch_target(batch);
    k_attn_mfma<<<dim3(mfma_grid_chunks(max_seq, nkh, target), nkh, batch), 64, 0, s>>>(
        q, kc, vc, part, max_seq, pos_dev, layer_off, nkh, group, scale, stride, q_stride, kv_stride,
        pstride, target, nullptr, 0u, 0u);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !out) return e;  // (no out: the caller merges the partials itself)
    k_attn_merge_h128<<<dim3(nqh, batch), 64 * kMergeRes, 0, s>>>(part, out, stride, pos_dev,
                                                                     max_seq, nkh, q_stride, pstride,
                                                                     target);
    return hipGetLastError();
}

}  // namespace vbs
