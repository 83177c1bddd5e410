// vbs_dev_common.h — device helpers shared by the gfx950 kernels.
//
// Block decoders here reproduce the reference dequantiser's arithmetic
// (src/vbs_dequant.c:123-333) one rounding at a time: every product and sum
// goes through an explicitly rounded intrinsic (__fmul_rn, __fadd_rn,
// __fsub_rn), so the compiler cannot fuse them into an FMA and the values are
// bit-identical to the host. The kernels' dot products may fuse freely.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vbs_half.h"

namespace vbs {

enum : int {
    kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14, kLNS8 = 40
};

template <int T> struct Geo;
template <> struct Geo<kF32> { static constexpr uint32_t E = 1, B = 4; };
template <> struct Geo<kF16> { static constexpr uint32_t E = 1, B = 2; };
template <> struct Geo<kQ4_0> { static constexpr uint32_t E = 32, B = 18; };
template <> struct Geo<kQ4_1> { static constexpr uint32_t E = 32, B = 20; };
template <> struct Geo<kQ8_0> { static constexpr uint32_t E = 32, B = 34; };
template <> struct Geo<kQ4_K> { static constexpr uint32_t E = 256, B = 144; };
template <> struct Geo<kQ6_K> { static constexpr uint32_t E = 256, B = 210; };
template <> struct Geo<kLNS8> { static constexpr uint32_t E = 32, B = 36; };

__device__ __forceinline__ uint16_t ld16(const uint8_t *p) {
    return *reinterpret_cast<const uint16_t *>(p);  // every block field is 2-B aligned
}
__device__ __forceinline__ float h2f(uint16_t h) { return vbs_h2f(h); }

// The reference's dequantiser runs on the host's SSE arithmetic, whose NaN
// results follow two rules: a NaN operand comes back quieted with its sign and
// payload (the first operand when both are NaN), and an invalid operation
// (0 x inf, inf - inf) gives the negative default NaN 0xFFC00000. The VALU
// differs on both (a subtraction adds the negated operand, so a NaN
// subtrahend changes sign; its default NaN is positive), so the block
// decoders rebuild NaN results by the host's rules: NaN scales in a GGUF block
// then dequantise to the same words as on the host.
__device__ __forceinline__ float nan_as_host(float r, float a, float b) {
    if (!__builtin_isnan(r)) return r;
    if (__builtin_isnan(a)) return vbs_half_bits_to_float(vbs_float_to_bits(a) | 0x00400000u);
    if (__builtin_isnan(b)) return vbs_half_bits_to_float(vbs_float_to_bits(b) | 0x00400000u);
    return vbs_half_bits_to_float(0xFFC00000u);
}
__device__ __forceinline__ float hmul(float a, float b) { return nan_as_host(__fmul_rn(a, b), a, b); }
__device__ __forceinline__ float hadd(float a, float b) { return nan_as_host(__fadd_rn(a, b), a, b); }
__device__ __forceinline__ float hsub(float a, float b) { return nan_as_host(__fsub_rn(a, b), a, b); }

// 6-bit scale and min of sub-block j of a Q4_K super-block
// (src/vbs_dequant.c:225-233).
__device__ __forceinline__ void q4k_scale_min(const uint8_t *s, int j, int &sc, int &mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// Exact value of element e of one block (src/vbs_dequant.c:123-333).
template <int T> __device__ __forceinline__ float deq_elem(const uint8_t *b, uint32_t e);

template <> __device__ __forceinline__ float deq_elem<kF32>(const uint8_t *b, uint32_t e) {
    return reinterpret_cast<const float *>(b)[e];
}
template <> __device__ __forceinline__ float deq_elem<kF16>(const uint8_t *b, uint32_t e) {
    return h2f(ld16(b + 2 * e));
}
template <> __device__ __forceinline__ float deq_elem<kQ4_0>(const uint8_t *b, uint32_t e) {
    float d = h2f(ld16(b));
    uint8_t byte = b[2 + (e & 15)];
    int nib = e < 16 ? (byte & 15) : (byte >> 4);
    return hmul(__fsub_rn((float)nib, 8.0f), d);
}
template <> __device__ __forceinline__ float deq_elem<kQ4_1>(const uint8_t *b, uint32_t e) {
    float d = h2f(ld16(b)), m = h2f(ld16(b + 2));
    uint8_t byte = b[4 + (e & 15)];
    int nib = e < 16 ? (byte & 15) : (byte >> 4);
    return hadd(hmul(d, (float)nib), m);
}
template <> __device__ __forceinline__ float deq_elem<kQ8_0>(const uint8_t *b, uint32_t e) {
    return hmul(h2f(ld16(b)), (float)(int8_t)b[2 + e]);
}
template <> __device__ __forceinline__ float deq_elem<kQ4_K>(const uint8_t *b, uint32_t e) {
    float d = h2f(ld16(b)), dmin = h2f(ld16(b + 2));
    int sc, mn;
    q4k_scale_min(b + 4, (int)(e >> 5), sc, mn);
    uint8_t byte = b[16 + 32 * (e >> 6) + (e & 31)];
    int nib = (e & 32) ? (byte >> 4) : (byte & 15);
    return hsub(hmul(hmul(d, (float)sc), (float)nib), hmul(dmin, (float)mn));
}
template <> __device__ __forceinline__ float deq_elem<kQ6_K>(const uint8_t *b, uint32_t e) {
    uint32_t h = e >> 7, q = (e >> 5) & 3, l = e & 31;
    int lo = (b[64 * h + 32 * (q & 1) + l] >> (q >= 2 ? 4 : 0)) & 15;
    int hi = (b[128 + 32 * h + l] >> (2 * q)) & 3;
    int v = (lo | (hi << 4)) - 32;
    float d = h2f(ld16(b + 208));
    float sc = (float)(int8_t)b[192 + 8 * h + 2 * q + (l >> 4)];
    return hmul(hmul(d, sc), (float)v);
}
// LNS8 (src/vbs_host_math.h:111-121): 32 log-codes then an f32 scale at byte
// 32; value = exp2f(q) * scale. exp2f of an integer code is the exact power
// of two for q <= 127 and +inf above, so it is assembled directly.
template <> __device__ __forceinline__ float deq_elem<kLNS8>(const uint8_t *b, uint32_t e) {
    uint32_t q = b[e];
    float p = q < 128u ? vbs_half_bits_to_float((q + 127u) << 23) : INFINITY;
    float scale = *reinterpret_cast<const float *>(b + 32);
    return hmul(p, scale);
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
// Wave reductions: the butterfly v = op(v, v of lane l ^ m) for m = 32, 16,
// 8, 4, 2, 1, so that every lane ends with the same value and the adds happen
// in one fixed order whatever kernel runs them. The partners come without
// LDS: m = 32 and 16 from the gfx950 lane swaps (v_permlane32_swap,
// v_permlane16_swap); from m = 8 on, a value depends on lane mod 2m only, so
// the row rotation by m (DPP row_ror: lane l reads lane (l - m) mod 16 of its
// row) reads a lane holding the value of lane l ^ m. The whole wave must be
// active.
template <int M>
__device__ __forceinline__ uint32_t bfly_partner(uint32_t v, uint32_t lane) {
    if constexpr (M == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return lane < 32u ? r[1] : r[0];
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16u) ? r[0] : r[1];
    } else {
        static_assert(M == 8 || M == 4 || M == 2 || M == 1, "butterfly step");
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x120 + M, 0xF, 0xF, false);
    }
}
template <int M>
__device__ __forceinline__ float bfly_partner(float v, uint32_t lane) {
    return __builtin_bit_cast(float, bfly_partner<M>(__builtin_bit_cast(uint32_t, v), lane));
}
template <int M>
__device__ __forceinline__ double bfly_partner(double v, uint32_t lane) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = bfly_partner<M>((uint32_t)u, lane), hi = bfly_partner<M>((uint32_t)(u >> 32), lane);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
// The value that lane l ^ M holds, for any values: M = 16 or 32, by the lane
// swaps (no LDS round trip). The whole wave must be active.
template <int M, class T>
__device__ __forceinline__ T lane_xor(T v) {
    static_assert(M == 16 || M == 32, "lane_xor: 16 or 32");
    return bfly_partner<M>(v, __lane_id());
}
template <class T, class Op>
__device__ __forceinline__ T wave_butterfly(T v, Op op) {
    const uint32_t lane = __lane_id();
    v = op(v, bfly_partner<32>(v, lane));
    v = op(v, bfly_partner<16>(v, lane));
    v = op(v, bfly_partner<8>(v, lane));
    v = op(v, bfly_partner<4>(v, lane));
    v = op(v, bfly_partner<2>(v, lane));
    v = op(v, bfly_partner<1>(v, lane));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    return wave_butterfly(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ double wave_sum_d(double v) {
    return wave_butterfly(v, [](double a, double b) { return a + b; });
}
__device__ __forceinline__ float wave_max(float v) {
    return wave_butterfly(v, [](float a, float b) { return fmaxf(a, b); });
}

}  // namespace vbs
