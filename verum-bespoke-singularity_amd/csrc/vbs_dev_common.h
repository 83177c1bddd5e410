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
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

}  // namespace vbs
