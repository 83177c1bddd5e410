/* vbs_half.h — the reference's half-precision conversions, usable from host C
 * and from HIP device code.
 *
 * f16 -> f32 follows src/vbs_dequant.c:21-44 (exact, NaN payload kept).
 * f32 -> f16 follows src/vbs_dequant.c:46-74, which is NOT the IEEE
 * conversion: normal results round to nearest even, but results below the
 * smallest normal round half UP from the 24-bit significand, values under
 * 2^-25 flush to signed zero, and every NaN becomes 0x7C01 (sign kept).
 * The hardware converter (v_cvt_f16_f32) rounds subnormals to nearest even,
 * so the KV-cache store uses this integer form to stay bit-identical.
 */
#ifndef VBS_HALF_H
#define VBS_HALF_H

#include <stdint.h>

#if defined(__HIPCC__)
#define VBS_HD __host__ __device__ __forceinline__
#else
#define VBS_HD static inline
#endif

VBS_HD float vbs_half_bits_to_float(uint32_t bits) {
    union { uint32_t u; float f; } c;
    c.u = bits;
    return c.f;
}

VBS_HD uint32_t vbs_float_to_bits(float f) {
    union { uint32_t u; float f; } c;
    c.f = f;
    return c.u;
}

VBS_HD float vbs_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 31u, man = h & 1023u;
    if (e == 31u) return vbs_half_bits_to_float(sign | 0x7F800000u | (man << 13));
    if (e != 0u) return vbs_half_bits_to_float(sign | ((e + 112u) << 23) | (man << 13));
    if (man == 0u) return vbs_half_bits_to_float(sign);
    /* subnormal: man * 2^-24 is an exact normal float */
    float mag = (float)man * 5.9604644775390625e-08f;
    return vbs_half_bits_to_float(sign | vbs_float_to_bits(mag));
}

VBS_HD uint16_t vbs_f2h(float f) {
    uint32_t u = vbs_float_to_bits(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    int be = (int)((u >> 23) & 255u);
    uint32_t frac = u & 0x7FFFFFu;
    if (be == 255) return (uint16_t)(sign | 0x7C00u | (frac ? 1u : 0u));
    int he = be - 112;
    if (he >= 31) return (uint16_t)(sign | 0x7C00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)sign;
        uint32_t sh = (uint32_t)(14 - he);
        uint32_t q = ((frac | 0x800000u) + (1u << (sh - 1u))) >> sh;
        return (uint16_t)(sign | (q >= 1024u ? 1024u : q));
    }
    uint32_t r = frac + 4095u + ((frac >> 13) & 1u);
    if (r & 0x800000u) { r = 0; he++; }
    if (he >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)he << 10) | (r >> 13));
}

/* f32 -> f16 as the CPU model's Q8 activation scales are rounded
 * (src/vbs_cpu.c:74-93): round to nearest even everywhere, subnormals
 * included; |f| < 2^-25 (and a tie at 2^-25) gives signed zero; |f| >= 2^16,
 * infinities and NaNs give signed infinity. For finite inputs this is the
 * IEEE conversion. */
VBS_HD uint16_t vbs_f2h_rne(float f) {
    uint32_t u = vbs_float_to_bits(f);
    uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a >= 0x47800000u) return (uint16_t)(sign | 0x7C00u);
    if (a >= 0x38800000u) { /* normal half: rebias 127 -> 15, keep 10 bits */
        uint32_t h = (a >> 13) - (112u << 10), rest = a & 0x1FFFu;
        h += (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ? 1u : 0u;
        return (uint16_t)(sign | h); /* a carry out of the mantissa is exact */
    }
    if (a < 0x33000000u) return (uint16_t)sign;
    /* subnormal half: value / 2^-24 = significand >> (-e - 1), e in [-25, -15] */
    uint32_t sig = (a & 0x7FFFFFu) | 0x800000u;
    uint32_t sh = 126u - (a >> 23);
    uint32_t h = sig >> sh, rest = sig & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    h += (rest > half || (rest == half && (h & 1u))) ? 1u : 0u;
    return (uint16_t)(sign | h);
}

#endif
