// vbs_mfma.h — the batch-1 matrix-core matvec (shared by vbs_kern_mfma.hip,
// vbs_kern_mfma_blk.hip and vbs_kern_mfma_batch.hip): x digits, weight-type
// policies, the k_mvf kernel template and its launch plan.
//
// y[r] (+)= sum_c deq(W[r,c]) * x[c] with W in native GGUF super-blocks
// (src/vbs_dequant.c:225-277 for Q4_K, 316-333 for Q6_K); the reference's
// linear is vbs_host_linear_tile (src/vbs_host_math.h:223-267).
//
// x in digit form: every 32-element sub-block j of x gets an exponent e_j with
// 2^e_j > max|x| over the sub-block, and each element becomes the integer
// X = rint(x * 2^(22 - e_j)) (|X| <= 2^22), split into three balanced signed
// bytes X = D0 + 2^8 D1 + 2^16 D2. A dot of quantised weights with x is then
// an exact integer dot per digit plane, scaled back by 2^(e_j - 22): x is
// represented to 2^-22 of its sub-block maximum, which keeps each row within
// ~1e-7 of the reference's double-accumulated result.
//
// The three digit planes make the batch-1 matvec a skinny integer GEMM, which
// is what v_mfma_i32_16x16x64_i8 computes: A (16 x 64) holds digit planes of
// x, B (64 x 16) the unpacked quants of 16 weight rows, and D (16 x 16) gets,
// per row, one integer dot per (scale group, plane). Operand layout: lane l
// holds A[l%16][ks(l/16, b)] and B[ks(l/16, b)][l%16] for its 16 bytes b, and
// D[4(l/16)+r][l%16] for r < 4 (checked on the device with a one-hot probe).
// A row 4t+p carries plane p of scale group t at exactly the lanes whose B
// bytes belong to group t, so lane (n, g) = (l%16, l/16) of D receives the
// three plane dots of group g of row n. A rows of other groups are zero (read
// from a 16-byte zero pad).
//
// Work split. A workgroup owns TPW tiles of 16 rows; its nw waves split each
// row by super-blocks (wave w takes blocks w, w + nw, ..., so the waves read
// adjacent blocks together) and leave one sum per (row, block) in LDS; a row
// adds its blocks in index order at the end, so its value does not depend on
// the split (fused and per-op launches of one matrix agree bit for bit). A
// wave streams its (tile, block) items with one in flight ahead of the one it
// computes, and turns x into digits one 256-element block at a time, right
// before the first item that needs it; it reads only the digits of its own
// blocks, so no barrier stands between the first weight bytes and the matrix
// cores. With an RMSNorm in front, the sum of squares over all x blocks comes
// first (one barrier; the loads of the first item are already out). Deeper
// streams or x travelling with the items measured no faster: the memory
// system is saturated from the first requests on.
//
// Q4_K (144-byte blocks). Lane (n, g) reads the 16-byte header of row n and 16
// bytes of nibbles at qs offsets 16g and 64 + 16g. qs bytes 32s..32s+31 hold
// sub-block 2s in their low and 2s+1 in their high nibbles; per 64-byte span
// one MFMA takes the low and one the high nibbles, accumulating into one D in
// which group g is sub-block 4*span + g. Value per sub-block, as the
// reference's d*sc*nib - dmin*m summed: d*sc*2^(e-22)*S - dmin*m*sum(x).
//
// Q6_K (210-byte blocks, 6-bit quants, 16-element int8 scales). Lane group
// g = (h, u) covers elements 16u..16u+15 of every 32-element quarter of half h
// of the block: it reads the ql bytes of quarters 0/2 and 1/3 and the qh bytes
// of those elements, plus the 16 scales and d. MFMA q in 0..3 takes quarter q
// of both halves, so every shift in the 6-bit unpack is the same for all
// lanes, and lane group g holds scale group 8h + 2q + u. Value per group, as
// d*sc*(q - 32) summed: d*sc*(2^(e-22)*S - 32*sum16(x)).
#pragma once

#include <type_traits>

#include "vbs_dev_common.h"
#include "vbs_internal.h"
#include "vbs_lds_dma.h"

namespace vbs {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---- digit buffer ---------------------------------------------------------------
// [3][cols] int8 planes | 16 zero bytes | float2 xs[cols/32] = {2^(e-22), sum x}
// | float xs16[cols/16] = sum of x per 16 elements.
struct XqLayout {
    uint32_t zero, xs, xs16, bytes;
};
__host__ __device__ inline XqLayout xq_layout(uint32_t cols) {
    XqLayout L;
    L.zero = 3u * cols;
    L.xs = (L.zero + 16u + 15u) & ~15u;
    L.xs16 = L.xs + 8u * (cols / 32u);
    L.bytes = L.xs16 + 4u * (cols / 16u);
    return L;
}

// Where the digits of one 256-element block live: plane p at base + p *
// pstride, its xs (8 float2) and xs16 (16 floats), and a 16-byte zero pad.
// Launches with one tile per workgroup give each wave a single slot that it
// refills for every block (a wave's blocks are used once, in turn), so their
// LDS does not grow with the row length; the others keep [3][cols] planes.
struct DigitView {
    uint8_t *base;
    uint32_t pstride;
    float2 *xs;
    float *xs16;
    const uint8_t *zero;
};
constexpr uint32_t kSlotBytes = 3u * 256u + 64u + 64u;  // planes | xs16 | xs


// Group reductions over aligned lane groups with DPP (every lane of the group
// gets the result): L = 4 (quads) or 8 (half rows).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_sum(float v) {
    v = v + dpp_f<0xB1>(v);  // quad_perm [1,0,3,2]
    return v + dpp_f<0x4E>(v);  // quad_perm [2,3,0,1]
}
__device__ __forceinline__ float quad_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    return fmaxf(v, dpp_f<0x4E>(v));
}
__device__ __forceinline__ float half_row_other(float v) { return dpp_f<0x141>(v); }  // lane i <-> 7-i

// Digits of block b of x (256 elements) by one wave: lane l holds elements
// 4l..4l+3 (v), so a 16-element item is a lane quad and a 32-element
// sub-block a half row. Writes the three planes, xs and xs16 of the block.
// Sums: per lane in element order, then the quad, then the two quads of a
// sub-block (the same value in every lane of the group).
__device__ __forceinline__ void prep_block(const float *v, uint32_t lane, const DigitView &dv) {
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    const float sum4 = ((v[0] + v[1]) + v[2]) + v[3];
    amax = quad_max(amax);
    amax = fmaxf(amax, half_row_other(amax));
    const float sum16 = quad_sum(sum4);
    const float other = half_row_other(sum16);
    const float sum32 = (lane & 4u) ? other + sum16 : sum16 + other;  // same order in both quads
    int e;
    (void)frexpf(amax, &e);  // amax < 2^e
    const bool finite = amax <= 3.4028235e38f;
    // X = rint(x 2^(22-e)) with |X| < 2^22: adding 1.5 * 2^23 rounds to the
    // nearest integer (ties to even, as rint) and leaves 2^22 + X in the low 23
    // bits. U = X + 0x808080 then holds the balanced digits as biased bytes:
    // D_i = byte_i(U) - 128, i.e. byte_i(U) ^ 0x80 in int8 form (the same
    // digits as D0 = int8(X), D1 = int8((X - D0) / 256), ...). Sub-blocks whose
    // maximum is not finite get a NaN scale, which makes their digits moot.
    uint32_t u[4];
#pragma unroll
    for (int k = 0; k < 4; k++)
        u[k] = __float_as_uint(__fadd_rn(ldexpf(v[k], 22 - e), 12582912.0f)) + 0x408080u;
    const uint32_t lo01 = __builtin_amdgcn_perm(u[1], u[0], 0x05010400u);
    const uint32_t lo23 = __builtin_amdgcn_perm(u[3], u[2], 0x05010400u);
    const uint32_t hi01 = __builtin_amdgcn_perm(u[1], u[0], 0x0c0c0602u);
    const uint32_t hi23 = __builtin_amdgcn_perm(u[3], u[2], 0x0c0c0602u);
    uint8_t *const at = dv.base + 4u * lane;
    *reinterpret_cast<uint32_t *>(at) = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u) ^ 0x80808080u;
    *reinterpret_cast<uint32_t *>(at + dv.pstride) =
        __builtin_amdgcn_perm(lo23, lo01, 0x07060302u) ^ 0x80808080u;
    *reinterpret_cast<uint32_t *>(at + 2u * dv.pstride) =
        __builtin_amdgcn_perm(hi23, hi01, 0x05040100u) ^ 0x80808080u;
    if ((lane & 3u) == 0) dv.xs16[lane / 4u] = sum16;
    if ((lane & 7u) == 0)
        dv.xs[lane / 8u] =
            make_float2(finite ? ldexpf(1.0f, e - 22) : __builtin_nanf(""), sum32);
}

// Sum of squares of block b of x (lane l: elements 4l..4l+3 in element
// order, then a butterfly over the wave), in double. The RMSNorm adds the
// blocks in index order; k_rms_norm uses the same order.
__device__ __forceinline__ double block_sumsq(const float *v) {
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 4; k++) ss = fma((double)v[k], (double)v[k], ss);
    return wave_sum_d(ss);
}

// ---- helpers ------------------------------------------------------------------------
// 16 bytes from a 16-byte aligned address.
__device__ __forceinline__ u32x4 lda4(const uint8_t *p) {
    return *reinterpret_cast<const u32x4 *>(p);
}
// 16 bytes from a 2-byte aligned address (used on LDS).
__device__ __forceinline__ u32x4 ldu(const uint8_t *p) {
    typedef u32x4 __attribute__((aligned(2))) u32x4u;
    return *reinterpret_cast<const u32x4u *>(p);
}
__device__ __forceinline__ i32x4 lda(const uint8_t *p) {
    return *reinterpret_cast<const i32x4 *>(p);
}
__device__ __forceinline__ float cvt_h(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t w) {
    return __builtin_amdgcn_ubfe(v, off, w);
}
__device__ __forceinline__ i32x4 mfma(i32x4 a, i32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
// The three plane dots combined, exact up to one rounding (|D0 + 256 D1| < 2^24).
__device__ __forceinline__ float plane_sum(i32x4 D) {
    return fmaf((float)D[2], 65536.f, (float)(D[0] + D[1] * 256));
}

// ---- weight types ---------------------------------------------------------------------
// Where a wave's tile lives: row r of the matrix starts at w + r * rb; rows of
// the tile past the end re-read the last row; no load reaches past w + bytes.
// Offsets are 32-bit (the matrix is below 4 GiB) from the wave-uniform base w,
// so loads take the scalar-base form.
struct Src {
    const uint8_t *w;
    uint32_t bytes, rb, row0, rows;
    __device__ uint32_t row(uint32_t n) const { return min(row0 + n, rows - 1u) * rb; }
};

// load(): this lane's share of block b of the tile (NLD 16-byte words).
// dot(): the block's contribution to the lane's row partial sum; (n, g) is the
// lane as MFMA operand (A row n, lane group g); `scratch` is the wave's LDS.
struct Q4K {
    static constexpr uint32_t BYTES = 144, NLD = 3, SCRATCH = 0;
    __device__ static void load(const Src &src, uint32_t b, uint32_t n, uint32_t g, u32x4 *r) {
        const uint8_t *blk = src.w + (src.row(n) + b * BYTES);
        r[0] = lda4(blk);
        r[1] = lda4(blk + 16u * g + 16u);
        r[2] = lda4(blk + 16u * g + 80u);
    }
    // The x side of a block's dot, the same for every tile of rows: the digit
    // planes as MFMA A operands and the sub-block x scales of lane group g.
    // A row n = 4t+p: lane group g carries sub-blocks 2(g>>1) (low nibbles,
    // t even) and 2(g>>1)+1 (high nibbles, t odd) at element offset 16(g&1).
    struct X {
        i32x4 A0l, A0h, A1l, A1h;
        float2 xs0, xs1;
    };
    __device__ static X x_operands(const DigitView &dv, uint32_t n, uint32_t g) {
        const uint32_t t = n >> 2, p = n & 3u;
        const bool on = p < 3u && (g >> 1) == (t >> 1);
        const uint8_t *ao = dv.base + p * dv.pstride + 32u * t + 16u * (g & 1u);
        X x;
        x.A0l = lda(on && !(t & 1u) ? ao : dv.zero);
        x.A0h = lda(on && (t & 1u) ? ao : dv.zero);
        x.A1l = lda(on && !(t & 1u) ? ao + 128u : dv.zero);
        x.A1h = lda(on && (t & 1u) ? ao + 128u : dv.zero);
        x.xs0 = dv.xs[g];
        x.xs1 = dv.xs[4u + g];
        return x;
    }
    __device__ static float dot(const u32x4 *r, uint8_t *, const Src &, const DigitView &dv,
                                uint32_t b, uint32_t n, uint32_t g) {
        (void)b;
        return dot_x(r, x_operands(dv, n, g), g);
    }
    __device__ static float dot_x(const u32x4 *r, uint8_t *, const Src &, const X &x, uint32_t,
                                  uint32_t, uint32_t g) {
        return dot_x(r, x, g);
    }
    __device__ static float dot_x(const u32x4 *r, const X &x, uint32_t g) {
        const i32x4 A0l = x.A0l, A0h = x.A0h, A1l = x.A1l, A1h = x.A1h;
        const uint32_t M4 = 0x0F0F0F0Fu;
        const u32x4 qa = r[1], qb = r[2];
        const i32x4 B0l = {(int)(qa.x & M4), (int)(qa.y & M4), (int)(qa.z & M4), (int)(qa.w & M4)};
        const i32x4 B0h = {(int)((qa.x >> 4) & M4), (int)((qa.y >> 4) & M4),
                           (int)((qa.z >> 4) & M4), (int)((qa.w >> 4) & M4)};
        const i32x4 B1l = {(int)(qb.x & M4), (int)(qb.y & M4), (int)(qb.z & M4), (int)(qb.w & M4)};
        const i32x4 B1h = {(int)((qb.x >> 4) & M4), (int)((qb.y >> 4) & M4),
                           (int)((qb.z >> 4) & M4), (int)((qb.w >> 4) & M4)};
        const i32x4 z = {0, 0, 0, 0};
        const float S0 = plane_sum(mfma(A0h, B0h, mfma(A0l, B0l, z)));
        const float S1 = plane_sum(mfma(A1h, B1h, mfma(A1l, B1l, z)));
        // D group g: sub-blocks g (span 0) and 4 + g (span 1); scales and mins
        // as src/vbs_dequant.c:225-233
        const float2 xs0 = x.xs0, xs1 = x.xs1;
        const u32x4 hd = r[0];
        const uint32_t sh = 8u * g;
        const uint32_t sc0 = bfe(hd.y, sh, 6), m0 = bfe(hd.z, sh, 6);
        const uint32_t sc1 = bfe(hd.w, sh, 4) | (bfe(hd.y, sh + 6u, 2) << 4);
        const uint32_t m1 = bfe(hd.w, sh + 4u, 4) | (bfe(hd.z, sh + 6u, 2) << 4);
        const float d = cvt_h(hd.x & 0xFFFFu), dmin = cvt_h(hd.x >> 16);
        const float sd = fmaf((float)sc0 * xs0.x, S0, (float)sc1 * xs1.x * S1);
        const float sm = fmaf((float)m0, xs0.y, (float)m1 * xs1.y);
        return fmaf(d, sd, -dmin * sm);
    }
};

// 16 aligned bytes at a, of which only those below `end` (2-byte aligned) are
// read; the rest are zero.
__device__ __forceinline__ u32x4 ld_tail(const uint8_t *a, const uint8_t *end) {
    uint32_t v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint8_t *p = a + 4 * k;
        v[k] = p + 4 <= end   ? *reinterpret_cast<const uint32_t *>(p)
               : p + 2 <= end ? (uint32_t)*reinterpret_cast<const uint16_t *>(p)
                              : 0u;
    }
    const u32x4 r = {v[0], v[1], v[2], v[3]};
    return r;
}

struct Q6K {
    // A 210-byte block is 2-byte aligned, and 16-byte loads at such addresses
    // run at about half the rate of aligned ones. So the wave reads each block
    // of its 16 rows as 14 aligned 16-byte chunks per row (covering the block
    // at any 2-byte offset), chunk c = 14n + k going to lane c mod 64, stores
    // them to its LDS scratch in row order and reads its fields from there as
    // 4-byte aligned words, shifted into place in registers (16-byte LDS reads
    // at 2-byte aligned addresses are several times slower).
    static constexpr uint32_t BYTES = 210, NLD = 4, SCRATCH = 16u * 224u;
    __device__ static void load(const Src &src, uint32_t b, uint32_t n, uint32_t g, u32x4 *r) {
        const uint32_t lane = 16u * g + n;
        // Offsets are taken from w16, w rounded down to 16 bytes (w itself may
        // be only 2-byte aligned): chunk k of a block at byte s of the matrix
        // starts at ((s + wlo) & ~15) + 16 k from w16. Only the last block of
        // the matrix's last row has chunks that reach past its end (by at most
        // 14 bytes); those loads are bounded.
        const uint32_t wlo = (uint32_t)(uintptr_t)src.w & 15u;
        const uint8_t *const w16 = src.w - wlo;
        const uint32_t last = src.row(15u) + b * BYTES;
        const bool edge = __builtin_amdgcn_readfirstlane(
                              (uint32_t)(((last + wlo) & ~15u) + 224u > src.bytes + wlo)) != 0u;
        uint32_t a[4];
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            // chunk c of the tile: 16 aligned bytes
            const uint32_t c = min(lane + 64u * i, 223u);
            const uint32_t s = src.row(c / 14u) + b * BYTES;
            a[i] = ((s + wlo) & ~15u) + 16u * (c % 14u);
        }
        if (!edge) {
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) r[i] = lda4(w16 + a[i]);
        } else {
            const uint8_t *end = src.w + src.bytes;
#pragma unroll
            for (uint32_t i = 0; i < 4; i++)
                r[i] = a[i] + 16u <= src.bytes + wlo ? lda4(w16 + a[i]) : ld_tail(w16 + a[i], end);
        }
    }
    __device__ static void stage(const u32x4 *r, uint8_t *scratch, uint32_t n, uint32_t g) {
        const uint32_t lane = 16u * g + n;
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t c = lane + 64u * i;
            if (i < 3u || c < 224u) *reinterpret_cast<u32x4 *>(scratch + 16u * c) = r[i];
        }
    }
    __device__ static float dot(const u32x4 *r, uint8_t *scratch, const Src &src,
                                const DigitView &dv, uint32_t b, uint32_t n, uint32_t g) {
        stage(r, scratch, n, g);
        return dot_staged(scratch, src, dv, b, n, g);
    }
    // The x side of a block's dot, the same for every tile of rows: MFMA q's A
    // operand (row n = 4t+p carries plane p of the scale group of lane group
    // t), and the x scale and -32 x sum of lane group g's scale group 8h + 2q + u.
    struct X {
        i32x4 A[4];
        float xs[4], m32[4];
    };
    __device__ static X x_operands(const DigitView &dv, uint32_t n, uint32_t g) {
        const uint32_t h = g >> 1, u = g & 1u;
        const uint32_t t = n >> 2, p = n & 3u;
        const bool on = p < 3u && t == g;
        const uint8_t *a0 = dv.base + p * dv.pstride + 128u * (t >> 1) + 16u * (t & 1u);
        X x;
#pragma unroll
        for (uint32_t q = 0; q < 4; q++) {
            const uint32_t j = 4u * h + q;  // sub-block of the block
            x.A[q] = lda(on ? a0 + 32u * q : dv.zero);
            x.xs[q] = dv.xs[j].x;
            x.m32[q] = -32.f * dv.xs16[2u * j + u];
        }
        return x;
    }
    // The same from a scratch that already holds the tile's 224 chunks (chunk
    // 14 n + k at 16 (14 n + k): row n's aligned 16-byte chunk k).
    __device__ static float dot_staged(const uint8_t *scratch, const Src &src, const DigitView &dv,
                                       uint32_t b, uint32_t n, uint32_t g) {
        return dot_staged_x(scratch, src, x_operands(dv, n, g), b, n, g);
    }
    __device__ static float dot_staged_x(const uint8_t *scratch, const Src &src, const X &x,
                                         uint32_t b, uint32_t n, uint32_t g) {
        // row n's block starts o = (its address mod 16) into its 224 scratch
        // bytes; rw is the 4-byte aligned word at or below the start and sh
        // (0 or 2) the byte shift from there. Every word read lies in the row.
        const uint32_t o = ((uint32_t)(uintptr_t)src.w + src.row(n) + b * BYTES) & 15u;
        const uint32_t *rw = reinterpret_cast<const uint32_t *>(scratch + 224u * n + (o & 12u));
        const uint32_t sh = o & 2u;
        // 16 bytes at block byte f (a multiple of 4)
        auto field = [&](uint32_t f) {
            const uint32_t *p = rw + f / 4u;
            const uint32_t w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3], w4 = p[4];
            const u32x4 v = {__builtin_amdgcn_alignbyte(w1, w0, sh),
                             __builtin_amdgcn_alignbyte(w2, w1, sh),
                             __builtin_amdgcn_alignbyte(w3, w2, sh),
                             __builtin_amdgcn_alignbyte(w4, w3, sh)};
            return v;
        };
        // lane group g = (h, u) = (g >> 1, g & 1): half h of the block, elements
        // 16u..16u+15 of each of its 32-element quarters
        const uint32_t h = g >> 1, u = g & 1u;
        const u32x4 qe = field(64u * h + 16u * u);         // ql, quarters 0 / 2
        const u32x4 qo = field(64u * h + 32u + 16u * u);   // ql, quarters 1 / 3
        const u32x4 qh = field(128u + 32u * h + 16u * u);  // qh, 2 bits per quarter
        // int8 scales 8h..8h+7 (bytes 192 + 8h) and the f16 d (bytes 208..209)
        const uint32_t *ps = rw + 48u + 2u * h;
        const uint32_t s0 = ps[0], s1 = ps[1], s2 = ps[2];
        const uint32_t sc_lo = __builtin_amdgcn_alignbyte(s1, s0, sh);
        const uint32_t sc_hi = __builtin_amdgcn_alignbyte(s2, s1, sh);
        const uint32_t dbits = (rw[52] >> (8u * sh)) & 0xFFFFu;
        // MFMA q (quarter q of both halves): lane group g holds scale group
        // 8h + 2q + u
        const uint32_t qew[4] = {qe.x, qe.y, qe.z, qe.w}, qow[4] = {qo.x, qo.y, qo.z, qo.w};
        const uint32_t qhw[4] = {qh.x, qh.y, qh.z, qh.w};
        float acc = 0.f;
#pragma unroll
        for (uint32_t q = 0; q < 4; q++) {
            // 6-bit quants, src/vbs_dequant.c:316-333: low 4 bits from ql
            // (nibble q >> 1 of region q & 1), high 2 bits from qh bits 2q
            const uint32_t *ql = (q & 1u) ? qow : qew;
            int bw[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t hi = (q <= 2u ? (qhw[k] << (4u - 2u * q)) : (qhw[k] >> 2u)) &
                                    0x30303030u;
                bw[k] = (int)(((ql[k] >> (4u * (q >> 1))) & 0x0F0F0F0Fu) | hi);
            }
            const i32x4 B = {bw[0], bw[1], bw[2], bw[3]};
            const i32x4 z = {0, 0, 0, 0};
            const float S = plane_sum(mfma(x.A[q], B, z));
            // scale 8h + 2q + u: dword 2h + (q >> 1), byte 2(q & 1) + u; the group
            // is half u of sub-block 4h + q
            const uint32_t scd = (q >> 1) ? sc_hi : sc_lo;
            const float sc = (float)(int)(int8_t)bfe(scd, 16u * (q & 1u) + 8u * u, 8);
            acc = fmaf(sc, fmaf(x.xs[q], S, x.m32[q]), acc);
        }
        return cvt_h(dbits) * acc;
    }
};

// ---- 32-element block types: Q4_0, Q4_1, Q8_0 -------------------------------------------
// Eight consecutive GGUF blocks (256 elements) are one "block" of this kernel:
// 144 (Q4_0), 160 (Q4_1) or 272 (Q8_0) bytes at 2-byte alignment. As for
// Q6_K, a wave stages its 16 rows' bytes in LDS as aligned 16-byte chunks (CH
// per row) and reads its fields there, shifted into place by (row start +
// field offset) mod 4. MFMA layout: chain c (sub-blocks 4c..4c+3 = GGUF
// blocks), two MFMAs per chain (elements 0-15, 16-31 of each sub-block); lane
// group g holds sub-block 4c + g as B, A row n = 4t + p carries plane p of
// sub-block 4c + t at lane group t only, so D row 4g' + r of lane group g' is
// plane r of sub-block 4c + g'. Per sub-block j (d, m the block's f16 scale
// and min, S the plane-combined integer dot, 2^(e-22) and sum x from the
// digit buffer), as the reference's values summed (src/vbs_dequant.c:123-179):
//   Q8_0: d*q            -> d * 2^(e-22) * S
//   Q4_0: (nib - 8) * d  -> d * (2^(e-22) * S - 8 * sum x)
//   Q4_1: d * nib + m    -> d * 2^(e-22) * S + m * sum x
template <int TYPE>
struct KBlk {
    static constexpr uint32_t BB = TYPE == kQ8_0 ? 34u : TYPE == kQ4_1 ? 20u : 18u;  // GGUF block
    static constexpr uint32_t QOFF = TYPE == kQ4_1 ? 4u : 2u;  // quants within the GGUF block
    static constexpr bool NIB = TYPE != kQ8_0;
    static constexpr uint32_t BYTES = 8u * BB;
    static constexpr uint32_t CH = (BYTES + 14u + 15u) / 16u;  // chunks covering any 2-byte offset
    static constexpr uint32_t NCHUNK = 16u * CH;
    static constexpr uint32_t NLD = (NCHUNK + 63u) / 64u, SCRATCH = 16u * NCHUNK;
    __device__ static void load(const Src &src, uint32_t b, uint32_t n, uint32_t g, u32x4 *r) {
        const uint32_t lane = 16u * g + n;
        // offsets from w16 = w rounded down to 16 bytes, as for Q6_K; only the
        // last block of the matrix's last row has chunks past its end
        const uint32_t wlo = (uint32_t)(uintptr_t)src.w & 15u;
        const uint8_t *const w16 = src.w - wlo;
        const uint32_t last = src.row(15u) + b * BYTES;
        const bool edge = __builtin_amdgcn_readfirstlane(
                              (uint32_t)(((last + wlo) & ~15u) + 16u * CH > src.bytes + wlo)) != 0u;
        uint32_t a[NLD];
#pragma unroll
        for (uint32_t i = 0; i < NLD; i++) {
            const uint32_t c = min(lane + 64u * i, NCHUNK - 1u);
            const uint32_t s0 = src.row(c / CH) + b * BYTES;
            a[i] = ((s0 + wlo) & ~15u) + 16u * (c % CH);
        }
        if (!edge) {
#pragma unroll
            for (uint32_t i = 0; i < NLD; i++) r[i] = lda4(w16 + a[i]);
        } else {
            const uint8_t *end = src.w + src.bytes;
#pragma unroll
            for (uint32_t i = 0; i < NLD; i++)
                r[i] = a[i] + 16u <= src.bytes + wlo ? lda4(w16 + a[i]) : ld_tail(w16 + a[i], end);
        }
    }
    __device__ static float dot(const u32x4 *r, uint8_t *scratch, const Src &src,
                                const DigitView &dv, uint32_t b, uint32_t n, uint32_t g) {
        const uint32_t lane = 16u * g + n;
#pragma unroll
        for (uint32_t i = 0; i < NLD; i++) {
            const uint32_t c = lane + 64u * i;
            if (i + 1u < NLD || c < NCHUNK) *reinterpret_cast<u32x4 *>(scratch + 16u * c) = r[i];
        }
        // row n's block starts o bytes into its CH chunks
        const uint32_t o = ((uint32_t)(uintptr_t)src.w + src.row(n) + b * BYTES) & 15u;
        const uint32_t *rw = reinterpret_cast<const uint32_t *>(scratch + 16u * CH * n);
        auto field = [&](uint32_t f) {  // 16 bytes at block byte f (even)
            const uint32_t P = o + f, i = P >> 2, sh = P & 3u;
            const uint32_t w0 = rw[i], w1 = rw[i + 1u], w2 = rw[i + 2u], w3 = rw[i + 3u], w4 = rw[i + 4u];
            const u32x4 v = {__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh),
                             __builtin_amdgcn_alignbyte(w3, w2, sh), __builtin_amdgcn_alignbyte(w4, w3, sh)};
            return v;
        };
        auto half16 = [&](uint32_t f) {  // the f16 bits at block byte f (even)
            const uint32_t P = o + f;
            return (rw[P >> 2] >> (8u * (P & 3u))) & 0xFFFFu;
        };
        const uint32_t t = n >> 2, p = n & 3u;
        const bool on = p < 3u && t == g;
        const i32x4 z = {0, 0, 0, 0};
        float acc = 0.f;
#pragma unroll
        for (uint32_t c = 0; c < 2u; c++) {
            const uint32_t j = 4u * c + g;  // this lane group's sub-block (B) and D sub-block
            u32x4 q0, q1;
            if (NIB) {  // qs[16]: element e < 16 low nibble of qs[e], e >= 16 high nibble
                const u32x4 q = field(BB * j + QOFF);
                const uint32_t M4 = 0x0F0F0F0Fu;
                q0 = u32x4{q.x & M4, q.y & M4, q.z & M4, q.w & M4};
                q1 = u32x4{(q.x >> 4) & M4, (q.y >> 4) & M4, (q.z >> 4) & M4, (q.w >> 4) & M4};
            } else {  // int8 q[32]
                q0 = field(BB * j + QOFF);
                q1 = field(BB * j + QOFF + 16u);
            }
            const uint8_t *ao = dv.base + p * dv.pstride + 32u * (4u * c + t);
            const i32x4 A0 = lda(on ? ao : dv.zero);
            const i32x4 A1 = lda(on ? ao + 16u : dv.zero);
            const i32x4 D = mfma(A1, __builtin_bit_cast(i32x4, q1),
                                 mfma(A0, __builtin_bit_cast(i32x4, q0), z));
            const float S = plane_sum(D);
            const float2 x2 = dv.xs[j];
            const float d = cvt_h(half16(BB * j));
            if (TYPE == kQ8_0) acc = fmaf(d * x2.x, S, acc);
            else if (TYPE == kQ4_0) acc = fmaf(d, fmaf(x2.x, S, -8.f * x2.y), acc);
            else acc = fmaf(d * x2.x, S, fmaf(cvt_h(half16(BB * j + 2u)), x2.y, acc));
        }
        return acc;
    }
};
using Q40 = KBlk<kQ4_0>;
using Q41 = KBlk<kQ4_1>;
using Q80 = KBlk<kQ8_0>;

// ---- jobs -------------------------------------------------------------------------------
// One launch computes the rows of up to three matrices that share x (and its
// type and column count), with an optional RMSNorm of x in front and one of
// these epilogues on each finished row value t (every arithmetic step is the
// reference's own):
//   E_STORE  y[row] = t                       (vbs_host_linear_tile)
//   E_ACC    y[row] = y[row] + t              (linear, then ELEMENTWISE add)
//   E_QKV    matrix roles q, k, v: RoPE of q and k rows at the device position
//            (src/vbs_host_math.h:38-51), q to y[0] in f32, k and v to the f16
//            caches (src/vbs_host_math.h:150-159)
//   E_SILU   gate and up: y[0][row] = gate / (1 + expf(-gate)) * up
//            (src/vbs_host_math.h:53-57)
enum : int { E_STORE = 0, E_ACC = 1, E_QKV = 2, E_SILU = 3 };

// A row's per-block partial sums, kept in LDS by the kernels that split a
// row's blocks over waves: part_slots(nblk) of them, nblk rounded up to 16
// (the slots past the row hold +0.0), row t's at pb + t * part_stride(nblk)
// floats (16-byte aligned; the threads of 16 rows read distinct banks).
__host__ __device__ constexpr uint32_t part_slots(uint32_t nblk) { return (nblk + 15u) & ~15u; }
__host__ __device__ constexpr uint32_t part_stride(uint32_t nblk) { return part_slots(nblk) + 4u; }
// Their sum in block order, s = ((0 + p[0]) + p[1]) + ..., read 16 at a time.
// The padding's +0.0 leaves s unchanged: s starts at +0.0 and never becomes
// -0.0 (an exactly cancelling sum is +0.0 when rounding to nearest).
__device__ __forceinline__ float ordered_sum(const float *p, uint32_t nblk) {
    float s = 0.f;
    for (uint32_t k0 = 0; k0 < nblk; k0 += 16u) {
        float4 v[4];
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) v[i] = *reinterpret_cast<const float4 *>(p + k0 + 4u * i);
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            s += v[i].x;
            s += v[i].y;
            s += v[i].z;
            s += v[i].w;
        }
    }
    return s;
}

struct MvArgs {
    const uint8_t *w[3];
    float *y[3];
    uint32_t rows[3];
    uint32_t tile_end[3];  // cumulative 16-row tiles per matrix
    uint32_t nmat, cols;
    const float *x;
    const float *norm_w;  // RMSNorm weights (NORM launches)
    float eps;
    const float2 *rope;   // E_QKV: [max_ctx][hd/2] (cos, sin)
    const uint32_t *pos;  // E_QKV: device position
    uint32_t hd, kvd, role0;
    uint16_t *kc, *vc;
    uint64_t kv_layer;  // E_QKV: layer * max_ctx * kvd; the store joins: (layer * max_ctx + pos) * kvd
    // ranged launches: workgroups of matrix m end at rwg_end[m] (cumulative),
    // each taking rpw[m] rows of it (the last one of a matrix fewer)
    uint32_t rwg_end[3], rpw[3];
    // the backend shim's fused neighbours of a linear (NULL elsewhere): NORM
    // launches also store the normalised x here (workgroup 0), E_ACC launches
    // also store each row value t here (the linear's own output, to which the
    // add was applied); E_STORE launches with `hid` also store
    // silu(gate_in[row]) * t there (the ACTIVATION op after the up matvec),
    // and with `kin` the CACHE op after the V matvec: f16(t) to vc and
    // f16(kin[row]) to kc at kv_layer + row
    float *xn, *ycopy;
    const float *gate_in, *kin;
    float *hid;
    // the backend shim's grouped ops also keep the f32 rows that the ops one
    // by one write: E_QKV the rotated k rows and the v rows (kout, vout),
    // E_SILU the gate and up rows (gout, uout); NULL elsewhere
    float *kout, *vout, *gout, *uout;
};

// The E_STORE neighbours above for row `row` with value t.
__device__ __forceinline__ void store_joins(const MvArgs &a, uint32_t row, float t) {
    if (a.hid) {
        const float g = a.gate_in[row];
        a.hid[row] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), t);
    }
    if (a.kin) {
        a.vc[a.kv_layer + row] = vbs_f2h(t);
        a.kc[a.kv_layer + row] = vbs_f2h(a.kin[row]);
    }
}

// The fused attn_norm + Q/K/V + RoPE + KV store launch of k_mvl
// (vbs_kern_mvl.hip) for Q4_K rows of 16 blocks and 4096 or more rows in all;
// hipErrorNotSupported elsewhere (k_mvf then runs). Bit-identical to k_mvf.
hipError_t launch_q4k_mvl_qkv(const MvArgs &a, hipStream_t s);

// E_QKV: row `row` of matrix m (role role0 + m) with value t, its RoPE
// partner row (row ^ 1) holding `other`: q rows and k rows rotated at the
// device position p by rope(i) = (cos, sin) of pair i, q stored as f32, k and
// v into the f16 caches.
template <class Rope>
__device__ __forceinline__ void qkv_store(const MvArgs &a, uint32_t m, uint32_t row, float t,
                                          float other, uint32_t p, Rope rope) {
    const uint32_t role = a.role0 + m;
    float v = t;
    if (role < 2u) {
        const float2 cs = rope((row % a.hd) / 2u);
        const bool even = (row & 1u) == 0u;
        const float x0 = even ? t : other, x1 = even ? other : t;
        v = even ? __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y))
                 : __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
    }
    if (role == 0u) {
        a.y[0][row] = v;
    } else {
        (role == 1u ? a.kc : a.vc)[a.kv_layer + (uint64_t)p * a.kvd + row] = vbs_f2h(v);
        float *const o = role == 1u ? a.kout : a.vout;
        if (o) o[row] = v;
    }
}

// The register set that holds a block's x operands when k_mvf reads them once
// for its tiles: Q4_K only (Q6_K's 24 registers would take its four-tile
// head launches past 128 VGPRs, one workgroup per CU instead of two).
template <class T, bool>
struct XOf {
    using type = char;
};
template <class T>
struct XOf<T, true> {
    using type = typename T::X;
};

// RANGED: workgroup b takes rows [r0, r1) of one matrix (MvArgs::rwg_end,
// rpw) as TPW tiles from r0, rows past r1 re-reading row r1 - 1, so that every
// CU streams an even share when the tiles do not divide evenly over the CUs
// (E_SILU: the same rows of gate, tiles 0 .. TPW/2 - 1, and of up, the rest).
template <class T, uint32_t KS, uint32_t TPW, uint32_t MAXT, bool NORM, int EPI, bool RANGED = false>
__global__ __launch_bounds__(MAXT) void k_mvf(const MvArgs a) {
    extern __shared__ __align__(16) uint8_t xq[];
    __shared__ double bsum[128];
    constexpr uint32_t NI = KS * TPW;  // work items (tile, block) per wave
    constexpr uint32_t P0 = 1;         // items issued with x, before anything is computed
    constexpr uint32_t P = 1;          // items in flight ahead of the one computed
    const uint32_t cols = a.cols;
    const uint32_t nblk = cols >> 8;
    const uint32_t rb = nblk * T::BYTES;
    const XqLayout L = xq_layout(cols);
    const uint32_t nth = blockDim.x;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t nw = nth >> 6;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t total = a.tile_end[a.nmat - 1u];

    // matrix and local tile of this workgroup's tile j
    uint32_t mt[TPW], lt[TPW];
    Src src[TPW];
    uint32_t rm = 0, r0 = 0, r1 = 0;  // RANGED: the workgroup's matrix and rows
    if constexpr (RANGED) {
        rm = (uint32_t)(blockIdx.x >= a.rwg_end[0]) + (uint32_t)(blockIdx.x >= a.rwg_end[1]);
        r0 = (blockIdx.x - (rm ? a.rwg_end[rm - 1u] : 0u)) * a.rpw[rm];
        r1 = min(r0 + a.rpw[rm], a.rows[rm]);
    }
#pragma unroll
    for (uint32_t j = 0; j < TPW; j++) {
        if constexpr (RANGED) {
            constexpr uint32_t H = EPI == E_SILU ? TPW / 2u : TPW;
            mt[j] = EPI == E_SILU ? (uint32_t)(j >= H) : rm;
            lt[j] = 0u;
            src[j] = Src{a.w[mt[j]], a.rows[mt[j]] * rb, rb, r0 + 16u * (j % H), r1};
            continue;
        }
        if (EPI == E_SILU) {
            mt[j] = j;
            lt[j] = blockIdx.x;
        } else {
            const uint32_t gt = min(blockIdx.x * TPW + j, total - 1u);
            mt[j] = (gt >= a.tile_end[0]) + (a.nmat > 2u && gt >= a.tile_end[1]);
            lt[j] = gt - (mt[j] ? a.tile_end[mt[j] - 1u] : 0u);
        }
        const uint8_t *w = a.w[mt[j]];
        src[j] = Src{w, a.rows[mt[j]] * rb, rb, lt[j] * 16u, a.rows[mt[j]]};
    }
    // Block k of this wave: wave + nw * k (at each step the workgroup's waves
    // read adjacent blocks of the same rows). Item i is block slot i % KS of
    // tile i / KS, or, where a block's x operands are read once for its tiles
    // (Q4_K with several tiles), tile i % TPW of block slot i / TPW. Slots
    // past the row re-read its last block and contribute zero. A wave
    // prepares the digits of its own blocks only, so the waves share no x
    // data and need no barrier before the matrix work.
    constexpr bool kHoist = std::is_same<T, Q4K>::value && TPW > 1u;
    auto slot = [&](uint32_t i) { return kHoist ? i / TPW : i % KS; };
    auto tile = [&](uint32_t i) { return kHoist ? i % TPW : i / KS; };
    auto bk = [&](uint32_t k) { return wave + nw * k; };
    auto blk = [&](uint32_t i) { return bk(slot(i)); };

    // x of this wave's blocks, lane l: elements 4l..4l+3 (x may be only
    // 4-byte aligned), and with the RMSNorm its weights: all requested first.
    typedef float4 __attribute__((aligned(4))) f4u;
    float4 xv[KS], wv[NORM ? KS : 1];
    auto load_x = [&](uint32_t k) {
        const uint32_t e0 = 256u * min(bk(k), nblk - 1u) + 4u * lane;
        xv[k] = *reinterpret_cast<const f4u *>(a.x + e0);
        if (NORM) wv[k] = *reinterpret_cast<const f4u *>(a.norm_w + e0);
    };
    u32x4 r[NI][T::NLD];
    auto issue = [&](uint32_t i) { T::load(src[tile(i)], min(blk(i), nblk - 1u), n, g, r[i]); };

    // 1-2. x, then the first items
#pragma unroll
    for (uint32_t k = 0; k < KS; k++) load_x(k);
#pragma unroll
    for (uint32_t i = 0; i < P0 && i < NI; i++) issue(i);
    __builtin_amdgcn_sched_barrier(0);

    // 3. RMSNorm scale: block sums of squares, added in block order
    float sc = 1.0f;
    if (NORM) {
#pragma unroll
        for (uint32_t k = 0; k < KS; k++) {
            const float v[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
            const double ss = block_sumsq(v);
            if (lane == 0 && bk(k) < nblk) bsum[bk(k)] = ss;
        }
        __syncthreads();
        double t = 0.0;
        for (uint32_t b = 0; b < nblk; b++) t += bsum[b];
        const float mean = (float)(t / (double)cols);
        sc = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, a.eps)));
    }
    // digits: one slot per wave (TPW == 1: [16-byte zero pad][nw slots]) or
    // [3][cols] planes with the pad after them
    constexpr bool kRing = TPW == 1u;
    const uint32_t zero_off = kRing ? 0u : L.zero;
    const uint32_t digit_bytes = kRing ? 16u + nw * kSlotBytes : L.bytes;
    if (lane < 4u) reinterpret_cast<uint32_t *>(xq + zero_off)[lane] = 0u;  // each wave's own pad
    auto view = [&](uint32_t b) {
        DigitView dv;
        dv.zero = xq + zero_off;
        if constexpr (kRing) {
            dv.base = xq + 16u + wave * kSlotBytes;
            dv.pstride = 256u;
            dv.xs16 = reinterpret_cast<float *>(dv.base + 768u);
            dv.xs = reinterpret_cast<float2 *>(dv.base + 832u);
        } else {
            dv.base = xq + 256u * b;
            dv.pstride = cols;
            dv.xs16 = reinterpret_cast<float *>(xq + L.xs16) + 16u * b;
            dv.xs = reinterpret_cast<float2 *>(xq + L.xs) + 8u * b;
        }
        return dv;
    };

    // 4. stream: issue item i + P, prepare x of a new block, compute item i
    // (loads return in issue order, so the wait is for item i alone)
    uint8_t *scratch = xq + digit_bytes + wave * T::SCRATCH;
    // per-block row sums, [TPW * 16 rows][part_stride(nblk)]: every row adds
    // its blocks in index order at the end, so a row's value does not depend
    // on the work split
    float *pb = reinterpret_cast<float *>(xq + digit_bytes + nw * T::SCRATCH);
    const uint32_t ps = part_stride(nblk), slots = part_slots(nblk);
    // a block's x operands, read once for its TPW tiles
    typename XOf<T, kHoist>::type xo{};
#pragma unroll
    for (uint32_t i = 0; i < NI; i++) {
#pragma unroll
        for (uint32_t j = i == 0 ? P0 : max(P0, i + P); j <= i + P && j < NI; j++) issue(j);
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t k = slot(i), tl = tile(i);
        if (tl == 0u && blk(i) < nblk) {
            float v[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
            if (NORM) {
                const float w4[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
#pragma unroll
                for (int k = 0; k < 4; k++) v[k] = __fmul_rn(__fmul_rn(v[k], sc), w4[k]);
                if (a.xn && blockIdx.x == 0)
                    *reinterpret_cast<float4 *>(a.xn + 256u * blk(i) + 4u * lane) =
                        make_float4(v[0], v[1], v[2], v[3]);
            }
            prep_block(v, lane, view(blk(i)));
        }
        const uint32_t bi = min(blk(i), nblk - 1u);
        float part;
        if constexpr (kHoist) {
            if (tl == 0u) xo = T::x_operands(view(bi), n, g);
            part = T::dot_x(r[i], scratch, src[tl], xo, bi, n, g);
        } else {
            part = T::dot(r[i], scratch, src[tl], view(bi), bi, n, g);
        }
        // the four lane groups of a row hold different groups of the block
        part += lane_xor<16>(part);
        part += lane_xor<32>(part);
        // (slots past the row: +0.0)
        if (lane < 16u && blk(i) < slots) pb[(tl * 16u + n) * ps + blk(i)] = blk(i) < nblk ? part : 0.f;
        // finish item i here: otherwise its arithmetic may sink past later
        // items and hold their registers
        asm volatile("" ::"v"(part));
        __builtin_amdgcn_sched_barrier(0);
    }

    // the slots no wave covers: +0.0
    const uint32_t covered = min(nw * KS, slots), pad = slots - covered;
    for (uint32_t e = threadIdx.x; e < TPW * 16u * pad; e += nth)
        pb[(e / pad) * ps + covered + e % pad] = 0.f;

    // 5. tile j finished by wave j % nw (both tiles by wave 0 for E_SILU)
    __syncthreads();
    if constexpr (RANGED && EPI == E_SILU) {  // row tile j: gate tile j, up tile j + TPW / 2
        constexpr uint32_t H = TPW / 2u;
#pragma unroll
        for (uint32_t j = 0; j < H; j++) {
            if (wave != j % nw) continue;
            const float gate = ordered_sum(pb + (j * 16u + n) * ps, nblk);
            const float up = ordered_sum(pb + ((j + H) * 16u + n) * ps, nblk);
            const uint32_t row = r0 + 16u * j + n;
            if (lane < 16u && row < r1) {
                const float den = __fadd_rn(1.0f, expf(-gate));
                a.y[0][row] = __fmul_rn(__fdiv_rn(gate, den), up);
                if (a.gout) a.gout[row] = gate;
                if (a.uout) a.uout[row] = up;
            }
        }
        return;
    }
    float prev = 0.f;  // E_SILU: the gate row value
#pragma unroll
    for (uint32_t j = 0; j < TPW; j++) {
        if (wave != (EPI == E_SILU ? 0u : j % nw)) continue;
        const float t = ordered_sum(pb + (j * 16u + n) * ps, nblk);
        // every lane holds the value of row n of the tile
        const uint32_t m = mt[j];
        const bool own = (RANGED || EPI == E_SILU || blockIdx.x * TPW + j < total);
        const uint32_t row = RANGED ? r0 + 16u * j + n : lt[j] * 16u + n;
        const bool st = lane < 16u && own && row < (RANGED ? r1 : a.rows[m]);
        if (EPI == E_STORE) {
            if (st) {
                a.y[m][row] = t;
                store_joins(a, row, t);
            }
        } else if (EPI == E_ACC) {
            if (st) {
                a.y[m][row] = __fadd_rn(a.y[m][row], t);
                if (a.ycopy) a.ycopy[row] = t;
            }
        } else if (EPI == E_SILU) {
            if (j == 0) {
                prev = t;
            } else if (st) {
                const float den = __fadd_rn(1.0f, expf(-prev));
                a.y[0][row] = __fmul_rn(__fdiv_rn(prev, den), t);
                if (a.gout) a.gout[row] = prev;
                if (a.uout) a.uout[row] = t;
            }
        } else {  // E_QKV
            const float other = __shfl_xor(t, 1, 64);  // the RoPE partner row
            if (st) {
                const uint32_t p = a.pos[0];
                qkv_store(a, m, row, t, other, p,
                          [&](uint32_t i) { return a.rope[(uint64_t)p * (a.hd / 2u) + i]; });
            }
        }
    }
}

// ---- launch ---------------------------------------------------------------------------
struct MvPlan {
    uint32_t ks, tpw, nw;
};

// The ranged split of a launch's matrices: the smallest even row count per
// workgroup (at most three tiles) whose workgroups, every one with rows, fit
// one per CU; false if none does.
static inline bool ranged_split(MvArgs &a, uint32_t cus) {
    uint32_t total = 0;
    for (uint32_t m = 0; m < a.nmat; m++) {
        if (a.rows[m] & 1u) return false;  // (RoPE pairs stay in one workgroup)
        total += a.rows[m];
    }
    for (uint32_t rpw = ((total + cus - 1u) / cus + 1u) & ~1u; rpw <= 48u; rpw += 2u) {
        uint32_t wgs = 0;
        for (uint32_t m = 0; m < 3u; m++) {
            if (m < a.nmat) wgs += (a.rows[m] + rpw - 1u) / rpw;
            a.rwg_end[m] = wgs;
            a.rpw[m] = rpw;
        }
        if (wgs <= cus) return true;
    }
    return false;
}

// Blocks per wave (KS) and waves per tile: enough waves to split the row and
// enough items per wave that the stream runs ahead of the arithmetic.
// (The gate/up launch, two tiles per workgroup, keeps four blocks per wave:
// eight waves of two would not all be resident at once.)
template <class T>
static MvPlan mv_plan(uint32_t cols, bool two_tiles, bool fused) {
    const uint32_t nblk = cols / 256u;
    MvPlan p;
    p.ks = nblk <= 16u && !two_tiles ? 2u : nblk <= 32u ? 4u : nblk <= 48u ? 6u
         : nblk <= 64u || nblk > 112u ? 8u : 14u;
    if (fused && p.ks == 14u) p.ks = 8u;  // (fused and normed launches keep eight)
    // Q6_K rows of 33-48 blocks (7B down): four blocks per wave, eleven waves
    // (measured 8% faster than six blocks on eight waves at 4096 x 11008)
    if (T::BYTES == 210u && !fused && !two_tiles && nblk > 32u && nblk <= 48u) p.ks = 4u;
    p.nw = (nblk + p.ks - 1u) / p.ks;
    p.tpw = 1u;
    return p;
}

template <class T, uint32_t KS, uint32_t TPW, uint32_t MAXT, bool NORM, int EPI, bool RANGED = false>
static hipError_t launch_t(const MvArgs &a, uint32_t nw, uint32_t wgs, hipStream_t s) {
    const size_t digits = TPW == 1u ? 16u + (size_t)nw * kSlotBytes : xq_layout(a.cols).bytes;
    const size_t lds = digits + (size_t)nw * T::SCRATCH +
                       (size_t)TPW * 16u * part_stride(a.cols / 256u) * sizeof(float);
    if (lds > 65536u) {  // beyond the default per-workgroup LDS window: opt in once
        static size_t granted = 0;
        if (lds > granted) {
            if (hipFuncSetAttribute((const void *)k_mvf<T, KS, TPW, MAXT, NORM, EPI, RANGED>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
                hipSuccess) {
                (void)hipGetLastError();
                return hipErrorNotSupported;
            }
            granted = lds;
        }
    }
    k_mvf<T, KS, TPW, MAXT, NORM, EPI, RANGED><<<wgs, 64u * nw, lds, s>>>(a);
    return hipGetLastError();
}

template <class T, bool NORM, int EPI, uint32_t TPW>
static hipError_t launch_ks(const MvArgs &a, const MvPlan &p, uint32_t wgs, hipStream_t s) {
#define VBS_MV(KS, MAXT) return launch_t<T, KS, TPW, MAXT, NORM, EPI>(a, p.nw, wgs, s)
    if (p.ks == 2u) {
        if (p.nw <= 8u) VBS_MV(2, 512);
        VBS_MV(2, 1024);
    }
    if (p.ks == 4u) {
        if (p.nw <= 8u) VBS_MV(4, 512);
        VBS_MV(4, 1024);
    }
    if (p.ks == 6u) {
        if (p.nw <= 8u) VBS_MV(6, 512);
        VBS_MV(6, 1024);
    }
    // rows of 65-112 blocks (70B down: 112), one tile per workgroup; rows of
    // at most 16 blocks over few tiles, one block per wave
    if constexpr ((EPI == E_STORE || EPI == E_ACC) && TPW == 1 && !NORM) {
        if (p.ks == 14u) VBS_MV(14, 512);
        if (p.ks == 1u) VBS_MV(1, 1024);
    }
    if constexpr (EPI == E_QKV) {  // the Q/K/V plans of launch_plan
        if (TPW == 2u && p.ks == 1u) VBS_MV(1, 1024);
        if (TPW == 1u && p.ks == 1u) VBS_MV(1, 1024);
        if (TPW == 1u && p.ks == 8u && p.nw <= 4u) VBS_MV(8, 256);
    }
    VBS_MV(8, 1024);
#undef VBS_MV
}

template <class T, bool NORM, int EPI>
static hipError_t launch_plan(const MvArgs &a, hipStream_t s) {
    const uint32_t total = a.tile_end[a.nmat - 1u];
    MvPlan p = mv_plan<T>(a.cols, EPI == E_SILU, NORM || EPI == E_SILU || EPI == E_QKV);
    if (p.ks == 14u && a.tile_end[a.nmat - 1u] >= 1024u) {  // (several tiles: keep eight)
        p.ks = 8u;
        p.nw = (a.cols / 256u + 7u) / 8u;
    }
    // Unfused launches of rows of at most 16 blocks over few tiles: one block
    // per wave on up to sixteen waves (measured 2-12% faster at up to 384
    // tiles for every type, and for Q6_K up to 688; slower for the other types
    // at 688 tiles)
    if constexpr ((EPI == E_STORE || EPI == E_ACC) && !NORM) {
        const uint32_t nblk = a.cols / 256u;
        if (nblk <= 16u && (total <= 384u || (T::BYTES == 210u && total < 1024u))) {
            p.ks = 1u;
            p.nw = nblk;
        }
    }
    // Fused RMSNorm + Q/K/V launches (measured over the tile and block splits
    // this kernel offers, weights streamed from HBM): rows of at most 16
    // blocks (7B) take two tiles per workgroup on sixteen waves of one block
    // (8.4 -> 7.6 us at 6144 x 4096); rows of 17-32 blocks (70B) eight
    // blocks per wave (18.2 -> 17.0 us at 10240 x 8192).
    if constexpr (EPI == E_QKV) {
        const uint32_t nblk = a.cols / 256u;
        // Q4_K rows of 17-32 blocks (70B: 8192 + 1024 + 1024 rows of 32): an
        // even range of at most three tiles per workgroup on sixteen waves of
        // two blocks, so that no CU streams three tiles while others stream
        // two (640 tiles over 256 CUs)
        if constexpr (std::is_same<T, Q4K>::value) {
            if (nblk > 16u && nblk <= 32u) {
                MvArgs r = a;
                if (ranged_split(r, device_cus()))
                    return launch_t<T, 2, 3, 1024, NORM, EPI, true>(r, 16u, r.rwg_end[2], s);
            }
        }
        if (nblk <= 16u) {
            p.ks = 1u;
            p.nw = nblk;
            // a few tiles (the shim's K + RoPE, 64 tiles): one per workgroup,
            // else two per workgroup would leave most CUs idle
            if (total < device_cus()) return launch_ks<T, NORM, EPI, 1>(a, p, total, s);
            return launch_ks<T, NORM, EPI, 2>(a, p, (total + 1u) / 2u, s);
        }
        if (nblk <= 32u) {
            p.ks = 8u;
            p.nw = (nblk + 7u) / 8u;
        }
    }
    if (p.nw > 16u) return hipErrorNotSupported;
    if constexpr (EPI == E_SILU && std::is_same<T, Q4K>::value) {
        // Q4_K rows of 16 blocks whose tile pairs do not divide evenly over
        // the CUs (7B: 688 over 256) and fit three per CU: an even range of
        // rows per workgroup, three gate and three up tiles on sixteen waves
        // of one block
        const uint32_t cus = device_cus(), rpw = (a.rows[0] + cus - 1u) / cus;
        if (a.cols == 4096u && rpw > 32u && rpw <= 48u && a.tile_end[0] % cus) {
            MvArgs r = a;
            const uint32_t wgs = (a.rows[0] + rpw - 1u) / rpw;
            for (uint32_t m = 0; m < 3u; m++) {
                r.rwg_end[m] = wgs;
                r.rpw[m] = rpw;
            }
            return launch_t<T, 1, 6, 1024, NORM, EPI, true>(r, 16u, wgs, s);
        }
    }
    if constexpr (EPI == E_SILU)  // a gate tile and the same up tile
        return launch_ks<T, NORM, EPI, 2>(a, p, a.tile_end[0], s);
    // Unfused Q4_K launches of rows of 17-32 blocks with at least two tiles
    // per CU: two tiles per workgroup, a block's x operands serving both
    // (measured at 8192 x 8192: 11.2-11.5 -> 10.4-10.7 us; four tiles, which
    // leave half the CUs idle there, and the fused Q/K/V launch were slower)
    if constexpr ((EPI == E_STORE || EPI == E_ACC) && !NORM && std::is_same<T, Q4K>::value) {
        if (p.ks == 4u && total >= 2u * device_cus() && total < 1024u)
            return launch_ks<T, NORM, EPI, 2>(a, p, (total + 1u) / 2u, s);
    }
    // Launches that would need several rounds of resident workgroups give each
    // workgroup four tiles instead: x (and the RMSNorm) is prepared once per
    // four tiles and every workgroup is resident from the start.
    if constexpr (EPI == E_STORE || EPI == E_ACC) {
        if (total >= 1024u) return launch_ks<T, NORM, EPI, 4>(a, p, (total + 3u) / 4u, s);
    }
    return launch_ks<T, NORM, EPI, 1>(a, p, total, s);
}

// Shape and alignment range of the matrix-core path: at most 16 waves of at
// most 8 super-blocks (the digits of x and the Q6_K scratch must also fit the
// LDS, else the launch reports it unsupported); Q4_K rows are 16-byte
// multiples, so its 16-byte loads need an aligned w; Q6_K aligns every load.
// The 32-element block types (batch-1 store / accumulate launches only).
static inline bool mv_fits_blk(int type, const uint8_t *w, const float *x, uint32_t cols, uint32_t rows) {
    if (type != kQ4_0 && type != kQ4_1 && type != kQ8_0) return false;
    if (cols % 256u || cols / 256u > 128u || ((uintptr_t)x & 3u) || ((uintptr_t)w & 1u)) return false;
    return (uint64_t)rows * row_bytes(type, cols) + 256u < (1ull << 32);
}

static inline bool mv_fits(int type, const uint8_t *w, const float *x, uint32_t cols, uint32_t rows) {
    if (type != kQ4_K && type != kQ6_K) return false;
    if (cols % 256u || cols / 256u > 128u || ((uintptr_t)x & 3u)) return false;
    // (32-bit offsets: the matrix and the 16-byte chunks around it)
    if ((uint64_t)rows * (cols / 256u) * (type == kQ4_K ? 144u : 210u) + 256u >= (1ull << 32)) return false;
    return ((uintptr_t)w & (type == kQ4_K ? 15u : 1u)) == 0;
}

static inline void set_tiles(MvArgs &a) {
    uint32_t t = 0;
    for (uint32_t m = 0; m < a.nmat; m++) {
        t += (a.rows[m] + 15u) / 16u;
        a.tile_end[m] = t;
    }
}

}  // namespace vbs
