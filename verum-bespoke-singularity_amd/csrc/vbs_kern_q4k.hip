// vbs_kern_q4k.hip — batch-1 Q4_K matvec on the vector ALUs (v_dot4), for the
// matrices the matrix-core kernels do not take: 4 GiB of weights or more (their
// offsets are 32-bit). Rows up to 32768 columns, 16-byte aligned weights.
//
// y[r] (+)= sum_c deq(W[r,c]) * x[c], W in native GGUF Q4_K super-blocks
// (144 B: f16 d, f16 dmin, 12 B of 6-bit scales/mins, 128 B of nibbles;
// src/vbs_dequant.c:225-277).
//
// Design
//  * One workgroup per CU (<= 1024 threads) streams many rows and keeps x in
//    registers. Lane (b, g) of a wave owns the 64 elements of group g of
//    super-block b: per row it issues three 128-bit loads (the 16-B header,
//    shared by the 4 lanes of the block, and its 32 B of nibbles). A wave
//    covers 16 super-blocks (4096 columns); wider rows use several waves per
//    row and combine their partial sums in LDS. Each wave keeps R rows of
//    loads in flight and refills a slot as soon as it has consumed it; the
//    first R rows are requested before x is prepared, so HBM latency overlaps
//    the preparation.
//  * x is turned, once per workgroup, into an exact integer form per 32-element
//    sub-block: X_i = rint(x_i * 2^(22-e)) with 2^e > max|x| (|X| <= 2^22),
//    split into three signed bytes (X = D2*2^16 + D1*2^8 + D0). The weight
//    nibbles then meet x through v_dot4_i32_i8: sum_i n_i*X_i is computed
//    exactly in int32, three dot4 per 4 weights, and scaled back by 2^(e-22).
//    x is thereby represented to 2^-22 of its sub-block maximum (fp32 itself
//    keeps 2^-23 relative), which keeps the row result within ~1e-7 of the
//    double-accumulated reference. A sub-block holding inf or NaN yields NaN.
//  * The reference's value is d*sc*nib - dmin*m per element; summed over a
//    sub-block that is d*sc*sum(nib*x) - dmin*m*sum(x), so the per-element
//    scale multiply disappears and sum(x) is computed once per sub-block.
//  * Row sums use DPP cross-lane adds (quad perms, row mirrors, row
//    broadcasts) — no LDS traffic inside a wave.
#include "vbs_dev_common.h"
#include "vbs_internal.h"

namespace vbs {

constexpr uint32_t kQ4kMaxCols = 32768;  // LDS holds 3 digit planes of x

// v moved across lanes by one DPP control; lanes of rows outside ROW_MASK get 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes; the total is returned to every lane.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_f<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141, 0xF>(v);  // row_half_mirror
    v += dpp_f<0x140, 0xF>(v);  // row_mirror: each 16-lane row holds its sum
    v += dpp_f<0x142, 0xA>(v);  // row_bcast15 into rows 1 and 3
    v += dpp_f<0x143, 0xC>(v);  // row_bcast31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Plain (temporal) loads: each cache line of a row is touched by three load
// instructions of the wave, and a non-temporal hint evicts it in between.
__device__ __forceinline__ u32x4 ld128(const uint8_t *p) {
    return *reinterpret_cast<const u32x4 *>(p);
}

// Exact f16 -> f32 with the hardware converter (v_cvt_f32_f16).
__device__ __forceinline__ float hw_h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 255) | ((uint32_t)(b & 255) << 8) | ((uint32_t)(c & 255) << 16) |
           ((uint32_t)d << 24);
}

// Partial row sum of one lane: 64 nibbles (two sub-blocks) against its digits.
__device__ __forceinline__ float q4k_lane_dot(u32x4 hdr, u32x4 qa, u32x4 qb, const uint32_t *P0,
                                              const uint32_t *P1, const uint32_t *P2,
                                              uint32_t half_sh, bool upper, float xs_lo,
                                              float xs_hi, float xm_lo, float xm_hi) {
    const uint32_t qd[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    int a0l = 0, a1l = 0, a2l = 0, a0h = 0, a1h = 0, a2h = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int lo = (int)(qd[j] & 0x0F0F0F0Fu);
        const int hi = (int)((qd[j] >> 4) & 0x0F0F0F0Fu);
        a0l = __builtin_amdgcn_sdot4(lo, (int)P0[j], a0l, false);
        a1l = __builtin_amdgcn_sdot4(lo, (int)P1[j], a1l, false);
        a2l = __builtin_amdgcn_sdot4(lo, (int)P2[j], a2l, false);
        a0h = __builtin_amdgcn_sdot4(hi, (int)P0[8 + j], a0h, false);
        a1h = __builtin_amdgcn_sdot4(hi, (int)P1[8 + j], a1h, false);
        a2h = __builtin_amdgcn_sdot4(hi, (int)P2[8 + j], a2h, false);
    }
    // digits 0 and 1 combine exactly in int32 (|a0 + 256*a1| < 2^24)
    const float S_lo = fmaf((float)a2l, 65536.f, (float)(a0l + a1l * 256));
    const float S_hi = fmaf((float)a2h, 65536.f, (float)(a0h + a1h * 256));
    const float d = hw_h2f(hdr.x & 0xFFFFu);
    const float dmin = hw_h2f(hdr.x >> 16);
    // scale/min bytes of sub-blocks j = 2g, 2g+1 (src/vbs_dequant.c:225-233)
    const uint32_t Y = (hdr.y >> half_sh) & 0xFFFFu;  // s[j]   (j-4 when upper)
    const uint32_t Z = (hdr.z >> half_sh) & 0xFFFFu;  // s[j+4] (j when upper)
    const uint32_t W = (hdr.w >> half_sh) & 0xFFFFu;  // s[j+8] (j+4 when upper)
    uint32_t sc_lo, sc_hi, m_lo, m_hi;
    if (upper) {
        sc_lo = (W & 15u) | ((Y >> 2) & 0x30u);
        sc_hi = ((W >> 8) & 15u) | ((Y >> 10) & 0x30u);
        m_lo = ((W >> 4) & 15u) | ((Z >> 2) & 0x30u);
        m_hi = ((W >> 12) & 15u) | ((Z >> 10) & 0x30u);
    } else {
        sc_lo = Y & 63u;
        sc_hi = (Y >> 8) & 63u;
        m_lo = Z & 63u;
        m_hi = (Z >> 8) & 63u;
    }
    return d * ((float)sc_lo * xs_lo * S_lo + (float)sc_hi * xs_hi * S_hi) -
           dmin * ((float)m_lo * xm_lo + (float)m_hi * xm_hi);
}

// One 16-element half of a sub-block of x: load it (float4 when aligned).
__device__ __forceinline__ void x_load16(const float *x, bool x16, uint32_t item, bool valid,
                                         float *v) {
    const float *xp = x + (valid ? item * 16u : 0u);
    if (x16) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = reinterpret_cast<const float4 *>(xp)[q];
            v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; k++) v[k] = xp[k];
    }
}

// Exponent, sum and three signed digit planes of one half sub-block; the two
// halves of a sub-block are adjacent lanes (item and item ^ 1).
__device__ __forceinline__ void x_prep16(const float *v, uint32_t item, bool valid,
                                         uint8_t *planes, float *xsc, float *xsm, uint32_t cols) {
    float amax = 0.f, sum = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        amax = fmaxf(amax, fabsf(v[k]));
        sum += v[k];
    }
    const uint32_t h = item & 1u;
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    const float other = __shfl_xor(sum, 1, 64);
    sum = h ? other + sum : sum + other;  // same order in both lanes
    if (!valid) return;
    int e;
    (void)frexpf(amax, &e);  // amax < 2^e
    const bool finite = amax <= 3.4028235e38f;
    uint32_t d0[4], d1[4], d2[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        int D0[4], D1[4], D2[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int X = finite ? __float2int_rn(ldexpf(v[4 * q + k], 22 - e)) : 0;
            const int a = (int)(int8_t)X;
            const int X1 = (X - a) >> 8;
            const int c = (int)(int8_t)X1;
            D0[k] = a;
            D1[k] = c;
            D2[k] = (X1 - c) >> 8;
        }
        d0[q] = pack4(D0[0], D0[1], D0[2], D0[3]);
        d1[q] = pack4(D1[0], D1[1], D1[2], D1[3]);
        d2[q] = pack4(D2[0], D2[1], D2[2], D2[3]);
    }
    const uint32_t off = item * 16u, sb = item >> 1;
    *reinterpret_cast<uint4 *>(planes + off) = make_uint4(d0[0], d0[1], d0[2], d0[3]);
    *reinterpret_cast<uint4 *>(planes + cols + off) = make_uint4(d1[0], d1[1], d1[2], d1[3]);
    *reinterpret_cast<uint4 *>(planes + 2u * cols + off) = make_uint4(d2[0], d2[1], d2[2], d2[3]);
    if (h == 0) {
        xsc[sb] = finite ? ldexpf(1.0f, e - 22) : __builtin_nanf("");
        xsm[sb] = sum;
    }
}

template <uint32_t R, bool X2>
__global__ __launch_bounds__(1024) void k_q4k_mv(const uint8_t *__restrict__ w,
                                                 const float *__restrict__ x,
                                                 float *__restrict__ y, uint32_t cols,
                                                 uint32_t rows, int accumulate, uint32_t nw,
                                                 uint32_t streams) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t nblk = cols >> 8, nsub = cols >> 5;
    const uint64_t rb = (uint64_t)nblk * 144u;
    uint8_t *planes = lds;                                    // [3][cols] int8 digits
    float *xsc = reinterpret_cast<float *>(lds + 3u * cols);  // [nsub] 2^(e-22)
    float *xsm = xsc + nsub;                                  // [nsub] sum(x)
    float *red = xsm + nsub;                                  // [streams][R][nw]
    const uint32_t tid = threadIdx.x, nth = blockDim.x;

    // ---- x first: VMEM loads return in order, so the preparation must not be
    // queued behind the weight stream. Each thread prepares <= 2 half sub-blocks.
    const bool x16 = ((uintptr_t)x & 15u) == 0;
    const uint32_t items = 2u * nsub;
    const uint32_t i0 = tid, i1 = tid + nth;
    float v0[16];
    x_load16(x, x16, i0, i0 < items, v0);

    // ---- lane identity; request this wave's first R rows ---------------------
    const uint32_t wave = tid >> 6, lane = tid & 63u;
    const uint32_t s = wave / nw, wr = wave % nw;
    const uint32_t b = wr * 16u + (lane >> 2), g = lane & 3u;
    const bool act = b < nblk;
    // lanes past the last block re-read the last block (in bounds, same cache
    // lines as their neighbours) and contribute zero; rows past the end re-read
    // the last row and are not stored
    const uint64_t boff = (uint64_t)(act ? b : nblk - 1u) * 144u;
    const uint32_t wstride = gridDim.x * streams;
    const uint32_t first = blockIdx.x * streams + s;
    const uint32_t last = rows - 1u;
    u32x4 hdr[R], qa[R], qb[R];
#pragma unroll
    for (uint32_t k = 0; k < R; k++) {
        const uint8_t *p = w + (uint64_t)min(first + k * wstride, last) * rb + boff;
        hdr[k] = ld128(p);
        qa[k] = ld128(p + 16u + 32u * g);
        qb[k] = ld128(p + 32u + 32u * g);
    }

    // keep the weight loads behind the x loads in the instruction stream
    __builtin_amdgcn_sched_barrier(0);

    // ---- x -> per-sub-block exponent + three signed digit planes (LDS) ------
    x_prep16(v0, i0, i0 < items, planes, xsc, xsm, cols);
    if (X2) {  // rows wider than 16 x threads: a second half sub-block per thread
        float v1[16];
        x_load16(x, x16, i1, i1 < items, v1);
        x_prep16(v1, i1, i1 < items, planes, xsc, xsm, cols);
    }
    __syncthreads();

    // ---- per-lane constants: its 64 elements of x as digits ---------------
    uint32_t P0[16], P1[16], P2[16];
    float xs_lo, xs_hi, xm_lo, xm_hi;
    {
        const uint32_t base = (act ? b : 0u) * 256u + g * 64u;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 a = *reinterpret_cast<const uint4 *>(planes + base + 16u * q);
            const uint4 c = *reinterpret_cast<const uint4 *>(planes + cols + base + 16u * q);
            const uint4 e = *reinterpret_cast<const uint4 *>(planes + 2u * cols + base + 16u * q);
            P0[4 * q] = a.x; P0[4 * q + 1] = a.y; P0[4 * q + 2] = a.z; P0[4 * q + 3] = a.w;
            P1[4 * q] = c.x; P1[4 * q + 1] = c.y; P1[4 * q + 2] = c.z; P1[4 * q + 3] = c.w;
            P2[4 * q] = e.x; P2[4 * q + 1] = e.y; P2[4 * q + 2] = e.z; P2[4 * q + 3] = e.w;
        }
        const uint32_t sb = (act ? b : 0u) * 8u + 2u * g;
        xs_lo = xsc[sb];
        xs_hi = xsc[sb + 1];
        xm_lo = xsm[sb];
        xm_hi = xsm[sb + 1];
    }
    const uint32_t half_sh = 16u * (g & 1u);
    const bool upper = g >= 2u;

    // ---- rows: compute all R slots, then store (stores are deferred so the
    // waits for the next slot's data stay exact) ------------------------------
    for (uint32_t it = 0; (uint64_t)it * R * wstride < rows; it++) {
        if (it > 0) {  // uniform: a further round of this wave's rows
#pragma unroll
            for (uint32_t k = 0; k < R; k++) {
                const uint8_t *p =
                    w + (uint64_t)min(first + (it * R + k) * wstride, last) * rb + boff;
                hdr[k] = ld128(p);
                qa[k] = ld128(p + 16u + 32u * g);
                qb[k] = ld128(p + 32u + 32u * g);
            }
        }
        float tot[R];
#pragma unroll
        for (uint32_t k = 0; k < R; k++) {
            tot[k] = 0.f;
            if (first + (it * R + k) * wstride < rows) {  // uniform: skip the tail slots
                const float part = q4k_lane_dot(hdr[k], qa[k], qb[k], P0, P1, P2, half_sh,
                                                upper, xs_lo, xs_hi, xm_lo, xm_hi);
                tot[k] = wave_sum_dpp(act ? part : 0.f);
            }
        }
        if (nw == 1) {
            if (lane < R) {
                float t = tot[0];
#pragma unroll
                for (uint32_t k = 1; k < R; k++) t = lane == k ? tot[k] : t;
                const uint32_t row = first + (it * R + lane) * wstride;
                if (row < rows) y[row] = accumulate ? y[row] + t : t;
            }
        } else {
            if (lane < R) {
                float t = tot[0];
#pragma unroll
                for (uint32_t k = 1; k < R; k++) t = lane == k ? tot[k] : t;
                red[(s * R + lane) * nw + wr] = t;
            }
            __syncthreads();
            if (wr == 0 && lane < R) {
                const uint32_t row = first + (it * R + lane) * wstride;
                if (row < rows) {
                    float t = 0.f;
                    for (uint32_t k = 0; k < nw; k++) t += red[(s * R + lane) * nw + k];
                    y[row] = accumulate ? y[row] + t : t;
                }
            }
            __syncthreads();
        }
    }
}

template <uint32_t R, bool X2>
static hipError_t launch_r(dim3 grid, dim3 block, size_t lds, hipStream_t s, const uint8_t *w,
                           const float *x, float *y, uint32_t cols, uint32_t rows, int acc,
                           uint32_t nw, uint32_t streams) {
    if (lds > 65536u) {  // beyond the default per-workgroup LDS window: opt in once
        static size_t granted = 0;
        if (lds > granted) {
            if (hipFuncSetAttribute((const void *)k_q4k_mv<R, X2>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
                hipSuccess) {
                (void)hipGetLastError();
                return hipErrorNotSupported;
            }
            granted = lds;
        }
    }
    k_q4k_mv<R, X2><<<grid, block, lds, s>>>(w, x, y, cols, rows, acc, nw, streams);
    return hipGetLastError();
}

// Returns hipErrorNotSupported when the shape is outside this kernel's range
// (the caller then uses the generic kernel).
hipError_t launch_q4k_fast(const uint8_t *w, const float *x, float *y, uint32_t cols,
                           uint32_t rows, int accumulate, hipStream_t s) {
    const uint32_t nblk = cols / 256u;
    if (cols % 256u || cols > kQ4kMaxCols || nblk == 0 || rows == 0) return hipErrorNotSupported;
    if (((uintptr_t)w & 15u) || ((uintptr_t)x & 3u)) return hipErrorNotSupported;
    const uint32_t nw = (nblk + 15u) / 16u;  // waves per row
    if (nw > 16u) return hipErrorNotSupported;
    const uint32_t cus = 256u;
    // streams (independent row walkers) per workgroup; at least cols/16 threads
    // so each prepares one half sub-block of x (two when the row is very wide)
    uint32_t min_streams = (cols / 16u + nw * 64u - 1u) / (nw * 64u);
    if (min_streams * nw > 16u) min_streams = (cols / 32u + nw * 64u - 1u) / (nw * 64u);
    auto rounds = [&](uint32_t g, uint32_t st) { return (rows + g * st - 1u) / (g * st); };
    // A: one 16-wave workgroup per CU; B: two smaller ones per CU. Measured on
    // the 7B shapes: A wins when every wave holds one row, B when waves hold
    // several rows or a row spans several waves.
    uint32_t stA = 16u / nw < min_streams ? min_streams : 16u / nw;
    uint32_t stB = 8u / nw < min_streams ? min_streams : (8u / nw ? 8u / nw : 1u);
    if (stB * nw > 16u) stB = stA;
    uint32_t grid = cus, streams = stA;
    if (rounds(cus, stA) > 1u && rounds(2u * cus, stB) <= 3u) {
        grid = 2u * cus;
        streams = stB;
    }
    if (rows < grid * streams) {  // short matrix: one row per wave, spread over the CUs
        uint32_t st = (rows + cus - 1u) / cus;
        streams = st < min_streams ? min_streams : st;
        grid = (rows + streams - 1u) / streams;
        if (grid > cus) grid = cus;
    }
    const uint32_t per_stream = rounds(grid, streams);
    // at most three rows in flight per wave (the 128-VGPR budget of 16 waves/CU)
    const uint32_t R = per_stream < 3u ? per_stream : 3u;
    const size_t lds = 3u * (size_t)cols + 8u * (cols / 32u) + 4u * (size_t)streams * 3u * nw;
    const dim3 g(grid), blk(streams * nw * 64u);
    const bool x2 = cols / 16u > streams * nw * 64u;
#define VBS_Q4K_LAUNCH(RR)                                                                      \
    return x2 ? launch_r<RR, true>(g, blk, lds, s, w, x, y, cols, rows, accumulate, nw, streams) \
              : launch_r<RR, false>(g, blk, lds, s, w, x, y, cols, rows, accumulate, nw, streams)
    switch (R) {
        case 1: VBS_Q4K_LAUNCH(1);
        case 2: VBS_Q4K_LAUNCH(2);
        default: VBS_Q4K_LAUNCH(3);
    }
#undef VBS_Q4K_LAUNCH
}

}  // namespace vbs
