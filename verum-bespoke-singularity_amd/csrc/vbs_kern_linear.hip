// vbs_kern_linear.hip — batch-1 linear (matvec) kernels for every hot-path
// weight type, plus the batched (skinny) variant.
//
// Semantics: vbs_host_linear_tile (src/vbs_host_math.h:223-267) —
// y[r] (+)= sum_c deq(W[r,c]) * x[c]. Each weight is dequantised with the
// reference's exact roundings (vbs_dev_common.h) and then accumulated in
// fp32 with fused multiply-adds; rows are reduced across the wavefront.
//
// Work split: a wavefront owns one row; its 64 lanes walk the row's 32-element
// units (a legacy block, or one sub-block of a 256-element super-block).
#include "vbs_dev_common.h"
#include "vbs_internal.h"

namespace vbs {

// Dot of unit u (elements 32u .. 32u+31) of a packed row with x.
template <int T> __device__ __forceinline__ float unit_dot(const uint8_t *row, uint32_t u,
                                                          const float *x);

template <> __device__ __forceinline__ float unit_dot<kQ4_0>(const uint8_t *row, uint32_t u,
                                                            const float *x) {
    const uint8_t *b = row + 18u * u;
    const float *xb = x + 32u * u;
    float d = h2f(ld16(b));
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
        uint16_t two = ld16(b + 2 + i);
#pragma unroll
        for (int k = 0; k < 2; k++) {
            uint32_t byte = (two >> (8 * k)) & 255u;
            float lo = __fmul_rn((float)(byte & 15u) - 8.0f, d);
            float hi = __fmul_rn((float)(byte >> 4) - 8.0f, d);
            acc = fmaf(lo, xb[i + k], acc);
            acc = fmaf(hi, xb[16 + i + k], acc);
        }
    }
    return acc;
}

template <> __device__ __forceinline__ float unit_dot<kQ4_1>(const uint8_t *row, uint32_t u,
                                                            const float *x) {
    const uint8_t *b = row + 20u * u;
    const float *xb = x + 32u * u;
    float d = h2f(ld16(b)), m = h2f(ld16(b + 2));
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
        uint16_t two = ld16(b + 4 + i);
#pragma unroll
        for (int k = 0; k < 2; k++) {
            uint32_t byte = (two >> (8 * k)) & 255u;
            float lo = __fadd_rn(__fmul_rn(d, (float)(byte & 15u)), m);
            float hi = __fadd_rn(__fmul_rn(d, (float)(byte >> 4)), m);
            acc = fmaf(lo, xb[i + k], acc);
            acc = fmaf(hi, xb[16 + i + k], acc);
        }
    }
    return acc;
}

template <> __device__ __forceinline__ float unit_dot<kQ8_0>(const uint8_t *row, uint32_t u,
                                                            const float *x) {
    const uint8_t *b = row + 34u * u;
    const float *xb = x + 32u * u;
    float d = h2f(ld16(b));
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
        uint16_t two = ld16(b + 2 + i);
        acc = fmaf(__fmul_rn(d, (float)(int8_t)(two & 255u)), xb[i], acc);
        acc = fmaf(__fmul_rn(d, (float)(int8_t)(two >> 8)), xb[i + 1], acc);
    }
    return acc;
}

template <> __device__ __forceinline__ float unit_dot<kQ4_K>(const uint8_t *row, uint32_t u,
                                                            const float *x) {
    const uint8_t *b = row + 144u * (u >> 3);
    uint32_t j = u & 7u;
    const float *xb = x + 32u * u;
    float d = h2f(ld16(b)), dmin = h2f(ld16(b + 2));
    int sc, mn;
    q4k_scale_min(b + 4, (int)j, sc, mn);
    float dsc = __fmul_rn(d, (float)sc), dm = __fmul_rn(dmin, (float)mn);
    const uint8_t *qs = b + 16 + 32 * (j >> 1);
    uint32_t shift = (j & 1u) * 4u;
    float acc = 0.f;
#pragma unroll
    for (int l = 0; l < 32; l += 2) {
        uint16_t two = ld16(qs + l);
        float w0 = __fsub_rn(__fmul_rn(dsc, (float)((two >> shift) & 15u)), dm);
        float w1 = __fsub_rn(__fmul_rn(dsc, (float)((two >> (8u + shift)) & 15u)), dm);
        acc = fmaf(w0, xb[l], acc);
        acc = fmaf(w1, xb[l + 1], acc);
    }
    return acc;
}

template <> __device__ __forceinline__ float unit_dot<kQ6_K>(const uint8_t *row, uint32_t u,
                                                            const float *x) {
    const uint8_t *b = row + 210u * (u >> 3);
    uint32_t j = u & 7u, h = j >> 2, q = j & 3u;
    const float *xb = x + 32u * u;
    float d = h2f(ld16(b + 208));
    float s0 = __fmul_rn(d, (float)(int8_t)b[192 + 8 * h + 2 * q]);
    float s1 = __fmul_rn(d, (float)(int8_t)b[192 + 8 * h + 2 * q + 1]);
    const uint8_t *ql = b + 64 * h + 32 * (q & 1u);
    const uint8_t *qh = b + 128 + 32 * h;
    uint32_t lsh = q >= 2 ? 4u : 0u, hsh = 2u * q;
    float acc = 0.f;
#pragma unroll
    for (int l = 0; l < 32; l += 2) {
        uint16_t lo2 = ld16(ql + l), hi2 = ld16(qh + l);
#pragma unroll
        for (int k = 0; k < 2; k++) {
            int lo = (lo2 >> (8 * k + lsh)) & 15;
            int hi = (hi2 >> (8 * k + hsh)) & 3;
            float s = (l + k) < 16 ? s0 : s1;
            acc = fmaf(__fmul_rn(s, (float)((lo | (hi << 4)) - 32)), xb[l + k], acc);
        }
    }
    return acc;
}

template <> __device__ __forceinline__ float unit_dot<kLNS8>(const uint8_t *row, uint32_t u,
                                                            const float *x) {
    const uint8_t *b = row + 36u * u;
    const float *xb = x + 32u * u;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) acc = fmaf(deq_elem<kLNS8>(b, i), xb[i], acc);
    return acc;
}

template <int T>
__global__ __launch_bounds__(256) void k_linear_units(const uint8_t *__restrict__ w,
                                                      const float *__restrict__ x,
                                                      float *__restrict__ y, uint32_t cols,
                                                      uint32_t rows, uint64_t rb, int accumulate) {
    uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    uint32_t lane = threadIdx.x & 63u;
    if (row >= rows) return;  // uniform per wavefront
    const uint8_t *rp = w + (uint64_t)row * rb;
    float acc = 0.f;
    for (uint32_t u = lane; u < cols / 32u; u += 64u) acc += unit_dot<T>(rp, u, x);
    acc = wave_sum(acc);
    if (lane == 0) y[row] = accumulate ? y[row] + acc : acc;
}

// F32 / F16 rows: element-granular (cols need not be a multiple of 32).
template <int T>
__global__ __launch_bounds__(256) void k_linear_dense(const uint8_t *__restrict__ w,
                                                      const float *__restrict__ x,
                                                      float *__restrict__ y, uint32_t cols,
                                                      uint32_t rows, uint64_t rb, int accumulate) {
    uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    uint32_t lane = threadIdx.x & 63u;
    if (row >= rows) return;
    const uint8_t *rp = w + (uint64_t)row * rb;
    float acc = 0.f;
    for (uint32_t c = lane; c < cols; c += 64u) acc = fmaf(deq_elem<T>(rp, c), x[c], acc);
    acc = wave_sum(acc);
    if (lane == 0) y[row] = accumulate ? y[row] + acc : acc;
}

hipError_t launch_linear(int type, const uint8_t *w, const float *x, float *y, uint32_t cols,
                         uint32_t rows, int accumulate, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (type == kQ4_K || type == kQ6_K || type == kQ4_0 || type == kQ4_1 || type == kQ8_0) {
        hipError_t e = launch_kq_linear(type, w, x, y, cols, rows, accumulate, s);
        if (e != hipErrorNotSupported) return e;
    }
    if (type == kQ4_K) {
        hipError_t e = launch_q4k_fast(w, x, y, cols, rows, accumulate, s);
        if (e != hipErrorNotSupported) return e;
    }
    uint64_t rb = row_bytes(type, cols);
    dim3 grid((rows + 3u) / 4u), block(256);
    switch (type) {
        case kF32: k_linear_dense<kF32><<<grid, block, 0, s>>>(w, x, y, cols, rows, rb, accumulate); break;
        case kF16: k_linear_dense<kF16><<<grid, block, 0, s>>>(w, x, y, cols, rows, rb, accumulate); break;
        case kQ4_0: k_linear_units<kQ4_0><<<grid, block, 0, s>>>(w, x, y, cols, rows, rb, accumulate); break;
        case kQ4_1: k_linear_units<kQ4_1><<<grid, block, 0, s>>>(w, x, y, cols, rows, rb, accumulate); break;
        case kQ8_0: k_linear_units<kQ8_0><<<grid, block, 0, s>>>(w, x, y, cols, rows, rb, accumulate); break;
        case kQ4_K: k_linear_units<kQ4_K><<<grid, block, 0, s>>>(w, x, y, cols, rows, rb, accumulate); break;
        case kQ6_K: k_linear_units<kQ6_K><<<grid, block, 0, s>>>(w, x, y, cols, rows, rb, accumulate); break;
        case kLNS8: k_linear_units<kLNS8><<<grid, block, 0, s>>>(w, x, y, cols, rows, rb, accumulate); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Batched: a wavefront owns one row and loops the batch, so each weight unit
// is decoded once and used `batch` times (weights read once from HBM).
template <int T, int NB>
__global__ __launch_bounds__(256) void k_linear_batch(const uint8_t *__restrict__ w,
                                                      const float *__restrict__ x, uint32_t xs,
                                                      float *__restrict__ y, uint32_t ys,
                                                      uint32_t cols, uint32_t rows, uint64_t rb,
                                                      uint32_t batch) {
    uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    uint32_t lane = threadIdx.x & 63u;
    if (row >= rows) return;
    const uint8_t *rp = w + (uint64_t)row * rb;
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = 0.f;
    if (Geo<T>::E == 1) {
        for (uint32_t c = lane; c < cols; c += 64u) {
            float wv = deq_elem<T>(rp, c);
#pragma unroll
            for (int b = 0; b < NB; b++)
                if ((uint32_t)b < batch) acc[b] = fmaf(wv, x[(uint64_t)b * xs + c], acc[b]);
        }
    } else {
        float wv[32];
        for (uint32_t u = lane; u < cols / 32u; u += 64u) {
            const uint8_t *blk = rp + (uint64_t)(u / (Geo<T>::E / 32u)) * Geo<T>::B;
            uint32_t e0 = (u % (Geo<T>::E / 32u)) * 32u;
#pragma unroll
            for (int i = 0; i < 32; i++) wv[i] = deq_elem<T>(blk, e0 + i);
#pragma unroll
            for (int b = 0; b < NB; b++) {
                if ((uint32_t)b < batch) {
                    const float *xb = x + (uint64_t)b * xs + 32u * u;
                    float a = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; i++) a = fmaf(wv[i], xb[i], a);
                    acc[b] += a;
                }
            }
        }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        if ((uint32_t)b < batch) {
            float t = wave_sum(acc[b]);
            if (lane == 0) y[(uint64_t)b * ys + row] = t;
        }
    }
}

hipError_t launch_linear_batch(int type, const uint8_t *w, const float *x, uint32_t xs, float *y,
                               uint32_t ys, uint32_t cols, uint32_t rows, uint32_t batch,
                               hipStream_t s) {
    if (rows == 0 || batch == 0) return hipSuccess;
    // K-quants: the matrix-core kernel, eight vectors per launch
    if (type == kQ4_K || type == kQ6_K) {
        hipError_t e = hipSuccess;
        for (uint32_t b0 = 0; b0 < batch && e == hipSuccess; b0 += 8u)
            e = launch_kq_linear_batch(type, w, x + (uint64_t)b0 * xs, xs, y + (uint64_t)b0 * ys, ys,
                                       cols, rows, min(8u, batch - b0), s);
        if (e != hipErrorNotSupported) return e;  // the shape check fails on the first launch
    }
    uint64_t rb = row_bytes(type, cols);
    dim3 grid((rows + 3u) / 4u), block(256);
#define VBS_LB(T) k_linear_batch<T, 16><<<grid, block, 0, s>>>(w, x, xs, y, ys, cols, rows, rb, batch)
    switch (type) {
        case kF32: VBS_LB(kF32); break;
        case kF16: VBS_LB(kF16); break;
        case kQ4_0: VBS_LB(kQ4_0); break;
        case kQ4_1: VBS_LB(kQ4_1); break;
        case kQ8_0: VBS_LB(kQ8_0); break;
        case kQ4_K: VBS_LB(kQ4_K); break;
        case kQ6_K: VBS_LB(kQ6_K); break;
        case kLNS8: VBS_LB(kLNS8); break;
        default: return hipErrorInvalidValue;
    }
#undef VBS_LB
    return hipGetLastError();
}

}  // namespace vbs
