// vbs_kern_prims.hip — gather, RMSNorm, RoPE, KV-cache store, SiLU*up and
// residual add for gfx950.
//
// Gather, KV store, RoPE and add are bit-identical to the reference host math;
// RMSNorm accumulates the sum of squares in double as the reference does
// (src/vbs_host_math.h:30-35), so it matches to the last bit except in the
// rare case where the double sums (different order) round to different floats.
#include "vbs_dev_common.h"
#include "vbs_internal.h"

namespace vbs {

// ---- embedding gather / row dequantisation --------------------------------
// out[r*dim + e] = deq(row ids[r] (or `token` when ids is NULL and n_rows==1,
// or row r when ids is NULL), element e). src/vbs_host_math.h:94-142.
template <int T>
__global__ __launch_bounds__(256) void k_dequant_rows(const uint8_t *__restrict__ w, uint64_t rb,
                                                      const uint32_t *__restrict__ ids,
                                                      uint32_t token, uint32_t dim,
                                                      float *__restrict__ out) {
    uint32_t e = blockIdx.x * 256u + threadIdx.x;
    uint32_t r = blockIdx.y;
    if (e >= dim) return;
    uint32_t src = ids ? ids[r] : (token != 0xFFFFFFFFu ? token : r);
    const uint8_t *row = w + (uint64_t)src * rb;
    const uint8_t *blk = row + (uint64_t)(e / Geo<T>::E) * Geo<T>::B;
    out[(uint64_t)r * dim + e] = deq_elem<T>(blk, e % Geo<T>::E);
}

hipError_t launch_dequant_rows(int type, const uint8_t *w, const uint32_t *ids, uint32_t token,
                               uint32_t n_rows, uint32_t dim, float *out, hipStream_t s) {
    if (n_rows == 0 || dim == 0) return hipSuccess;
    uint64_t rb = row_bytes(type, dim);
    dim3 grid((dim + 255u) / 256u, n_rows), block(256);
    switch (type) {
        case kF32: k_dequant_rows<kF32><<<grid, block, 0, s>>>(w, rb, ids, token, dim, out); break;
        case kF16: k_dequant_rows<kF16><<<grid, block, 0, s>>>(w, rb, ids, token, dim, out); break;
        case kQ4_0: k_dequant_rows<kQ4_0><<<grid, block, 0, s>>>(w, rb, ids, token, dim, out); break;
        case kQ4_1: k_dequant_rows<kQ4_1><<<grid, block, 0, s>>>(w, rb, ids, token, dim, out); break;
        case kQ8_0: k_dequant_rows<kQ8_0><<<grid, block, 0, s>>>(w, rb, ids, token, dim, out); break;
        case kQ4_K: k_dequant_rows<kQ4_K><<<grid, block, 0, s>>>(w, rb, ids, token, dim, out); break;
        case kQ6_K: k_dequant_rows<kQ6_K><<<grid, block, 0, s>>>(w, rb, ids, token, dim, out); break;
        case kLNS8: k_dequant_rows<kLNS8><<<grid, block, 0, s>>>(w, rb, ids, token, dim, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- RMSNorm (src/vbs_host_math.h:28-36) -----------------------------------
// ss = sum of x^2 in double, in a fixed order that any block size reproduces
// (the matrix-core matvec's fused RMSNorm uses the same): x in blocks of 256
// elements; in a block, lane l of a wave adds the squares of elements
// 4l..4l+3 in element order, a wave butterfly adds the 64 lanes, and the
// blocks are added in index order. Then, as the reference,
// scale = 1 / sqrtf((float)(ss / n) + eps) and out = x * scale * w.
__global__ __launch_bounds__(1024) void k_rms_norm(const float *__restrict__ in,
                                                   const float *__restrict__ w,
                                                   float *__restrict__ out, uint32_t n,
                                                   float eps) {
    extern __shared__ double bpart[];  // one entry per 256-element block
    __shared__ float s_scale;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t blocks = (n + 255u) / 256u;
    // the wave's first block (x and the norm weights) is requested up front and
    // kept in registers for the output; later blocks (n > 4096) are re-read
    float xr[4] = {0.f, 0.f, 0.f, 0.f}, wr[4] = {0.f, 0.f, 0.f, 0.f};
    if (wave < blocks) {
#pragma unroll
        for (uint32_t k = 0; k < 4u; k++) {
            const uint32_t i = 256u * wave + 4u * lane + k;
            if (i < n) {
                xr[k] = in[i];
                wr[k] = w[i];
            }
        }
    }
    for (uint32_t b = wave; b < blocks; b += 16u) {
        double ss = 0.0;
        for (uint32_t k = 0; k < 4u; k++) {
            const uint32_t i = 256u * b + 4u * lane + k;
            if (i < n) {
                const double v = b == wave ? xr[k] : in[i];
                ss = fma(v, v, ss);  // v*v is exact in double, so fusing changes nothing
            }
        }
        ss = wave_sum_d(ss);
        if (lane == 0) bpart[b] = ss;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (uint32_t k = 0; k < blocks; k++) t += bpart[k];
        float mean = (float)(t / (double)n);
        s_scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
    }
    __syncthreads();
    const float sc = s_scale;
    for (uint32_t b = wave; b < blocks; b += 16u) {
#pragma unroll
        for (uint32_t k = 0; k < 4u; k++) {
            const uint32_t i = 256u * b + 4u * lane + k;
            if (i < n) {
                const float x = b == wave ? xr[k] : in[i], wv = b == wave ? wr[k] : w[i];
                out[i] = __fmul_rn(__fmul_rn(x, sc), wv);
            }
        }
    }
}

hipError_t launch_rms_norm(const float *in, const float *w, float *out, uint32_t n, float eps,
                           hipStream_t s) {
    if (n == 0) return hipSuccess;
    const size_t blocks = (n + 255u) / 256u;
    if (blocks * sizeof(double) > 64u * 1024u) return hipErrorInvalidValue;
    k_rms_norm<<<1, 1024, blocks * sizeof(double), s>>>(in, w, out, n, eps);
    return hipGetLastError();
}

// ---- RoPE (src/vbs_host_math.h:38-51) --------------------------------------
// cos/sin of every pair angle come from the host's libm (the same powf, cosf
// and sinf the reference calls) and travel in the kernel arguments.
struct RopeTab {
    float c[256];
    float s[256];
};

__global__ __launch_bounds__(256) void k_rope(float *__restrict__ x, uint32_t hd, uint32_t nh,
                                              RopeTab tab) {
    uint32_t pairs = hd / 2u;
    uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= pairs * nh) return;
    uint32_t h = idx / pairs, p = idx % pairs;
    float *v = x + (uint64_t)h * hd + 2u * p;
    float x0 = v[0], x1 = v[1], c = tab.c[p], sn = tab.s[p];
    v[0] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, sn));
    v[1] = __fadd_rn(__fmul_rn(x0, sn), __fmul_rn(x1, c));
}

hipError_t launch_rope(float *x, uint32_t hd, uint32_t nh, const float *cs, hipStream_t s) {
    uint32_t pairs = hd / 2u;
    if (pairs == 0 || nh == 0) return hipSuccess;
    if (pairs > 256u) return hipErrorInvalidValue;
    RopeTab tab;
    for (uint32_t p = 0; p < pairs; p++) {
        tab.c[p] = cs[2 * p];
        tab.s[p] = cs[2 * p + 1];
    }
    uint32_t n = pairs * nh;
    k_rope<<<(n + 255u) / 256u, 256, 0, s>>>(x, hd, nh, tab);
    return hipGetLastError();
}

// ---- KV-cache store (src/vbs_host_math.h:150-159) ---------------------------
__global__ __launch_bounds__(256) void k_cache_store(const float *__restrict__ k,
                                                     const float *__restrict__ v,
                                                     uint16_t *__restrict__ kc,
                                                     uint16_t *__restrict__ vc, uint64_t base,
                                                     uint32_t kv_dim) {
    uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= kv_dim) return;
    kc[base + i] = vbs_f2h(k[i]);
    vc[base + i] = vbs_f2h(v[i]);
}

hipError_t launch_cache_store(const float *k, const float *v, uint16_t *kc, uint16_t *vc,
                              uint64_t base, uint32_t kv_dim, hipStream_t s) {
    if (kv_dim == 0) return hipSuccess;
    k_cache_store<<<(kv_dim + 255u) / 256u, 256, 0, s>>>(k, v, kc, vc, base, kv_dim);
    return hipGetLastError();
}

// ---- SiLU * up (src/vbs_host_math.h:53-57) and add (59-62) -----------------
__global__ __launch_bounds__(256) void k_silu_mul(const float *__restrict__ g,
                                                  const float *__restrict__ u,
                                                  float *__restrict__ out, uint32_t n) {
    uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    float gv = g[i];
    float den = __fadd_rn(1.0f, expf(-gv));
    out[i] = __fmul_rn(__fdiv_rn(gv, den), u[i]);
}

hipError_t launch_silu_mul(const float *g, const float *u, float *out, uint32_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    k_silu_mul<<<(n + 255u) / 256u, 256, 0, s>>>(g, u, out, n);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_add(const float *a, const float *b, float *out,
                                             uint32_t n) {
    uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    out[i] = __fadd_rn(a[i], b[i]);
}

hipError_t launch_add(const float *a, const float *b, float *out, uint32_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    k_add<<<(n + 255u) / 256u, 256, 0, s>>>(a, b, out, n);
    return hipGetLastError();
}

}  // namespace vbs
