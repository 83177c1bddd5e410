// vbs_kern_hot.hip — the CPU hot-kernel table's arithmetic (ABI v1,
// include/vbs_hotpath.h:38-57 of the reference) and the CPU model's Q8
// activation quantiser, on gfx950, bit-identical to the reference.
//
// The table's contract fixes the float order: one sum per row, added to block
// by block (element by element for F32/F16) in column order
// (src/hotkernels/vbs_hot_ref_impl.h:49-129). The kernels keep that order and
// parallelise only what is exact: a wave owns a row, its 64 lanes form the
// terms of 64 consecutive blocks at once (integer dots on v_dot4_i32_i8, each
// product rounded separately), and the running sum then takes the 64 terms in
// order through lane reads. Every product and sum is an explicitly rounded
// intrinsic, so nothing is fused.
#include "vbs_dev_common.h"
#include "vbs_internal.h"

namespace vbs {

enum : int { HK_Q8_0 = 0, HK_Q4_0 = 1, HK_Q4_1 = 2, HK_F32 = 3, HK_F16 = 4 };

// Four bytes at a 2-byte aligned address (every block field is 2-B aligned).
__device__ __forceinline__ int ld_w32(const uint8_t *p) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    return (int)((uint32_t)h[0] | ((uint32_t)h[1] << 16));
}

__device__ __forceinline__ float lane_f(float v, uint32_t k) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)k));
}

// y[row] for one row per wave, 4 rows per 256-thread workgroup.
template <int K>
__global__ __launch_bounds__(256) void k_hot_matvec(const uint8_t *__restrict__ w, uint32_t rows,
                                                    uint32_t cols, const void *__restrict__ act,
                                                    const float *__restrict__ qd,
                                                    const float *__restrict__ qsum,
                                                    float *__restrict__ y) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (row >= rows) return;  // whole wave
    constexpr bool kQuant = K == HK_Q8_0 || K == HK_Q4_0 || K == HK_Q4_1;
    constexpr uint32_t kBytes = K == HK_Q8_0 ? 34u : K == HK_Q4_0 ? 18u : 20u;
    const uint32_t units = kQuant ? cols / 32u : cols;
    float sum = 0.0f;
    for (uint32_t base = 0; base < units; base += 64u) {
        const uint32_t u = base + lane;
        float t0 = 0.0f, t1 = 0.0f;
        if (u < units) {
            if constexpr (kQuant) {
                const uint8_t *blk = w + ((uint64_t)row * units + u) * kBytes;
                const int *xw = reinterpret_cast<const int *>(static_cast<const int8_t *>(act) +
                                                              (uint64_t)u * 32u);
                int dot = 0;
                if constexpr (K == HK_Q8_0) {
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        dot = __builtin_amdgcn_sdot4(ld_w32(blk + 2 + 4 * j), xw[j], dot, false);
                } else {
                    // nibbles 0..15 are valid int8 lanes; Q4_0's "- 8" is
                    // applied as -8 * sum(xq), which is the same integer
                    constexpr uint32_t qo = K == HK_Q4_0 ? 2u : 4u;
                    int xs = 0;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int q = ld_w32(blk + qo + 4 * j);
                        dot = __builtin_amdgcn_sdot4(q & 0x0F0F0F0F, xw[j], dot, false);
                        dot = __builtin_amdgcn_sdot4((q >> 4) & 0x0F0F0F0F, xw[4 + j], dot, false);
                        if constexpr (K == HK_Q4_0) {
                            xs = __builtin_amdgcn_sdot4(0x01010101, xw[j], xs, false);
                            xs = __builtin_amdgcn_sdot4(0x01010101, xw[4 + j], xs, false);
                        }
                    }
                    if constexpr (K == HK_Q4_0) dot -= 8 * xs;
                }
                t0 = __fmul_rn(__fmul_rn(h2f(ld16(blk)), qd[u]), (float)dot);
                if constexpr (K == HK_Q4_1) t1 = __fmul_rn(h2f(ld16(blk + 2)), qsum[u]);
            } else {
                const float xv = static_cast<const float *>(act)[u];
                const uint64_t at = (uint64_t)row * cols + u;
                const float wv = K == HK_F32 ? reinterpret_cast<const float *>(w)[at]
                                             : h2f(reinterpret_cast<const uint16_t *>(w)[at]);
                t0 = __fmul_rn(wv, xv);
            }
        }
        const uint32_t n = min(64u, units - base);
        for (uint32_t k = 0; k < n; k++) {
            sum = __fadd_rn(sum, lane_f(t0, k));
            if constexpr (K == HK_Q4_1) sum = __fadd_rn(sum, lane_f(t1, k));
        }
    }
    if (lane == 0) y[row] = sum;
}

// One thread per 32-element block (src/vbs_cpu.c:166-182).
__global__ __launch_bounds__(256) void k_quantize_q8(const float *__restrict__ x, uint32_t nblk,
                                                     int8_t *__restrict__ xq,
                                                     float *__restrict__ qd,
                                                     float *__restrict__ qsum) {
    const uint32_t b = blockIdx.x * 256u + threadIdx.x;
    if (b >= nblk) return;
    const float *xb = x + (uint64_t)b * 32u;
    float v[32];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        v[i] = xb[i];
        amax = fabsf(v[i]) > amax ? fabsf(v[i]) : amax;
    }
    const float d = __fdiv_rn(amax, 127.0f);
    const float inv = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    int total = 0;
    uint32_t packed[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int q = (int)roundf(__fmul_rn(v[4 * j + i], inv));
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            total += q;
            word |= ((uint32_t)q & 255u) << (8 * i);
        }
        packed[j] = word;
    }
    uint32_t *out = reinterpret_cast<uint32_t *>(xq + (uint64_t)b * 32u);
#pragma unroll
    for (int j = 0; j < 8; j++) out[j] = packed[j];
    qd[b] = h2f(vbs_f2h_rne(d));
    qsum[b] = h2f(vbs_f2h_rne(__fmul_rn((float)total, d)));
}

}  // namespace vbs

using namespace vbs;

static bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

extern "C" {

int vbs_gfx950_quantize_q8(const float *x, uint32_t cols, int8_t *xq, float *qd, float *qsum) {
    if (!rt_ready()) return 0;
    if (cols % 32u) return rt_fail("quantize_q8: cols %u not a multiple of 32", cols);
    if (cols == 0) return 1;
    if (!x || !xq || !qd || !qsum) return rt_fail("quantize_q8: null pointer");
    if (!aligned(x, 4) || !aligned(xq, 4) || !aligned(qd, 4) || !aligned(qsum, 4))
        return rt_fail("quantize_q8: buffers must be 4-byte aligned");
    const uint32_t nblk = cols / 32u;
    hipLaunchKernelGGL(k_quantize_q8, dim3((nblk + 255u) / 256u), dim3(256), 0, rt_stream(), x,
                       nblk, xq, qd, qsum);
    return rt_hip_ok(hipGetLastError(), "quantize_q8");
}

int vbs_gfx950_hot_matvec(int type, const void *w, uint32_t rows, uint32_t cols, const void *act,
                          const float *qd, const float *qsum, float *y) {
    if (!rt_ready()) return 0;
    int kind;
    switch (type) {
        case kQ8_0: kind = HK_Q8_0; break;
        case kQ4_0: kind = HK_Q4_0; break;
        case kQ4_1: kind = HK_Q4_1; break;
        case kF32: kind = HK_F32; break;
        case kF16: kind = HK_F16; break;
        default: return rt_fail("hot_matvec: type %d is not in the hot-kernel table", type);
    }
    const bool quant = kind <= HK_Q4_1;
    if (quant && cols % 32u) return rt_fail("hot_matvec: cols %u not a multiple of 32", cols);
    if (rows == 0) return 1;
    if (rows > 0x7FFFFFFFu) return rt_fail("hot_matvec: too many rows (%u)", rows);
    if (!y || (cols && (!w || !act))) return rt_fail("hot_matvec: null pointer");
    if (quant && cols && (!qd || (kind == HK_Q4_1 && !qsum)))
        return rt_fail("hot_matvec: null activation scales");
    if (!aligned(w, kind == HK_F32 ? 4 : 2) || !aligned(act, 4) || !aligned(y, 4) ||
        !aligned(qd, 4) || !aligned(qsum, 4))
        return rt_fail("hot_matvec: misaligned buffer");
    const dim3 grid((rows + 3u) / 4u), block(256);
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    hipStream_t s = rt_stream();
    switch (kind) {
        case HK_Q8_0: hipLaunchKernelGGL(k_hot_matvec<HK_Q8_0>, grid, block, 0, s, wb, rows, cols, act, qd, qsum, y); break;
        case HK_Q4_0: hipLaunchKernelGGL(k_hot_matvec<HK_Q4_0>, grid, block, 0, s, wb, rows, cols, act, qd, qsum, y); break;
        case HK_Q4_1: hipLaunchKernelGGL(k_hot_matvec<HK_Q4_1>, grid, block, 0, s, wb, rows, cols, act, qd, qsum, y); break;
        case HK_F32: hipLaunchKernelGGL(k_hot_matvec<HK_F32>, grid, block, 0, s, wb, rows, cols, act, qd, qsum, y); break;
        default: hipLaunchKernelGGL(k_hot_matvec<HK_F16>, grid, block, 0, s, wb, rows, cols, act, qd, qsum, y); break;
    }
    return rt_hip_ok(hipGetLastError(), "hot_matvec");
}

}  // extern "C"
