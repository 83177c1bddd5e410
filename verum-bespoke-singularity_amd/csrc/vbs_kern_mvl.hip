// vbs_kern_mvl.hip — Q4_K matvec with the whole row range of a workgroup in
// flight at once (rows of 16 super-blocks, 4096-12288 rows).
//
// One 16-wave workgroup per CU owns an even range of at most 48 rows (T tiles
// of 16). Wave w owns super-block w of every row: before it computes anything
// it requests, by LDS DMA (global_load_lds_dwordx4), its x block and the
// block's 16 x 144 bytes of each of its T tiles, as contiguous 144-byte row
// runs. Nothing waits on anything else, so a CU has all of its ~110 KB of
// weights in flight from the start; the items are then computed in arrival
// order with the batch-1 kernel's arithmetic (Q4K::dot on the digits of x,
// vbs_mfma.h), and every row adds its blocks' partial sums in block order at
// the end, as k_mvf does: the results equal k_mvf's bit for bit. Measured
// against k_mvf (weights streamed from HBM): 11008 x 4096 7.8 against 8.4 us
// per launch, 12288 x 4096 8.0 against 8.7 us, 4096 x 4096 4.8 against 4.9 us.
//
// The DMA is issued by inline assembly (M0 = the wave-uniform LDS address):
// the compiler's builtin makes it insert waits for all loads before every
// LDS access. The compiler does not see these loads, so each wait for them is
// an explicit s_waitcnt; nothing else in this kernel uses M0.
#include "vbs_mfma.h"

namespace vbs {

constexpr uint32_t kMvlWaves = 16, kMvlItem = 16u * 144u, kMvlSlot = 1024u, kMvlMaxT = 3;

__device__ __forceinline__ void mvl_dma16(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}
template <uint32_t N>
__device__ __forceinline__ void mvl_vmcnt_le() {  // vmcnt <= N, other counters untouched
    static_assert(N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15u) | ((N >> 4) << 14) | (7u << 4) | (15u << 8));
}

// EPI: E_STORE (y = W x) or E_ACC (y += W x). T tiles of 16 rows per workgroup,
// rpw <= 16 T rows each (the last workgroup's range may be shorter or empty).
template <uint32_t T, int EPI>
__global__ __launch_bounds__(64 * kMvlWaves) void k_mvl(const MvArgs a, uint32_t rpw) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t cols = a.cols, nblk = cols >> 8, rb = nblk * 144u;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t r0 = blockIdx.x * rpw, r1 = min(r0 + rpw, a.rows[0]);
    if (r0 >= r1) return;
    const uint32_t b = min(wave, nblk - 1u);  // this wave's block (waves past the row re-read the last)
    const bool own = wave < nblk;
    // LDS: [16 waves][T items of 2304 B] | 16 zero bytes | [16 waves][x / digit slot] | pb
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    const uint32_t stage = lds0 + wave * T * kMvlItem;
    uint8_t *const xq = lds + kMvlWaves * T * kMvlItem;
    uint8_t *const slot = xq + 16u + wave * kMvlSlot;
    float *const pb = reinterpret_cast<float *>(xq + 16u + kMvlWaves * kMvlSlot);
    const uint8_t *const w = a.w[0];

    // 1. all loads: x block b (one DMA), then the T items (three DMAs each:
    // chunk c = 9 n' + p is piece p of row n' of the tile, at item + 16 c)
    mvl_dma16(a.x + 256u * b + 4u * lane, (uint32_t)(uintptr_t)slot);
#pragma unroll
    for (uint32_t j = 0; j < T; j++) {
#pragma unroll
        for (uint32_t q = 0; q < 3; q++) {
            const uint32_t c = 64u * q + lane;
            const uint32_t row = min(r0 + 16u * j + c / 9u, r1 - 1u);
            const uint8_t *src = w + ((uint64_t)row * rb + b * 144u + 16u * (c % 9u));
            if (q < 2u || lane < 16u) mvl_dma16(src, stage + j * kMvlItem + 1024u * q);
        }
    }
    if (lane < 4u) reinterpret_cast<uint32_t *>(xq)[lane] = 0u;
    DigitView dv;
    dv.zero = xq;
    dv.base = slot;
    dv.pstride = 256u;
    dv.xs16 = reinterpret_cast<float *>(slot + 768u);
    dv.xs = reinterpret_cast<float2 *>(slot + 832u);

    // 2. x has landed (the 3 T item DMAs after it may still be in flight):
    // its digits, written over it in the same slot
    mvl_vmcnt_le<3u * T>();
    asm volatile("" ::: "memory");
    {
        const float4 xv = *reinterpret_cast<const float4 *>(slot + 16u * lane);
        const float v[4] = {xv.x, xv.y, xv.z, xv.w};
        if (own) prep_block(v, lane, dv);
    }

    // 3. the items in arrival order
    auto item = [&](uint32_t j) {
        const uint8_t *row = lds + (stage - lds0) + j * kMvlItem + 144u * n;
        u32x4 r[3];
        r[0] = lda4(row);
        r[1] = lda4(row + 16u + 16u * g);
        r[2] = lda4(row + 80u + 16u * g);
        const Src src{w, a.rows[0] * rb, rb, r0 + 16u * j, r1};
        float part = Q4K::dot(r, nullptr, src, dv, b, n, g);
        part += __shfl_xor(part, 16, 64);
        part += __shfl_xor(part, 32, 64);
        const uint32_t rr = 16u * j + n;
        if (lane < 16u && own && rr < rpw) pb[rr * nblk + b] = part;
        asm volatile("" ::"v"(part));
        __builtin_amdgcn_sched_barrier(0);
    };
    mvl_vmcnt_le<3u * (T - 1u)>();
    asm volatile("" ::: "memory");
    item(0);
    if constexpr (T > 1u) {
        mvl_vmcnt_le<3u * (T - 2u)>();
        asm volatile("" ::: "memory");
        item(1);
    }
    if constexpr (T > 2u) {
        mvl_vmcnt_le<0u>();
        asm volatile("" ::: "memory");
        item(2);
    }

    // 4. row t of the range: its blocks' sums in block order
    __syncthreads();
    const uint32_t t = threadIdx.x;
    if (t < r1 - r0) {
        float s = 0.f;
        const float *p = pb + t * nblk;
        for (uint32_t k = 0; k < nblk; k++) s += p[k];
        float *y = a.y[0] + r0 + t;
        *y = EPI == E_ACC ? __fadd_rn(*y, s) : s;
    }
}

static uint32_t mvl_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
    }
    return (uint32_t)cus;
}

template <uint32_t T, int EPI>
static hipError_t launch_mvl_t(const MvArgs &a, uint32_t wgs, uint32_t rpw, hipStream_t s) {
    const uint32_t nblk = a.cols / 256u;
    const size_t lds = (size_t)kMvlWaves * T * kMvlItem + 16u + (size_t)kMvlWaves * kMvlSlot +
                       (size_t)rpw * nblk * sizeof(float);
    static bool granted = false;
    if (!granted) {
        if (hipFuncSetAttribute((const void *)k_mvl<T, EPI>,
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(kMvlWaves * kMvlMaxT * kMvlItem + 16u + kMvlWaves * kMvlSlot +
                                      16u * kMvlMaxT * 16u * sizeof(float))) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorNotSupported;
        }
        granted = true;
    }
    k_mvl<T, EPI><<<wgs, 64 * kMvlWaves, lds, s>>>(a, rpw);
    return hipGetLastError();
}

hipError_t launch_q4k_mvl(const uint8_t *w, const float *x, float *y, uint32_t cols, uint32_t rows,
                          int accumulate, hipStream_t s) {
    // rows of exactly 16 blocks (every wave busy) and 4096-12288 rows (one to
    // three tiles per workgroup): measured faster than k_mvf there, slower on
    // narrower rows, where waves sit idle
    const uint32_t nblk = cols / 256u;
    if (cols % 256u || nblk != kMvlWaves || rows < 4096u || ((uintptr_t)w & 15u) ||
        ((uintptr_t)x & 15u))
        return hipErrorNotSupported;
    const uint32_t wgs = mvl_cus();
    const uint32_t rpw = (rows + wgs - 1u) / wgs, tiles = (rpw + 15u) / 16u;
    if (tiles > kMvlMaxT) return hipErrorNotSupported;
    MvArgs a{};
    a.w[0] = w;
    a.y[0] = y;
    a.rows[0] = rows;
    a.nmat = 1;
    a.cols = cols;
    a.x = x;
    const uint32_t g = (rows + rpw - 1u) / rpw;  // workgroups with rows
#define VBS_MVL(TT)                                                                              \
    return accumulate ? launch_mvl_t<TT, E_ACC>(a, g, rpw, s) : launch_mvl_t<TT, E_STORE>(a, g, rpw, s)
    if (tiles == 1u) VBS_MVL(1);
    if (tiles == 2u) VBS_MVL(2);
    VBS_MVL(3);
#undef VBS_MVL
}

}  // namespace vbs
