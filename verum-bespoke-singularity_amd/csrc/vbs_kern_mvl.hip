// vbs_kern_mvl.hip — batch-1 K-quant matvecs that keep a CU's weights in
// flight through LDS DMA: k_mvl (Q4_K, the whole row range of a workgroup at
// once: rows of 16 super-blocks, 4096-12288 rows) and k_mvr (Q6_K, a ring of
// slots per wave: rows of 33-48 super-blocks, 2049-4096 rows).
//
// One 16-wave workgroup per CU owns an even range of at most 48 rows (T tiles
// of 16). Wave w owns super-block w of every row: before it computes anything
// it requests, by LDS DMA (global_load_lds_dwordx4), its x block and the
// block's 16 x 144 bytes of each of its T tiles, as contiguous 144-byte row
// runs. Nothing waits on anything else, so a CU has all of its ~110 KB of
// weights in flight from the start; the items are then computed in arrival
// order with the batch-1 kernel's arithmetic (Q4K::dot_x on the digits of x,
// vbs_mfma.h; the x operands of the wave's block are read from LDS once, not
// per tile), and every row adds its blocks' partial sums in block order at
// the end, as k_mvf does: the results equal k_mvf's bit for bit. Measured
// against k_mvf (weights streamed from HBM): 11008 x 4096 7.4 against 8.4 us
// per launch, 4096 x 4096 4.9 against 5.0 us. Of the 11008 x 4096 launch,
// the arithmetic alone (no weight loads) takes 4.1 us and the loads alone
// (no arithmetic) 5.9 us; the x operands read per tile cost 0.2 us more, and
// a row sum that waited for each partial in turn another 0.3 us.
//
// The DMA is issued by inline assembly (M0 = the wave-uniform LDS address):
// the compiler's builtin makes it insert waits for all loads before every
// LDS access. The compiler does not see these loads, so each wait for them is
// an explicit s_waitcnt; nothing else in these kernels uses M0.
#include "vbs_lds_dma.h"
#include "vbs_mfma.h"

namespace vbs {

constexpr uint32_t kMvlWaves = 16, kMvlItem = 16u * 144u, kMvlSlot = 1024u, kMvlMaxT = 3;

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
    dma16(a.x + 256u * b + 4u * lane, (uint32_t)(uintptr_t)slot);
#pragma unroll
    for (uint32_t j = 0; j < T; j++) {
#pragma unroll
        for (uint32_t q = 0; q < 3; q++) {
            const uint32_t c = 64u * q + lane;
            const uint32_t row = min(r0 + 16u * j + c / 9u, r1 - 1u);
            const uint8_t *src = w + ((uint64_t)row * rb + b * 144u + 16u * (c % 9u));
            if (q < 2u || lane < 16u) dma16(src, stage + j * kMvlItem + 1024u * q);
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
    vmcnt_le<3u * T>();
    asm volatile("" ::: "memory");
    {
        const float4 xv = *reinterpret_cast<const float4 *>(slot + 16u * lane);
        const float v[4] = {xv.x, xv.y, xv.z, xv.w};
        if (own) prep_block(v, lane, dv);
    }

    // 3. the items in arrival order, the x operands of block b read once
    const Q4K::X xo = Q4K::x_operands(dv, n, g);
    const uint32_t ps = part_stride(nblk);
    auto item = [&](uint32_t j) {
        const uint8_t *row = lds + (stage - lds0) + j * kMvlItem + 144u * n;
        u32x4 r[3];
        r[0] = lda4(row);
        r[1] = lda4(row + 16u + 16u * g);
        r[2] = lda4(row + 80u + 16u * g);
        float part = Q4K::dot_x(r, xo, g);
        part += __shfl_xor(part, 16, 64);
        part += __shfl_xor(part, 32, 64);
        const uint32_t rr = 16u * j + n;
        if (lane < 16u && own && rr < rpw) pb[rr * ps + b] = part;
        asm volatile("" ::"v"(part));
        __builtin_amdgcn_sched_barrier(0);
    };
    vmcnt_le<3u * (T - 1u)>();
    asm volatile("" ::: "memory");
    item(0);
    if constexpr (T > 1u) {
        vmcnt_le<3u * (T - 2u)>();
        asm volatile("" ::: "memory");
        item(1);
    }
    if constexpr (T > 2u) {
        vmcnt_le<0u>();
        asm volatile("" ::: "memory");
        item(2);
    }

    // 4. row t of the range: its blocks' sums in block order
    __syncthreads();
    const uint32_t t = threadIdx.x;
    if (t < r1 - r0) {
        const float s = ordered_sum(pb + t * ps, kMvlWaves);
        float *y = a.y[0] + r0 + t;
        *y = EPI == E_ACC ? __fadd_rn(*y, s) : s;
    }
}

template <uint32_t T, int EPI>
static hipError_t launch_mvl_t(const MvArgs &a, uint32_t wgs, uint32_t rpw, hipStream_t s) {
    const uint32_t nblk = a.cols / 256u;
    const size_t lds = (size_t)kMvlWaves * T * kMvlItem + 16u + (size_t)kMvlWaves * kMvlSlot +
                       (size_t)rpw * part_stride(nblk) * sizeof(float);
    static bool granted = false;
    if (!granted) {
        if (hipFuncSetAttribute((const void *)k_mvl<T, EPI>,
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(kMvlWaves * kMvlMaxT * kMvlItem + 16u + kMvlWaves * kMvlSlot +
                                      16u * kMvlMaxT * part_stride(kMvlWaves) * sizeof(float))) !=
            hipSuccess) {
            (void)hipGetLastError();
            return hipErrorNotSupported;
        }
        granted = true;
    }
    k_mvl<T, EPI><<<wgs, 64 * kMvlWaves, lds, s>>>(a, rpw);
    return hipGetLastError();
}

// ---- ring variant for Q6_K: more items per wave than the LDS holds at once ---------------
// k_mvr: a workgroup per CU owns an even range of at most 16 T rows; wave w
// owns blocks w, w + 16, ... (NB of them; slots past the row re-read its last
// block and add nothing). Its items -- T tiles of each of its blocks -- stream
// by LDS DMA through a ring of R slots: R items are requested before anything
// is computed and item i + R as soon as item i is done, so a CU keeps ~115 KB
// of weights in flight for the whole launch. An item is the tile's 16 rows of
// the block as 14 aligned 16-byte chunks each (224 bytes covering the 210 at
// any 2-byte offset), in the layout Q6K::dot_staged reads. x comes by DMA as
// well, a block ahead (two slots per wave); the digits of a block are written
// over its x. Arithmetic and per-(row, block) sums are k_mvf's, so the results
// equal k_mvf's bit for bit. Every wait is an explicit s_waitcnt on the number
// of DMAs issued after the awaited one (the loads return in issue order).
// A block's x operands are read once for its T items, and the row sums read
// the partials 16 at a time (padded with +0.0 to a multiple of 16).
// Measured with the weights streamed from HBM: 4096 x 11008 (7B down)
// 10.7 against k_mvf's 11.9-12.4 us, 8192 x 28672 (70B down) 38.7-38.8
// against 47.3-52.2 us (11.0-11.3 and 39.6-39.8 with the x operands read per
// item and a row sum that waited for each partial in turn).
constexpr uint32_t kMvrItem = 16u * 224u, kMvrDma = 4u;

template <uint32_t NB, uint32_t T, uint32_t R>
struct MvrPlan {
    static constexpr uint32_t NI = NB * T, D = kMvrDma;
    static constexpr uint32_t XS = NB > 1u ? 2u : 1u;  // x slots per wave
    static_assert(R >= 1u && R <= NI && (NB == 1u || R <= T + 1u), "ring");
    // DMAs that item i brings: its own, after x when it opens a block
    static constexpr uint32_t with(uint32_t i) { return D + (i % T == 0u ? 1u : 0u); }
    // DMAs issued after item i's last one at the time item i is computed
    // (items up to i + R - 1 are out)
    static constexpr uint32_t after_item(uint32_t i) {
        uint32_t c = 0;
        for (uint32_t j = i + 1u; j < i + R && j < NI; j++) c += with(j);
        return c;
    }
    // ... and after the x of the block item i opens
    static constexpr uint32_t after_x(uint32_t i) { return D + after_item(i); }
    static constexpr size_t lds(uint32_t nblk) {
        return 16u * (size_t)R * kMvrItem + 16u + 16u * (size_t)XS * 1024u +
               16u * (size_t)T * part_stride(nblk) * sizeof(float);
    }
};

template <uint32_t NB, uint32_t T, uint32_t R, int EPI>
__global__ __launch_bounds__(1024) void k_mvr(const MvArgs a, uint32_t rpw) {
    using P = MvrPlan<NB, T, R>;
    constexpr uint32_t NI = P::NI;
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t cols = a.cols, nblk = cols >> 8, rb = nblk * Q6K::BYTES;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t r0 = blockIdx.x * rpw, r1 = min(r0 + rpw, a.rows[0]);
    if (r0 >= r1) return;
    // LDS: [16 waves][R slots] | 16 zero bytes | [16 waves][XS x slots] |
    // pb [16 T rows][part_stride(nblk)] (the 16 NB >= part_slots(nblk) block slots)
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    const uint32_t ring = lds0 + wave * R * kMvrItem;
    uint8_t *const zero = lds + 16u * R * kMvrItem;
    uint8_t *const xs0 = zero + 16u + wave * P::XS * 1024u;
    float *const pb = reinterpret_cast<float *>(zero + 16u + 16u * P::XS * 1024u);
    // offsets are taken from w rounded down to 16 bytes (as in Q6K::load)
    const uint8_t *const w = a.w[0];
    const uint32_t wlo = (uint32_t)(uintptr_t)w & 15u;

    auto issue = [&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        constexpr uint32_t k = i / T, j = i % T;
        const uint32_t b = min(wave + 16u * k, nblk - 1u);
        if constexpr (j == 0u)
            dma16(a.x + 256u * b + 4u * lane, (uint32_t)(uintptr_t)(xs0 + (k % P::XS) * 1024u));
        const uint32_t dst = ring + (i % R) * kMvrItem;
#pragma unroll
        for (uint32_t q = 0; q < kMvrDma; q++) {
            const uint32_t c = min(64u * q + lane, 223u);  // chunk 14 n' + k' of the tile
            const uint32_t st = min(r0 + 16u * j + c / 14u, r1 - 1u) * rb + b * 210u;
            const uint32_t off = ((st + wlo) & ~15u) + 16u * (c % 14u);
            if (q < 3u || lane < 32u) dma16(w - wlo + off, dst + 1024u * q);
        }
    };
    unroll_for<0u, R>(issue);
    if (lane < 4u) reinterpret_cast<uint32_t *>(zero)[lane] = 0u;

    Q6K::X xo;  // block k's x operands, read once for its T items
    unroll_for<0u, NI>([&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        constexpr uint32_t k = i / T, j = i % T;
        const uint32_t bw = wave + 16u * k;
        const bool own = bw < nblk;
        const uint32_t b = min(bw, nblk - 1u);
        uint8_t *const slot = xs0 + (k % P::XS) * 1024u;
        DigitView dv;
        dv.zero = zero;
        dv.base = slot;
        dv.pstride = 256u;
        dv.xs16 = reinterpret_cast<float *>(slot + 768u);
        dv.xs = reinterpret_cast<float2 *>(slot + 832u);
        if constexpr (j == 0u) {  // x of block b has landed: its digits, over it
            vmcnt_le<P::after_x(i)>();
            asm volatile("" ::: "memory");
            const float4 xv = *reinterpret_cast<const float4 *>(slot + 16u * lane);
            const float v[4] = {xv.x, xv.y, xv.z, xv.w};
            if (own) prep_block(v, lane, dv);
            xo = Q6K::x_operands(dv, n, g);
        }
        vmcnt_le<P::after_item(i)>();
        asm volatile("" ::: "memory");
        if (own) {
            const Src src{w, a.rows[0] * rb, rb, r0 + 16u * j, r1};
            float part = Q6K::dot_staged_x(lds + (ring - lds0) + (i % R) * kMvrItem, src, xo, b, n, g);
            part += __shfl_xor(part, 16, 64);
            part += __shfl_xor(part, 32, 64);
            const uint32_t rr = 16u * j + n;
            if (lane < 16u && rr < rpw) pb[rr * part_stride(nblk) + b] = part;
            asm volatile("" ::"v"(part));
        } else {  // a slot past the row: +0.0 for the row sums
            const uint32_t rr = 16u * j + n;
            if (lane < 16u && rr < rpw) pb[rr * part_stride(nblk) + bw] = 0.f;
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (i + R < NI) issue(std::integral_constant<uint32_t, i + R>{});
    });

    // row t of the range: its blocks' sums in block order
    __syncthreads();
    const uint32_t t = threadIdx.x;
    if (t < r1 - r0) {
        const float s = ordered_sum(pb + t * part_stride(nblk), nblk);
        float *y = a.y[0] + r0 + t;
        *y = EPI == E_ACC ? __fadd_rn(*y, s) : s;
    }
}

template <uint32_t NB, uint32_t T, uint32_t R, int EPI>
static hipError_t launch_mvr_t(const MvArgs &a, uint32_t wgs, uint32_t rpw, hipStream_t s) {
    const size_t lds = MvrPlan<NB, T, R>::lds(a.cols / 256u);
    static size_t granted = 0;
    if (lds > granted) {
        if (hipFuncSetAttribute((const void *)k_mvr<NB, T, R, EPI>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorNotSupported;
        }
        granted = lds;
    }
    k_mvr<NB, T, R, EPI><<<wgs, 1024, lds, s>>>(a, rpw);
    return hipGetLastError();
}

// Q6_K rows of 33-48 blocks over 2049-4096 rows (7B down: 4096 x 11008): one
// tile per workgroup, three blocks per wave; rows of 97-112 blocks over
// 4097-8192 rows (70B down: 8192 x 28672): two tiles, seven blocks per wave.
// Two items in flight per wave.
hipError_t launch_q6k_mvr(const uint8_t *w, const float *x, float *y, uint32_t cols, uint32_t rows,
                          int accumulate, hipStream_t s) {
    const uint32_t nblk = cols / 256u;
    const bool narrow = nblk > 32u && nblk <= 48u, wide = nblk > 96u && nblk <= 112u;
    if (cols % 256u || !(narrow || wide) || ((uintptr_t)w & 1u) || ((uintptr_t)x & 15u))
        return hipErrorNotSupported;
    const uint32_t wgs = device_cus();
    const uint32_t rpw = (rows + wgs - 1u) / wgs;
    if (narrow ? rows <= 2048u || rpw > 16u : rows <= 4096u || rpw > 32u) return hipErrorNotSupported;
    // every row-sum slot, the padding included, belongs to a wave's block slot
    if (16u * (wide ? 7u : 3u) < part_slots(nblk)) return hipErrorNotSupported;
    // the last row's last block read as aligned chunks must end inside the
    // matrix (the DMA has no bounded form); offsets are 32-bit
    const uint64_t rb = (uint64_t)nblk * 210u, bytes = rb * rows, wlo = (uintptr_t)w & 15u;
    const uint64_t last = bytes - 210u;
    if (((last + wlo) & ~(uint64_t)15u) + 224u > bytes + wlo || bytes + 256u >= (1ull << 32))
        return hipErrorNotSupported;
    MvArgs a{};
    a.w[0] = w;
    a.y[0] = y;
    a.rows[0] = rows;
    a.nmat = 1;
    a.cols = cols;
    a.x = x;
    const uint32_t g = (rows + rpw - 1u) / rpw;
    if (wide)
        return accumulate ? launch_mvr_t<7, 2, 2, E_ACC>(a, g, rpw, s)
                          : launch_mvr_t<7, 2, 2, E_STORE>(a, g, rpw, s);
    return accumulate ? launch_mvr_t<3, 1, 2, E_ACC>(a, g, rpw, s)
                      : launch_mvr_t<3, 1, 2, E_STORE>(a, g, rpw, s);
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
    const uint32_t wgs = device_cus();
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
