// vbs_kern_mvl.hip — batch-1 K-quant matvecs that keep a CU's weights in
// flight through LDS DMA: k_mvl (Q4_K, the whole row range of a workgroup at
// once: rows of 16 super-blocks, 4096-12288 rows; also the decoder's fused
// attn_norm + Q/K/V + RoPE + KV store launch over such rows) and k_mvr (Q6_K,
// a ring of slots per wave: rows of 33-48 super-blocks, 2049-4096 rows).
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
#include "vbs_attn_common.h"
#include "vbs_lds_dma.h"
#include "vbs_mfma.h"

namespace vbs {

constexpr uint32_t kMvlWaves = 16, kMvlItem = 16u * 144u, kMvlSlot = 1024u, kMvlMaxT = 3;
constexpr uint32_t kMvlQkvBytes = 16u + 1024u;  // E_QKV: position, RoPE row of hd <= 256

// EPI: E_STORE (y = W x), E_ACC (y += W x) or E_QKV (the nmat matrices' rows
// one after another, RoPE and the f16 cache stores of k_mvf's E_QKV). NORM:
// x is RMS-normalised first, as in k_mvf (each wave's block sum of squares,
// the sixteen added in block order). T tiles of 16 rows per workgroup,
// rpw <= 16 T rows each (the last workgroup's range may be shorter or empty).
template <uint32_t T, bool NORM, int EPI>
__global__ __launch_bounds__(64 * kMvlWaves) void k_mvl(const MvArgs a, uint32_t rpw) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ double bsum[NORM ? kMvlWaves : 1];
    const uint32_t cols = a.cols, nblk = cols >> 8, rb = nblk * 144u;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u, g = lane >> 4;
    // the launch's rows: matrix 0's, then matrix 1's, then matrix 2's
    const uint32_t e0 = a.rows[0], e1 = EPI == E_QKV && a.nmat > 1u ? e0 + a.rows[1] : e0;
    const uint32_t total = EPI == E_QKV && a.nmat > 2u ? e1 + a.rows[2] : e1;
    const uint32_t r0 = blockIdx.x * rpw, r1 = min(r0 + rpw, total);
    if (r0 >= r1) return;
    const uint32_t b = min(wave, nblk - 1u);  // this wave's block (waves past the row re-read the last)
    const bool own = wave < nblk;
    // LDS: [16 waves][T items of 2304 B] | 16 zero bytes | [16 waves][x / digit slot] |
    // (NORM) [16 waves][RMSNorm weights of the block] | (E_QKV) the position
    // (16 B) and its RoPE row (hd / 2 float2) | pb
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    const uint32_t stage = lds0 + wave * T * kMvlItem;
    uint8_t *const xq = lds + kMvlWaves * T * kMvlItem;
    uint8_t *const slot = xq + 16u + wave * kMvlSlot;
    uint8_t *const nslot = xq + 16u + kMvlWaves * kMvlSlot + wave * 1024u;
    uint8_t *const qpos = xq + 16u + kMvlWaves * kMvlSlot + (NORM ? kMvlWaves * 1024u : 0u);
    uint8_t *const qrope = qpos + 16u;
    float *const pb = reinterpret_cast<float *>(qpos + (EPI == E_QKV ? kMvlQkvBytes : 0u));
    // E_QKV: wave 0 (the one that finishes the rows) requests the position
    // before anything else and its RoPE row once the position is in: the
    // epilogue's operands arrive during the matrix work, not after it
    const bool w0 = EPI == E_QKV && __builtin_amdgcn_readfirstlane(wave) == 0u;
    // matrix m of row gr (E_QKV) and gr's first byte
    auto mat = [&](uint32_t gr) { return (uint32_t)(gr >= e0) + (uint32_t)(gr >= e1); };
    auto wrow = [&](uint32_t gr) {
        if constexpr (EPI == E_QKV) {
            const uint32_t m = mat(gr);
            const uint8_t *w = m == 0u ? a.w[0] : m == 1u ? a.w[1] : a.w[2];
            return w + (uint64_t)(gr - (m == 0u ? 0u : m == 1u ? e0 : e1)) * rb;
        } else {
            return a.w[0] + (uint64_t)gr * rb;
        }
    };

    // 1. all loads: x block b (one DMA) and its RMSNorm weights, then the T
    // items (three DMAs each: chunk c = 9 n' + p is piece p of row n' of the
    // tile, at item + 16 c)
    if (w0 && lane == 0u) dma4(a.pos, (uint32_t)(uintptr_t)qpos);
    dma16(a.x + 256u * b + 4u * lane, (uint32_t)(uintptr_t)slot);
    if constexpr (NORM) dma16(a.norm_w + 256u * b + 4u * lane, (uint32_t)(uintptr_t)nslot);
    // the lane's chunk c = 9 n' + p of each of a tile's three DMAs: row n' of
    // the tile, piece p of its 144 bytes
    uint32_t lrow[3], lchk[3];
#pragma unroll
    for (uint32_t q = 0; q < 3u; q++) {
        lrow[q] = (64u * q + lane) / 9u;
        lchk[q] = 16u * ((64u * q + lane) % 9u);
    }
    auto issue_tile = [&](uint32_t j) {
        // a tile inside one matrix (all but those across a Q/K or K/V border)
        // takes 32-bit offsets from that matrix's base in scalar registers
        const uint32_t t0 = r0 + 16u * j, tl = min(t0 + 15u, r1 - 1u);
        const uint32_t m = EPI == E_QKV ? mat(t0) : 0u;
        const bool one = EPI != E_QKV || m == mat(tl);
        const uint32_t start = m == 0u ? 0u : m == 1u ? e0 : e1;
        const uint8_t *const wm = m == 0u ? a.w[0] : m == 1u ? a.w[1] : a.w[2];
#pragma unroll
        for (uint32_t q = 0; q < 3; q++) {
            const uint32_t row = min(t0 + lrow[q], r1 - 1u);
            const uint32_t dst = stage + j * kMvlItem + 1024u * q;
            if (q < 2u || lane < 16u) {
                if (one)
                    dma16s(wm, (row - start) * rb + b * 144u + lchk[q], dst);
                else
                    dma16(wrow(row) + (b * 144u + lchk[q]), dst);
            }
        }
    };
    // With the RMSNorm, tiles from kPre on are requested after the barrier
    // that shares the block sums: a barrier waits until every wave has issued
    // everything before it, and issuing all of a CU's DMAs takes ~0.8 us.
    constexpr uint32_t kPre = NORM ? 1u : T;
#pragma unroll
    for (uint32_t j = 0; j < kPre; j++) issue_tile(j);
    if (lane < 4u) reinterpret_cast<uint32_t *>(xq)[lane] = 0u;
    DigitView dv;
    dv.zero = xq;
    dv.base = slot;
    dv.pstride = 256u;
    dv.xs16 = reinterpret_cast<float *>(slot + 768u);
    dv.xs = reinterpret_cast<float2 *>(slot + 832u);

    // 2. x has landed (the item DMAs after it may still be in flight): its
    // digits, written over it in the same slot
    vmcnt_le<3u * kPre>();
    asm volatile("" ::: "memory");
    {
        const float4 xv = *reinterpret_cast<const float4 *>(slot + 16u * lane);
        float v[4] = {xv.x, xv.y, xv.z, xv.w};
        if constexpr (NORM) {
            const double ss = block_sumsq(v);
            if (lane == 0u && own) bsum[wave] = ss;
            __syncthreads();
#pragma unroll
            for (uint32_t j = kPre; j < T; j++) issue_tile(j);
            double t = 0.0;
            for (uint32_t k = 0; k < nblk; k++) t += bsum[k];
            const float mean = (float)(t / (double)cols);
            const float sc = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, a.eps)));
            const float4 wv = *reinterpret_cast<const float4 *>(nslot + 16u * lane);
            const float w4[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int k = 0; k < 4; k++) v[k] = __fmul_rn(__fmul_rn(v[k], sc), w4[k]);
            if (a.xn && blockIdx.x == 0 && own)
                *reinterpret_cast<float4 *>(a.xn + 256u * b + 4u * lane) = make_float4(v[0], v[1], v[2], v[3]);
        }
        if (own) prep_block(v, lane, dv);
    }
    if (w0) {  // (the position landed before x)
        const uint32_t p = *reinterpret_cast<const uint32_t *>(qpos);
        if (lane < a.hd / 4u)
            dma16(a.rope + (uint64_t)p * (a.hd / 2u) + 2u * lane, (uint32_t)(uintptr_t)qrope);
    }
    // the wait for the items issued before the last N (wave 0 of E_QKV has
    // the RoPE DMA after them)
    auto wait_items = [&](auto N) {
        if (w0)
            vmcnt_le<decltype(N)::value + 1u>();
        else
            vmcnt_le<decltype(N)::value>();
        asm volatile("" ::: "memory");
    };

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
        part += lane_xor<16>(part);
        part += lane_xor<32>(part);
        const uint32_t rr = 16u * j + n;
        if (lane < 16u && own && rr < rpw) pb[rr * ps + b] = part;
        asm volatile("" ::"v"(part));
        __builtin_amdgcn_sched_barrier(0);
    };
    wait_items(std::integral_constant<uint32_t, 3u * (T - 1u)>{});
    item(0);
    if constexpr (T > 1u) {
        wait_items(std::integral_constant<uint32_t, 3u * (T - 2u)>{});
        item(1);
    }
    if constexpr (T > 2u) {
        wait_items(std::integral_constant<uint32_t, 0u>{});
        item(2);
    }

    // 4. row t of the range: its blocks' sums in block order
    __syncthreads();
    const uint32_t t = threadIdx.x;
    if constexpr (EPI == E_QKV) {
        // (ranges start and end on even rows: a row's RoPE partner t ^ 1 is in
        // the range and in the same wave)
        // (rows live in wave 0: rpw <= 48)
        if (w0) {
            vmcnt_le<0u>();
            asm volatile("" ::: "memory");
        }
        float s = 0.f;
        if (t < r1 - r0) s = ordered_sum(pb + t * ps, kMvlWaves);
        const float other = __shfl_xor(s, 1, 64);
        if (t < r1 - r0) {
            const uint32_t gr = r0 + t, m = mat(gr);
            const float2 *rp = reinterpret_cast<const float2 *>(qrope);
            qkv_store(a, m, gr - (m == 0u ? 0u : m == 1u ? e0 : e1), s, other,
                      *reinterpret_cast<const uint32_t *>(qpos), [&](uint32_t i) { return rp[i]; });
        }
    } else if (t < r1 - r0) {
        const float s = ordered_sum(pb + t * ps, kMvlWaves);
        float *y = a.y[0] + r0 + t;
        *y = EPI == E_ACC ? __fadd_rn(*y, s) : s;
        if (EPI == E_ACC && a.ycopy) a.ycopy[r0 + t] = s;
        if (EPI == E_STORE) store_joins(a, r0 + t, s);
    }
}

template <uint32_t T, bool NORM, int EPI>
static hipError_t launch_mvl_t(const MvArgs &a, uint32_t wgs, uint32_t rpw, hipStream_t s) {
    const uint32_t nblk = a.cols / 256u;
    const size_t fixed = (size_t)kMvlWaves * T * kMvlItem + 16u + (size_t)kMvlWaves * kMvlSlot +
                         (NORM ? (size_t)kMvlWaves * 1024u : 0u) + (EPI == E_QKV ? kMvlQkvBytes : 0u);
    const size_t lds = fixed + (size_t)rpw * part_stride(nblk) * sizeof(float);
    static bool granted = false;
    if (!granted) {
        if (hipFuncSetAttribute((const void *)k_mvl<T, NORM, EPI>,
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(fixed + 16u * T * part_stride(kMvlWaves) * sizeof(float))) !=
            hipSuccess) {
            (void)hipGetLastError();
            return hipErrorNotSupported;
        }
        granted = true;
    }
    k_mvl<T, NORM, EPI><<<wgs, 64 * kMvlWaves, lds, s>>>(a, rpw);
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
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t r0 = blockIdx.x * rpw, r1 = min(r0 + rpw, a.rows[0]);
    if (r0 >= r1) return;
    // the lane's chunk of each of an item's DMAs: chunk c = 14 n' + k' of the
    // tile, row n' of the tile and byte 16 k' of the row's run
    uint32_t lrow[kMvrDma], lchk[kMvrDma];
#pragma unroll
    for (uint32_t q = 0; q < kMvrDma; q++) {
        const uint32_t c = min(64u * q + lane, 223u);
        lrow[q] = c / 14u;
        lchk[q] = 16u * (c % 14u);
    }
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
            const uint32_t st = min(r0 + 16u * j + lrow[q], r1 - 1u) * rb + b * 210u;
            const uint32_t off = ((st + wlo) & ~15u) + lchk[q];
            if (q < 3u || lane < 32u) dma16s(w - wlo, off, dst + 1024u * q);
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
            part += lane_xor<16>(part);
            part += lane_xor<32>(part);
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
        if (EPI == E_ACC && a.ycopy) a.ycopy[r0 + t] = s;
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
                          int accumulate, hipStream_t s, float *ycopy) {
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
    a.ycopy = ycopy;
    const uint32_t g = (rows + rpw - 1u) / rpw;
    if (wide)
        return accumulate ? launch_mvr_t<7, 2, 2, E_ACC>(a, g, rpw, s)
                          : launch_mvr_t<7, 2, 2, E_STORE>(a, g, rpw, s);
    return accumulate ? launch_mvr_t<3, 1, 2, E_ACC>(a, g, rpw, s)
                      : launch_mvr_t<3, 1, 2, E_STORE>(a, g, rpw, s);
}

hipError_t launch_q4k_mvl(const uint8_t *w, const float *x, float *y, uint32_t cols, uint32_t rows,
                          int accumulate, hipStream_t s, const MvArgs *extra) {
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
    const bool norm = extra && extra->norm_w;
    if (extra) {  // the backend shim's fused neighbours: RMSNorm in front, or the copy of t
        if (norm && (accumulate || ((uintptr_t)extra->norm_w & 15u))) return hipErrorNotSupported;
        a.norm_w = extra->norm_w;
        a.eps = extra->eps;
        a.xn = extra->xn;
        a.ycopy = extra->ycopy;
        a.gate_in = extra->gate_in;
        a.hid = extra->hid;
        a.kin = extra->kin;
        a.kc = extra->kc;
        a.vc = extra->vc;
        a.kv_layer = extra->kv_layer;
        if ((a.hid || a.kin) && accumulate) return hipErrorNotSupported;
    }
    const uint32_t g = (rows + rpw - 1u) / rpw;  // workgroups with rows
#define VBS_MVL(TT)                                                                              \
    return norm         ? launch_mvl_t<TT, true, E_STORE>(a, g, rpw, s)                          \
           : accumulate ? launch_mvl_t<TT, false, E_ACC>(a, g, rpw, s)                           \
                        : launch_mvl_t<TT, false, E_STORE>(a, g, rpw, s)
    if (tiles == 1u) VBS_MVL(1);
    if (tiles == 2u) VBS_MVL(2);
    VBS_MVL(3);
#undef VBS_MVL
}

// ---- the attention merge inside the O launch -----------------------------------------
// k_mvl_attn: y += W attn for a decode step's O projection (Q4_K rows of 16
// blocks, one tile per workgroup), where attn -- the merge of the chunk
// launch's partials, head_dim 128, nqh = cols / 128 heads -- is made inside
// the launch instead of by a merge launch of its own. Workgroups are dealt to
// the eight XCDs round-robin in flat-index order, so with 8 nqh of them each
// XCD holds the 8 j + r for one r and every j < nqh: workgroup i merges q head
// i / 8 (waves 0..3, as k_attn_merge_h128: bit-identical), publishes it to its
// XCD's copy of the vector (its XCC_ID register) and raises the head's flag
// there, a 128-byte line of its own; then its wave 0 waits for all the
// heads' flags, read in the XCD's L2 by atomic adds of zero, copies the vector
// into the x slots, and the launch goes on as k_mvl's E_ACC form. The merge is
// the critical path, so its loads go out first (they cover the head's whole
// chunk stride, so they need not wait for the position) and the weights'
// DMAs after a barrier; waves 4..7 request blocks 0..3's weights together with
// their own, so waves 0..3 have no DMA in flight and wait on their own loads
// with the compiler's counts; everything else waits on explicit counts.
// Nothing in the launch reads a head's lines before its flag is up, so no
// CU's L1 holds a stale copy; no device-scope release or acquire is needed.
// The wait is bounded (spin polls): past it, wave 0 merges every head itself
// (merge_one_wave, bit-identical too), so a workgroup that ran on an
// unexpected XCD or late costs time, never the result. The chunk launch
// before it clears the flags.
// Measured (7B, ctx ~2065, eager under the tracer): 9.0 us against 4.9 +
// 4.4 us for k_mvl and the merge launch; 7B graph decode 691-695 against
// 676-692 tok/s. Forms measured slower: one flag line per XCD polled by four
// waves of every workgroup (the atomics on one line queue in the L2: 14.5
// us), and the position read by a scalar load with glc (35 us).
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 15u;
}
// The word at p as the XCD's L2 holds it: an atomic add of zero (atomics are
// performed in the L2; a plain load may be served by a line the CU's L1 took
// at an earlier poll). The zero is hidden from the compiler so that the add
// is not turned into a load.
__device__ __forceinline__ uint32_t load_l2(uint32_t *p) {
    uint32_t z = 0u;
    asm volatile("" : "+v"(z));
    return __hip_atomic_fetch_add(p, z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Every wave's LDS writes done, then the workgroup barrier (no wait on
// vector memory: the DMAs in flight stay in flight).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt and expcnt untouched
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__global__ __launch_bounds__(64 * kMvlWaves) void k_mvl_attn(const AttnOArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float2 red[kMergeRes][64];
    const uint32_t cols = a.cols, rb = kMvlWaves * 144u, nqh = cols / 128u;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t r0 = blockIdx.x * a.rpw, r1 = min(r0 + a.rpw, a.rows);
    const bool rows_here = r0 < r1;  // (a workgroup without rows still merges its head)
    const uint32_t xcc = xcc_id(), hh = blockIdx.x >> 3;
    const bool xok = xcc < kAttnOXcds;
    // LDS: [16 waves][item of 2304 B] | 16 zero bytes | [16 waves][x / digit slot] | pb
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    uint8_t *const xq = lds + kMvlWaves * kMvlItem;
    uint8_t *const slot0 = xq + 16u;
    float *const pb = reinterpret_cast<float *>(xq + 16u + kMvlWaves * kMvlSlot);
    const uint32_t ps = part_stride(kMvlWaves);

    // 1. waves 0..3: the partials of q head hh requested (residue `wave`
    // each) before any weight: the merge is the launch's critical path. The
    // loads cover the head's stride_chunks rows, so they need not wait for
    // the position; the rows from the chunk count on are dropped after.
    const float *ph = a.part + (uint64_t)hh * a.stride_chunks * kPartRow;
    float2 av[kMergeBatch];
    MergeMl ml{};
    if (wave < kMergeRes) {
        merge_residue_load(ph, a.stride_chunks, wave, lane, av);
        ml = merge_ml_load_bounded(ph, a.stride_chunks, lane);
    }
    if (lane < 4u) reinterpret_cast<uint32_t *>(xq)[lane] = 0u;
    lds_barrier();
    // 2. the items: block w's 16 x 144 bytes for wave w (waves 4..7 first
    // request those of blocks 0..3)
    auto issue_item = [&](uint32_t blk) {
#pragma unroll
        for (uint32_t q = 0; q < 3; q++) {
            const uint32_t c = 64u * q + lane;
            const uint32_t row = min(r0 + c / 9u, r1 - 1u);
            const uint8_t *src = a.w + ((uint64_t)row * rb + blk * 144u + 16u * (c % 9u));
            if (q < 2u || lane < 16u) dma16(src, lds0 + blk * kMvlItem + 1024u * q);
        }
    };
    if (rows_here) {
        if (wave >= 4u && wave < 8u) issue_item(wave - 4u);
        if (wave >= 4u) issue_item(wave);
    }

    // the position (only waves 0..3 read it: a compiler-counted load in a
    // wave with DMAs in flight would wait for all of them)
    uint32_t nc = 0;
    if (wave < kMergeRes) {
        nc = mfma_chunks(a.pos[0] + 1u, a.nkh);  // seq = pos + 1
        ml = merge_ml_mask(ml, nc, lane);
    }

    // 3. waves 0..3: the merge of head hh, as k_attn_merge_h128
    MergeStats st{};
    if (wave < kMergeRes) {
        st = merge_stats(ph, nc, lane, ml);
        red[wave][lane] = merge_residue_sum(ph, nc, st, wave, lane, av);
    }
    lds_barrier();

    // 4. wave 0 publishes the head to its XCD's copy, raises its flag (a line
    // of its own) once the stores are in the L2, then waits for the other
    // heads' flags -- one poller per workgroup -- and copies the whole vector
    // into the x slots
    if (wave == 0u) {
        float2 ar[kMergeRes];
#pragma unroll
        for (uint32_t r = 0; r < kMergeRes; r++) ar[r] = red[r][lane];
        const float2 o = merge_finish(ar, st.L);
        if (xok) *reinterpret_cast<float2 *>(a.mbuf + (uint64_t)xcc * cols + hh * 128u + 2u * lane) = o;
        if (a.attn) *reinterpret_cast<float2 *>(a.attn + hh * 128u + 2u * lane) = o;
        vmcnt_le<0u>();
        asm volatile("" ::: "memory");
        uint32_t *const fl = a.mflag + (uint64_t)xcc * nqh * kAttnOFlagStride;
        if (xok && lane == 0u) fl[hh * kAttnOFlagStride] = 1u;
        bool ready = false;
        if (xok) {
            for (uint32_t it = 0; it < a.spin; it++) {
                const uint32_t f = lane < nqh ? load_l2(fl + lane * kAttnOFlagStride) : 1u;
                if (__all(f != 0u)) {
                    ready = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        asm volatile("" ::: "memory");  // (the reads below stay behind the polls)
        if (ready) {
            const float *src = a.mbuf + (uint64_t)xcc * cols;
            float4 v[kMvlWaves];
#pragma unroll
            for (uint32_t i = 0; i < kMvlWaves; i++)
                v[i] = *reinterpret_cast<const float4 *>(src + 256u * i + 4u * lane);
#pragma unroll
            for (uint32_t i = 0; i < kMvlWaves; i++)
                *reinterpret_cast<float4 *>(slot0 + i * kMvlSlot + 16u * lane) = v[i];
        } else {  // the bounded wait ran out: every head merged here
            if (lane == 0u && a.fallbacks) atomicAdd(a.fallbacks, 1u);
            for (uint32_t h = 0; h < nqh; h++) {
                const float2 oh = merge_one_wave<4u>(a.part + (uint64_t)h * a.stride_chunks * kPartRow, nc, lane);
                *reinterpret_cast<float2 *>(slot0 + (h >> 1) * kMvlSlot + 512u * (h & 1u) + 8u * lane) = oh;
            }
        }
    }
    // waves 4..7: blocks 0..3's items have landed (their own may be in flight)
    if (rows_here && wave >= 4u && wave < 8u) vmcnt_le<3u>();
    lds_barrier();
    if (!rows_here) return;

    // 5. as k_mvl: the digits of x block `wave` over it, the wave's item, the
    // row sums in block order and the residual add
    uint8_t *const slot = slot0 + wave * kMvlSlot;
    DigitView dv;
    dv.zero = xq;
    dv.base = slot;
    dv.pstride = 256u;
    dv.xs16 = reinterpret_cast<float *>(slot + 768u);
    dv.xs = reinterpret_cast<float2 *>(slot + 832u);
    {
        const float4 xv = *reinterpret_cast<const float4 *>(slot + 16u * lane);
        const float v[4] = {xv.x, xv.y, xv.z, xv.w};
        prep_block(v, lane, dv);
    }
    const Q4K::X xo = Q4K::x_operands(dv, n, g);
    if (wave >= 4u) {
        vmcnt_le<0u>();
        asm volatile("" ::: "memory");
    }
    {
        const uint8_t *row = lds + wave * kMvlItem + 144u * n;
        u32x4 r[3];
        r[0] = lda4(row);
        r[1] = lda4(row + 16u + 16u * g);
        r[2] = lda4(row + 80u + 16u * g);
        float part = Q4K::dot_x(r, xo, g);
        part += lane_xor<16>(part);
        part += lane_xor<32>(part);
        if (lane < 16u && n < a.rpw) pb[n * ps + wave] = part;
    }
    __syncthreads();
    const uint32_t t = threadIdx.x;
    if (t < r1 - r0) {
        const float s = ordered_sum(pb + t * ps, kMvlWaves);
        float *y = a.y + r0 + t;
        *y = __fadd_rn(*y, s);
    }
}

size_t attn_o_exchange_bytes(uint32_t cols) {
    return (size_t)kAttnOXcds * cols * sizeof(float) + attn_o_flag_words(cols) * sizeof(uint32_t);
}

hipError_t launch_q4k_mvl_attn(const AttnOArgs &a, hipStream_t s) {
    const uint32_t nqh = a.cols / 128u, wgs = 8u * nqh;
    if (a.cols != 256u * kMvlWaves || a.rows == 0 || !a.part || !a.pos || !a.mbuf || !a.mflag ||
        ((uintptr_t)a.w & 15u) || ((uintptr_t)a.mbuf & 15u) || a.rpw == 0 || a.rpw > 16u ||
        (uint64_t)a.rpw * wgs < a.rows)
        return hipErrorNotSupported;
    const size_t lds = (size_t)kMvlWaves * kMvlItem + 16u + (size_t)kMvlWaves * kMvlSlot +
                       (size_t)a.rpw * part_stride(kMvlWaves) * sizeof(float);
    k_mvl_attn<<<wgs, 64 * kMvlWaves, lds, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_q4k_mvl_qkv(const MvArgs &a, hipStream_t s) {
    // the fused attn_norm + Q/K/V + RoPE + KV store launch over rows of exactly
    // 16 blocks and 4096 or more rows in all: every CU takes an even range
    // (k_mvf's two tiles per workgroup leave a quarter of the CUs idle at
    // 6144 rows)
    const uint32_t nblk = a.cols / 256u;
    if (a.cols % 256u || nblk != kMvlWaves || a.nmat == 0u || a.nmat > 3u || ((uintptr_t)a.x & 15u) ||
        ((uintptr_t)a.norm_w & 15u) || ((uintptr_t)a.rope & 15u) || ((uintptr_t)a.pos & 3u) ||
        a.hd % 4u || a.hd > 256u)
        return hipErrorNotSupported;
    uint32_t total = 0;
    for (uint32_t m = 0; m < a.nmat; m++) {
        if (((uintptr_t)a.w[m] & 15u) || (a.rows[m] & 1u)) return hipErrorNotSupported;
        total += a.rows[m];
    }
    if (total < 4096u) return hipErrorNotSupported;
    const uint32_t wgs = device_cus();
    const uint32_t rpw = ((total + wgs - 1u) / wgs + 1u) & ~1u, tiles = (rpw + 15u) / 16u;
    if (tiles > kMvlMaxT) return hipErrorNotSupported;
    const uint32_t g = (total + rpw - 1u) / rpw;
#define VBS_MVL(TT)                                                                              \
    return a.norm_w ? launch_mvl_t<TT, true, E_QKV>(a, g, rpw, s)                                \
                    : launch_mvl_t<TT, false, E_QKV>(a, g, rpw, s)
    if (tiles == 1u) VBS_MVL(1);
    if (tiles == 2u) VBS_MVL(2);
    VBS_MVL(3);
#undef VBS_MVL
}

}  // namespace vbs
