// vbs_kern_checksum.hip — XOR checksum of a device region (vbs_gfx950_checksum).
//
// Two uses: verifying that an upload arrived intact (the host XORs the same
// words), and the read floor beside the matvec roofline: it reads every byte
// once and does nothing else, in the shape of the fastest whole-chip read this
// part showed — spans of at most 112 KB per workgroup (the region split
// evenly over 256 of them while that suffices, so each CU streams one
// contiguous span), fetched in 1 KB runs (64 lanes x 16 bytes) straight into
// LDS (global_load_lds_dwordx4, streaming cache policy), every run of the
// span in flight at once.
//
// Workgroup w (16 waves) owns span [w S, (w + 1) S) of the region (S a
// multiple of 1 KB, at most 112 KB); run 16 u + v of the span goes to wave v's
// LDS slot u (u < 7), so each step of the waves' loads covers 16 adjacent
// runs. (Variants of the shape, timed as alternative floors: two 8-wave
// workgroups per CU, and 16-byte register loads instead of the DMA.) Each wave XORs the words of its chunks of a run as soon as that run
// has landed, folds its lanes with DPP and lane reads, and stores one partial
// word, partials[16 w + v]: no barrier and no serial tail after the last
// bytes arrive.
#include "vbs_dev_common.h"
#include "vbs_internal.h"

#include <type_traits>

namespace vbs {

constexpr uint32_t kCsWaves = 16, kCsRuns = 7;                  // runs per wave
constexpr uint32_t kCsWgs = 256;

// 16 bytes per lane from global memory to LDS at `lds` + 16 * lane (`lds`
// wave-uniform). The compiler does not track these loads; the kernel waits
// for them explicitly.
__device__ __forceinline__ void dma16_stream(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off sc1 nt" ::"v"(g),
                 "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}

template <uint32_t N>
__device__ __forceinline__ void vmcnt_le() {
    static_assert(N < 16, "vmcnt");
    __builtin_amdgcn_s_waitcnt(0x0F70 | N);  // vmcnt <= N, other counters untouched
}

// The read-floor variants that bench.py times beside the default shape
// (vbs_gfx950_checksum_variant): how W waves per workgroup, R runs per wave
// and the load path (LDS DMA, or 16-byte vector loads into registers)
// change the time to read the same bytes once.
template <uint32_t W, uint32_t R, bool REG>
__global__ __launch_bounds__(64 * W) void k_checksum(const uint8_t *__restrict__ p, uint64_t bytes,
                                                      uint32_t span, uint32_t *__restrict__ partials) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint64_t lo = (uint64_t)blockIdx.x * span;
    const uint64_t hi = lo + span < bytes ? lo + span : bytes;
    auto chunk = [&](uint32_t u) {  // this lane's chunk of the wave's run u
        return lo + (uint64_t)(W * u + wave) * 1024u + 16u * lane;
    };
    uint32_t x = 0;
    if constexpr (REG) {
        // every run's load in flight at once, XORed in issue order
        typedef uint32_t v4u __attribute__((ext_vector_type(4)));
        v4u v[R];
#pragma unroll
        for (uint32_t u = 0; u < R; u++)
            v[u] = chunk(u) + 16u <= hi
                       ? __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p + chunk(u)))
                       : v4u{0u, 0u, 0u, 0u};
#pragma unroll
        for (uint32_t u = 0; u < R; u++) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    } else {
        static_assert(R <= 7u, "vmcnt switch");
        const uint32_t slot0 = (uint32_t)(uintptr_t)lds + wave * R * 1024u;
        // a run is issued when its first chunk lies in the span (its later
        // lanes are masked past the end), so `nv` counts the wave's DMAs
        uint32_t nv = 0;
#pragma unroll
        for (uint32_t u = 0; u < R; u++) {
            if (chunk(u) + 16u <= hi) dma16_stream(p + chunk(u), slot0 + 1024u * u);
            nv += lo + (uint64_t)(W * u + wave) * 1024u + 16u <= hi;
        }
#pragma unroll
        for (uint32_t u = 0; u < R; u++) {
            if (u < nv) {
                switch (nv - 1u - u) {  // run u has landed once the later runs alone may be pending
                    case 0: vmcnt_le<0>(); break;
                    case 1: vmcnt_le<1>(); break;
                    case 2: vmcnt_le<2>(); break;
                    case 3: vmcnt_le<3>(); break;
                    case 4: vmcnt_le<4>(); break;
                    case 5: vmcnt_le<5>(); break;
                    default: vmcnt_le<6>(); break;
                }
                asm volatile("" ::: "memory");
                if (chunk(u) + 16u <= hi) {
                    const uint4 v =
                        *reinterpret_cast<const uint4 *>(lds + wave * R * 1024u + 1024u * u + 16u * lane);
                    x ^= v.x ^ v.y ^ v.z ^ v.w;
                }
            }
        }
    }
    // fold the lanes: XOR within each row of 16 by DPP shifts, then the rows' last lanes
    auto dpp_xor = [&](uint32_t v, auto ctrl) {
        return v ^ (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, decltype(ctrl)::value, 0xF, 0xF, false);
    };
    x = dpp_xor(x, std::integral_constant<int, 0x111>{});  // row_shr:1
    x = dpp_xor(x, std::integral_constant<int, 0x112>{});  // row_shr:2
    x = dpp_xor(x, std::integral_constant<int, 0x114>{});  // row_shr:4
    x = dpp_xor(x, std::integral_constant<int, 0x118>{});  // row_shr:8
    x = __builtin_amdgcn_readlane(x, 15) ^ __builtin_amdgcn_readlane(x, 31) ^
        __builtin_amdgcn_readlane(x, 47) ^ __builtin_amdgcn_readlane(x, 63);
    if (lane == 0) partials[blockIdx.x * W + wave] = x;
}

// Variant shapes: 0 the default (one 16-wave workgroup per CU, 112 KB spans
// by LDS DMA), 1 two 8-wave workgroups per CU (56 KB spans, LDS DMA), 2 the
// default shape with vector loads into registers instead of LDS DMA.
struct CsShape {
    uint32_t waves, runs, wgs;
    bool reg;
};
static CsShape cs_shape(int variant) {
    switch (variant) {
        case 1: return {8u, kCsRuns, 2u * kCsWgs, false};
        case 2: return {kCsWaves, kCsRuns, kCsWgs, true};
        default: return {kCsWaves, kCsRuns, kCsWgs, false};
    }
}

// Span per workgroup: the region over the shape's workgroups in whole KB, at
// most waves x runs KB.
static uint32_t checksum_span(uint64_t bytes, const CsShape &c) {
    const uint64_t max = (uint64_t)c.waves * c.runs * 1024u;
    const uint64_t per = ((bytes + c.wgs - 1) / c.wgs + 1023u) / 1024u * 1024u;
    return (uint32_t)(per < max ? per : max);
}

static uint32_t checksum_wgs(uint64_t bytes, const CsShape &c) {
    return (uint32_t)((bytes + checksum_span(bytes, c) - 1) / checksum_span(bytes, c));
}

uint32_t checksum_partials(uint64_t bytes, int variant) {
    const CsShape c = cs_shape(variant);
    return bytes ? c.waves * checksum_wgs(bytes, c) : 0u;
}

template <uint32_t W, uint32_t R, bool REG>
static hipError_t launch_cs(const uint8_t *p, uint64_t bytes, uint32_t *partials, const CsShape &c,
                            hipStream_t s) {
    const size_t lds = REG ? 0u : (size_t)W * R * 1024u;
    static bool granted = false;
    if (!granted && lds) {
        if (hipFuncSetAttribute((const void *)k_checksum<W, R, REG>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorNotSupported;
        }
        granted = true;
    }
    k_checksum<W, R, REG><<<checksum_wgs(bytes, c), 64 * W, lds, s>>>(p, bytes, checksum_span(bytes, c),
                                                                     partials);
    return hipGetLastError();
}

hipError_t launch_checksum(const uint8_t *p, uint64_t bytes, uint32_t *partials, int variant,
                           hipStream_t s) {
    if (bytes == 0) return hipSuccess;
    const CsShape c = cs_shape(variant);
    switch (variant) {
        case 1: return launch_cs<8u, kCsRuns, false>(p, bytes, partials, c, s);
        case 2: return launch_cs<kCsWaves, kCsRuns, true>(p, bytes, partials, c, s);
        default: return launch_cs<kCsWaves, kCsRuns, false>(p, bytes, partials, c, s);
    }
}

}  // namespace vbs
