// vbs_kern_mfma_batch.hip — batched (skinny) K-quant matvec on the gfx950 f16
// matrix cores: x preparation (k_xprep_b) and the k_mvb kernel, with the weight
// loads of the batch-1 kernel (vbs_mfma.h).
#include "vbs_attn_common.h"
#include "vbs_lds_dma.h"
#include "vbs_mfma.h"

namespace vbs {

// ==== batched (skinny) K-quant matvec: up to 8 activation vectors ====================
//
// Y[t][r] = sum_c deq(W[r,c]) * X[t][c] for t < batch <= 8, the reference's linear
// (src/vbs_host_math.h:223-267) once per vector, with W read once. This is a
// skinny GEMM, computed on the f16 matrix cores with fp32 accumulation:
//
// * x in f16 pairs. Every 256-element block b of vector t is scaled by
//   2^s_tb so that its largest |x| lies in [2^14, 2^15), and each element
//   x' = x 2^s_tb becomes hi + lo with hi = f16(x') and lo = f16(x' - hi): 22
//   significant bits, each element represented to ~2^-23 of itself (or of
//   2^-10 below its block's maximum). Plane 2t holds hi, plane 2t + 1 lo,
//   stored chunk-major: eight elements of plane 0, the same eight of plane
//   1, ... of plane 15, then the next eight, so the sixteen A rows of an
//   MFMA's k range are one contiguous 256-byte run per lane group (one load
//   instruction reads whole cache lines); A row n of an MFMA is plane n, so D row 2t + h is vector
//   t's dot with hi or lo, the two add up in fp32, and the block's sum is
//   scaled back by 2^-s_tb. Rows past 2 batch re-read the last plane and are
//   never stored. An inf or NaN in a block makes its lo plane NaN (inf - inf),
//   so the vector's outputs are NaN.
// * Q4_K (v_mfma_f32_16x16x32_f16). The weight operand is sc * nib, the 6-bit
//   sub-block scale times the nibble: an integer below 945, exact in f16. The
//   scale is inside the operand, so one MFMA may mix sub-blocks and the
//   eight MFMAs of a block chain into one accumulator; lane group g takes the
//   nibbles of its two 16-byte loads (qs bytes 16g.. and 64 + 16g..) in any
//   order as long as its A operand holds the same elements. The mins go
//   through a ninth MFMA: A = the per-sub-block sums of x'/32 (hi and lo
//   planes), B = the 6-bit mins, in lane group 0 only. Per block and row:
//   d * D - 32 dmin * Dmin, as the reference's sum of d*sc*nib - dmin*m.
// * Q6_K (v_mfma_f32_16x16x16_f16, one 16-element scale group per MFMA). The
//   int8 scale times (q - 32) can exceed f16's exact integers, so the weight
//   operand is q - 32 and the scale multiplies each group's dot afterwards:
//   d * sum_g sc_g * D_g. Rows are read as aligned 16-byte chunks staged in
//   LDS, as in the batch-1 kernel.
//
// Work split as in the batch-1 kernel: a workgroup owns TPW tiles of 16 rows,
// its waves split the row by super-blocks (wave w: blocks w, w + nw, ...), a
// wave's A operands of a block serve all its TPW tiles, and the loads of the
// next block are in flight while one block is computed. The waves' partial
// sums are added in wave order at the end.

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kBatchMax = 8;

// Prepared x: [cols/8][16 planes][8] f16 | [cols/256][16 planes][8] f16
// sub-block sums of x'/32 | int s[cols/256][8] (block, vector).
struct XbLayout {
    uint32_t msum, expo, bytes;
};
__host__ __device__ inline XbLayout xb_layout(uint32_t cols) {
    XbLayout L;
    L.msum = 32u * cols;
    L.expo = 33u * cols;
    L.bytes = 33u * cols + cols / 8u;
    return L;
}

// What the prep reads (XP_* in vbs_internal.h): x itself, rms_norm(x) * w
// (k_rms_norm's arithmetic and block order, src/vbs_host_math.h:28-36), or
// silu(gate) * up (src/vbs_host_math.h:53-57, the E_SILU epilogue's expression).
// One wave per (256-element block, vector): lane l holds elements 4l..4l+3.
// XP_NORM: the workgroup first sums the squares of the whole vector (blocks
// split over its waves, added in block order).
// Block b of vector t (one wave, lane l: elements 4l..4l+3 of the block in v)
// into the prepared form: its exponent, f16 hi/lo planes 2t and 2t + 1 and the
// sub-block sums of x'/32.
__device__ __forceinline__ void xprep_block(const float v[4], uint32_t lane, uint32_t t, uint32_t b,
                                            uint32_t cols, uint8_t *xp) {
    const uint32_t e0 = 256u * b + 4u * lane;
    const float amax = wave_max(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    int e = 0;
    (void)frexpf(amax, &e);  // amax < 2^e
    const int s = amax > 0.f ? 15 - e : 0;
    h2 hi[2], lo[2];
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float xs2 = ldexpf(v[k], s);
        const _Float16 h = (_Float16)xs2;
        hi[k >> 1][k & 1] = h;
        lo[k >> 1][k & 1] = (_Float16)(xs2 - (float)h);
        sum += xs2;
    }
    const XbLayout L = xb_layout(cols);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    // elements e0..e0+3: chunk e0 / 8, half lane & 1; planes 2t and 2t + 1
    _Float16 *ph = reinterpret_cast<_Float16 *>(xp) + 128u * (e0 >> 3) + 8u * (2u * t) + 4u * (lane & 1u);
    *reinterpret_cast<u32x2 *>(ph) = u32x2{__builtin_bit_cast(uint32_t, hi[0]), __builtin_bit_cast(uint32_t, hi[1])};
    *reinterpret_cast<u32x2 *>(ph + 8u) = u32x2{__builtin_bit_cast(uint32_t, lo[0]), __builtin_bit_cast(uint32_t, lo[1])};
    // sub-block sums of x'/32: eight lanes per 32 elements
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);
    sum += __shfl_xor(sum, 4, 64);
    if ((lane & 7u) == 0) {
        const float m = sum * 0.03125f;
        const _Float16 h = (_Float16)m;
        _Float16 *pm = reinterpret_cast<_Float16 *>(xp + L.msum) + 128u * b + 8u * (2u * t) + lane / 8u;
        pm[0] = h;
        pm[8] = (_Float16)(m - (float)h);
    }
    if (lane == 0) reinterpret_cast<int *>(xp + L.expo)[8u * b + t] = s;
}

template <int MODE>
__global__ __launch_bounds__(256) void k_xprep_b(const float *x, const float *x2, uint32_t xs,
                                                 const float *norm_w, float eps, uint32_t cols,
                                                 uint8_t *xp) {
    __shared__ double bsum[128];
    const uint32_t t = blockIdx.y, lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t b = blockIdx.x * 4u + wave, nblk = cols >> 8;
    typedef float4 __attribute__((aligned(4))) f4u;
    const float *xt = x + (uint64_t)t * xs;
    float sc = 1.0f;
    if (MODE == XP_NORM) {
        // the wave's blocks wave, wave + 4, ...: eight requested at a time,
        // then their sums of squares
        for (uint32_t k0 = wave; k0 < nblk; k0 += 32u) {
            float4 a[8];
#pragma unroll
            for (uint32_t j = 0; j < 8u; j++) {
                const uint32_t k = min(k0 + 4u * j, nblk - 1u);
                a[j] = *reinterpret_cast<const f4u *>(xt + 256u * k + 4u * lane);
            }
#pragma unroll
            for (uint32_t j = 0; j < 8u; j++) {
                const uint32_t k = k0 + 4u * j;
                if (k < nblk) {  // (wave-uniform)
                    const float v[4] = {a[j].x, a[j].y, a[j].z, a[j].w};
                    const double ss = block_sumsq(v);
                    if (lane == 0) bsum[k] = ss;
                }
            }
        }
        __syncthreads();
        double tot = 0.0;
        for (uint32_t k = 0; k < nblk; k++) tot += bsum[k];
        const float mean = (float)(tot / (double)cols);
        sc = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
    }
    if (b >= nblk) return;
    const uint32_t e0 = 256u * b + 4u * lane;
    const float4 xv = *reinterpret_cast<const f4u *>(xt + e0);
    float v[4] = {xv.x, xv.y, xv.z, xv.w};
    if (MODE == XP_NORM) {
        const float4 wv = *reinterpret_cast<const f4u *>(norm_w + e0);
        const float w4[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = __fmul_rn(__fmul_rn(v[k], sc), w4[k]);
    } else if (MODE == XP_SILU) {
        const float4 uv = *reinterpret_cast<const f4u *>(x2 + (uint64_t)t * xs + e0);
        const float u4[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
        for (int k = 0; k < 4; k++)
            v[k] = __fmul_rn(__fdiv_rn(v[k], __fadd_rn(1.0f, expf(-v[k]))), u4[k]);
    }
    xprep_block(v, lane, t, b, cols, xp);
}

// Up to three matrices of the same type and column count over one prepared x
// (Q, K, V or gate, up), tiles numbered across them.
struct MbArgs {
    const uint8_t *w[3];
    float *y[3];
    uint32_t ys[3], rows[3];
    uint32_t tile_end[3];  // cumulative 16-row tiles per matrix
    uint32_t nmat;
    const uint8_t *xp;
    uint32_t cols, batch;
    // E_QKV (the batched decoder's Q/K/V launch, matrices q, k, v): RoPE of the
    // q and k rows at sequence t's device position pos[t] (table rope[pos][hd/2]),
    // q rows to y[0], k and v rows as f16 to the caches at t * kv_seq +
    // layer_off + pos[t] * kvd (src/vbs_host_math.h:38-51, 150-159)
    const float2 *rope;
    const uint32_t *pos;
    uint16_t *kc, *vc;
    uint64_t kv_seq, layer_off;
    uint32_t hd, kvd, max_ctx;
    // ranged k_mvbr4 launches: workgroups of matrix m end at rwg_end[m]
    // (cumulative), each taking rpw[m] rows of it (the last one of a matrix fewer)
    uint32_t rwg_end[3], rpw[3];
};

// This lane's A row: its plane's first eight elements and first eight
// sub-block sums; element chunk c of the plane is at plane + 128 c, block b's
// sums at msum + 128 b.
struct XbView {
    const _Float16 *plane, *msum;
    const int *expo;
};

// {1024 + byte, 1024 + byte'} as an f16 pair: bytes (0, 1) of w for sel
// 0x00050004, (2, 3) for 0x00070006, (k, k) for 0x00040004 + 0x00010001 k.
__device__ __forceinline__ h2 f16_bytes(uint32_t w, uint32_t sel) {
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(w, 0x64646464u, sel));
}
__device__ __forceinline__ h8 join8(h2 a, h2 b, h2 c, h2 d) {
    const u32x4 v = {__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                     __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d)};
    return __builtin_bit_cast(h8, v);
}
__device__ __forceinline__ h4 join4(h2 a, h2 b) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = {__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
    return __builtin_bit_cast(h4, v);
}

struct Q4KB {
    typedef Q4K Load;
    static constexpr uint32_t BYTES = 144, NLD = Q4K::NLD, SCRATCH = 0;
    struct A {
        h8 m[8], mn;
        int2 s;  // block exponents of the lane's two D vectors
    };
    // MFMA m, lane group g, slot k: element 32 j + 16 (g & 1) + 8 (m & 1) + k of
    // the block, j = 4 (m >> 2) + 2 (g >> 1) + ((m >> 1) & 1) (the nibbles of
    // qs byte 16 g + 8 (m & 1) + k, or of byte 64 + ..., low or high half).
    __device__ static void load_a(const XbView &v, uint32_t b, uint32_t g, A &a) {
        // element 256 b + 32 j + 16 (g & 1) + 8 (m & 1): chunk 32 b + 4 j + 2 (g & 1) + (m & 1)
        const _Float16 *p = v.plane + 128u * (32u * b + 2u * (g & 1u));
#pragma unroll
        for (uint32_t m = 0; m < 8u; m++) {
            const uint32_t j = 4u * (m >> 2) + 2u * (g >> 1) + ((m >> 1) & 1u);
            a.m[m] = *reinterpret_cast<const h8 *>(p + 128u * (4u * j + (m & 1u)));
        }
        const h8 t = *reinterpret_cast<const h8 *>(v.msum + 128u * b), z = {};
        a.mn = g == 0u ? t : z;
        a.s = *reinterpret_cast<const int2 *>(v.expo + 8u * b + 2u * g);
    }
    __device__ static void dot(const u32x4 *r, const A &x, uint8_t *, const Src &, uint32_t,
                               uint32_t, uint32_t g, float acc[2]) {
        const u32x4 hd = r[0], qa = r[1], qb = r[2];
        // scales and mins, one per byte (src/vbs_dequant.c:225-233)
        const uint32_t sclo = hd.y & 0x3F3F3F3Fu;
        const uint32_t schi = (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u);
        const uint32_t mnlo = hd.z & 0x3F3F3F3Fu;
        const uint32_t mnhi = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
        const h2 n1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
        const h2 n64 = {(_Float16)-64.f, (_Float16)-64.f};
        const h2 r16 = {(_Float16)0.0625f, (_Float16)0.0625f};
        const uint32_t k0 = 0x00040004u + 0x00020002u * (g >> 1);  // byte 2 (g >> 1)
        // sub-blocks of this lane group: 2(g>>1) (qa low), +1 (qa high), 4 + 2(g>>1)
        // (qb low), +1 (qb high); low nibbles: fma(1024 + n, sc, -1024 sc),
        // high nibbles: fma(1024 + 16 n, sc / 16, -64 sc), both exactly sc * n
        const h2 s0 = f16_bytes(sclo, k0) + n1024, s1 = f16_bytes(sclo, k0 + 0x00010001u) + n1024;
        const h2 s2 = f16_bytes(schi, k0) + n1024, s3 = f16_bytes(schi, k0 + 0x00010001u) + n1024;
        const h2 mul[4] = {s0, s1 * r16, s2, s3 * r16};
        const h2 add[4] = {s0 * n1024, s1 * n64, s2 * n1024, s3 * n64};
        f4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t m = 0; m < 8u; m++) {
            const u32x4 q = (m >> 2) ? qb : qa;
            const uint32_t hs = (m >> 1) & 1u, si = 2u * (m >> 2) + hs;
            const uint32_t mask = hs ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
            const uint32_t w0 = ((m & 1u) ? q.z : q.x) & mask, w1 = ((m & 1u) ? q.w : q.y) & mask;
            const h8 B = join8(__builtin_elementwise_fma(f16_bytes(w0, 0x00050004u), mul[si], add[si]),
                               __builtin_elementwise_fma(f16_bytes(w0, 0x00070006u), mul[si], add[si]),
                               __builtin_elementwise_fma(f16_bytes(w1, 0x00050004u), mul[si], add[si]),
                               __builtin_elementwise_fma(f16_bytes(w1, 0x00070006u), mul[si], add[si]));
            D = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.m[m], B, D, 0, 0, 0);
        }
        const h8 Bm = join8(f16_bytes(mnlo, 0x00050004u) + n1024, f16_bytes(mnlo, 0x00070006u) + n1024,
                            f16_bytes(mnhi, 0x00050004u) + n1024, f16_bytes(mnhi, 0x00070006u) + n1024);
        const f4 z = {0.f, 0.f, 0.f, 0.f};
        const f4 Dm = __builtin_amdgcn_mfma_f32_16x16x32_f16(x.mn, Bm, z, 0, 0, 0);
        const float d = cvt_h(hd.x & 0xFFFFu), md = -32.f * cvt_h(hd.x >> 16);
        acc[0] += ldexpf(fmaf(d, D[0] + D[1], md * (Dm[0] + Dm[1])), -x.s.x);
        acc[1] += ldexpf(fmaf(d, D[2] + D[3], md * (Dm[2] + Dm[3])), -x.s.y);
    }
};

struct Q6KB {
    typedef Q6K Load;
    static constexpr uint32_t BYTES = 210, NLD = Q6K::NLD, SCRATCH = Q6K::SCRATCH;
    struct A {
        h4 g[16];
        int2 s;  // block exponents of the lane's two D vectors
    };
    // MFMA G = 8h + 2q + u (scale group G), lane group g, slot k: element
    // 128 h + 32 q + 16 u + 4 g + k (src/vbs_dequant.c:316-333)
    __device__ static void load_a(const XbView &v, uint32_t b, uint32_t g, A &a) {
        // element 256 b + 128 (G >> 3) + 32 ((G >> 1) & 3) + 16 (G & 1) + 4 g:
        // chunk 32 b + 16 (G >> 3) + 4 ((G >> 1) & 3) + 2 (G & 1) + (g >> 1), half g & 1
        const _Float16 *p = v.plane + 128u * (32u * b + (g >> 1)) + 4u * (g & 1u);
#pragma unroll
        for (uint32_t G = 0; G < 16u; G++)
            a.g[G] = *reinterpret_cast<const h4 *>(p + 128u * (16u * (G >> 3) + 4u * ((G >> 1) & 3u) +
                                                               2u * (G & 1u)));
        a.s = *reinterpret_cast<const int2 *>(v.expo + 8u * b + 2u * g);
    }
    __device__ static void dot(const u32x4 *r, const A &x, uint8_t *scratch, const Src &src,
                               uint32_t b, uint32_t n, uint32_t g, float acc[2]) {
        const uint32_t lane = 16u * g + n;
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t c = lane + 64u * i;
            if (i < 3u || c < 224u) *reinterpret_cast<u32x4 *>(scratch + 16u * c) = r[i];
        }
        dot_staged(scratch, x, src, b, n, g, acc);
    }
    // The same from a scratch that already holds the tile's 224 chunks (chunk
    // 14 n + k at 16 (14 n + k): row n's aligned 16-byte chunk k).
    __device__ static void dot_staged(const uint8_t *scratch, const A &x, const Src &src, uint32_t b,
                                      uint32_t n, uint32_t g, float acc[2]) {
        // row n's block starts o = (its address mod 16) into its 224 scratch bytes
        const uint32_t o = ((uint32_t)(uintptr_t)src.w + src.row(n) + b * BYTES) & 15u;
        const uint32_t *rw = reinterpret_cast<const uint32_t *>(scratch + 224u * n + (o & 12u));
        const uint32_t sh = o & 2u;
        auto dw = [&](uint32_t f) { return __builtin_amdgcn_alignbyte(rw[f / 4u + 1u], rw[f / 4u], sh); };
        uint32_t ql[8], qh[4], sc[4];
#pragma unroll
        for (uint32_t i = 0; i < 8u; i++)  // i = 4h + 2(q & 1) + u
            ql[i] = dw(64u * (i >> 2) + 32u * ((i >> 1) & 1u) + 16u * (i & 1u) + 4u * g);
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++)  // i = 2h + u
            qh[i] = dw(128u + 32u * (i >> 1) + 16u * (i & 1u) + 4u * g);
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) sc[i] = dw(192u + 4u * i);
        const uint32_t dbits = (rw[52] >> (8u * sh)) & 0xFFFFu;
        const h2 n1056 = {(_Float16)-1056.f, (_Float16)-1056.f};
        const f4 z = {0.f, 0.f, 0.f, 0.f};
        float a0 = 0.f, a1 = 0.f, c0 = 0.f, c1 = 0.f;
        auto bq = [&](uint32_t G) {
            const uint32_t h = G >> 3, q = (G >> 1) & 3u, u = G & 1u;
            const uint32_t l4 = (ql[4u * h + 2u * (q & 1u) + u] >> (4u * (q >> 1))) & 0x0F0F0F0Fu;
            const uint32_t h2b = (qh[2u * h + u] >> (2u * q)) & 0x03030303u;
            const uint32_t q6 = l4 | (h2b << 4);
            return join4(f16_bytes(q6, 0x00050004u) + n1056, f16_bytes(q6, 0x00070006u) + n1056);
        };
        auto scale = [&](uint32_t G) { return (float)(int)(int8_t)(sc[G >> 2] >> (8u * (G & 3u))); };
        // two independent chains (groups G and G + 8): each MFMA's result is
        // consumed after the other chain's MFMA has issued
#pragma unroll
        for (uint32_t G = 0; G < 8u; G++) {
            const f4 D0 = __builtin_amdgcn_mfma_f32_16x16x16f16(x.g[G], bq(G), z, 0, 0, 0);
            const f4 D1 = __builtin_amdgcn_mfma_f32_16x16x16f16(x.g[G + 8u], bq(G + 8u), z, 0, 0, 0);
            const float s0 = scale(G), s1 = scale(G + 8u);
            a0 = fmaf(s0, D0[0] + D0[1], a0);
            a1 = fmaf(s0, D0[2] + D0[3], a1);
            c0 = fmaf(s1, D1[0] + D1[1], c0);
            c1 = fmaf(s1, D1[2] + D1[3], c1);
        }
        a0 += c0;
        a1 += c1;
        const float d = cvt_h(dbits);
        acc[0] += ldexpf(d * a0, -x.s.x);
        acc[1] += ldexpf(d * a1, -x.s.y);
    }
};

template <class T, uint32_t TPW, bool ACC>
__global__ __launch_bounds__(512) void k_mvb(const MbArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t cols = a.cols, nblk = cols >> 8, rb = nblk * T::BYTES;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u, nw = blockDim.x >> 6;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const XbLayout L = xb_layout(cols);
    const uint32_t p = min(n, 2u * a.batch - 1u);
    const XbView xv{reinterpret_cast<const _Float16 *>(a.xp) + 8u * p,
                    reinterpret_cast<const _Float16 *>(a.xp + L.msum) + 8u * p,
                    reinterpret_cast<const int *>(a.xp + L.expo)};
    const uint32_t total = a.tile_end[a.nmat - 1u];
    Src src[TPW];
    uint32_t mt[TPW], lt[TPW];
#pragma unroll
    for (uint32_t j = 0; j < TPW; j++) {
        const uint32_t gt = min(blockIdx.x * TPW + j, total - 1u);
        mt[j] = (gt >= a.tile_end[0]) + (a.nmat > 2u && gt >= a.tile_end[1]);
        lt[j] = gt - (mt[j] ? a.tile_end[mt[j] - 1u] : 0u);
        src[j] = Src{a.w[mt[j]], a.rows[mt[j]] * rb, rb, lt[j] * 16u, a.rows[mt[j]]};
    }
    uint8_t *scratch = lds + wave * T::SCRATCH;
    float acc[TPW][2];
#pragma unroll
    for (uint32_t j = 0; j < TPW; j++) acc[j][0] = acc[j][1] = 0.f;

    typename T::A A0, A1;
    u32x4 W0[TPW][T::NLD], W1[TPW][T::NLD];
    auto issue = [&](uint32_t b, typename T::A &A, u32x4 (&W)[TPW][T::NLD]) {
        T::load_a(xv, b, g, A);
#pragma unroll
        for (uint32_t j = 0; j < TPW; j++) T::Load::load(src[j], b, n, g, W[j]);
    };
    auto compute = [&](uint32_t b, const typename T::A &A, const u32x4 (&W)[TPW][T::NLD]) {
#pragma unroll
        for (uint32_t j = 0; j < TPW; j++) T::dot(W[j], A, scratch, src[j], b, n, g, acc[j]);
    };
    // blocks wave, wave + nw, ...: two register sets, the next block's loads
    // in flight while the current one is computed
    uint32_t b = wave;
    if (b < nblk) {
        issue(b, A0, W0);
        for (;;) {
            const uint32_t b1 = b + nw;
            if (b1 < nblk) issue(b1, A1, W1);
            compute(b, A0, W0);
            if (b1 >= nblk) break;
            const uint32_t b2 = b1 + nw;
            if (b2 < nblk) issue(b2, A0, W0);
            compute(b1, A1, W1);
            if (b2 >= nblk) break;
            b = b2;
        }
    }

    // partial sums [TPW][nw][lane][2], added in wave order; lane (n, g) holds
    // row n of the tile for vectors 2g and 2g + 1
    float *red = reinterpret_cast<float *>(lds + nw * T::SCRATCH);
#pragma unroll
    for (uint32_t j = 0; j < TPW; j++) {
        red[(j * nw + wave) * 128u + 2u * lane] = acc[j][0];
        red[(j * nw + wave) * 128u + 2u * lane + 1u] = acc[j][1];
    }
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < TPW * 128u; q += blockDim.x) {
        const uint32_t j = q >> 7, l = (q >> 1) & 63u, tk = q & 1u;
        float s = 0.f;
        for (uint32_t w = 0; w < nw; w++) s += red[(j * nw + w) * 128u + 2u * l + tk];
        const uint32_t m = mt[j], row = lt[j] * 16u + (l & 15u), t = 2u * (l >> 4) + tk;
        if (blockIdx.x * TPW + j < total && row < a.rows[m] && t < a.batch) {
            float *dst = a.y[m] + (uint64_t)t * a.ys[m] + row;
            *dst = ACC ? __fadd_rn(*dst, s) : s;
        }
    }
}

// ---- ring form of the batched Q6_K launch ----------------------------------------------
// k_mvbr6: the batch-1 ring kernel's structure (k_mvr, vbs_kern_mvl.hip) with
// Q6KB's arithmetic. One 16-wave workgroup per CU owns an even range of at
// most 16 T rows; wave w owns blocks w, w + 16, ... (NB of them; slots past the
// row re-read its last block and add nothing). Its items -- T tiles of each of
// its blocks -- come by LDS DMA into a ring of R slots, item i + R requested
// as soon as item i is computed, and the A operands of a block (the prepared
// x planes and exponents) come into registers from inline assembly with the
// block's first item, a block ahead of their use. Per tile a wave adds its
// blocks in order, and the waves' sums are added in wave order at the end.
typedef int vi2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void q6kb_load_a_async(const XbView &v, uint32_t b, uint32_t g, h4 (&ag)[16],
                                                  vi2 &as) {
    const _Float16 *p = v.plane + 128u * (32u * b + (g >> 1)) + 4u * (g & 1u);
#pragma unroll
    for (uint32_t G = 0; G < 16u; G++)
        asm volatile("global_load_dwordx2 %0, %1, off"
                     : "=v"(ag[G])
                     : "v"(p + 128u * (16u * (G >> 3) + 4u * ((G >> 1) & 3u) + 2u * (G & 1u))));
    asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(as) : "v"(v.expo + 8u * b + 2u * g));
}

template <uint32_t NB, uint32_t T, uint32_t R>
struct MvbrPlan {
    static constexpr uint32_t NI = NB * T, D = 4u, ISZ = 16u * 224u;
    static_assert(R >= 1u && R <= NI && (NB == 1u || R <= T + 1u), "ring");
    // loads that item i brings: its four DMAs, after the block's 17 A loads
    // when it opens a block
    static constexpr uint32_t with(uint32_t i) { return D + (i % T == 0u ? 17u : 0u); }
    // loads issued after item i's last one when item i is computed
    static constexpr uint32_t after_item(uint32_t i) {
        uint32_t c = 0;
        for (uint32_t j = i + 1u; j < i + R && j < NI; j++) c += with(j);
        return c;
    }
    static constexpr size_t lds() { return 16u * (size_t)R * ISZ + (size_t)T * 16u * 128u * sizeof(float); }
};

template <uint32_t NB, uint32_t T, uint32_t R, bool ACC>
__global__ __launch_bounds__(1024) void k_mvbr6(const MbArgs a, uint32_t rpw) {
    using P = MvbrPlan<NB, T, R>;
    constexpr uint32_t NI = P::NI, ISZ = P::ISZ;
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t cols = a.cols, nblk = cols >> 8, rb = nblk * 210u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t r0 = blockIdx.x * rpw, r1 = min(r0 + rpw, a.rows[0]);
    if (r0 >= r1) return;
    const XbLayout L = xb_layout(cols);
    const uint32_t pl = min(n, 2u * a.batch - 1u);
    // the lane's chunk of each of an item's four DMAs: chunk c = 14 n' + k'
    // of the tile, row n' of the tile and byte 16 k' of the row's run
    uint32_t lrow[4], lchk[4];
#pragma unroll
    for (uint32_t q = 0; q < 4u; q++) {
        const uint32_t c = min(64u * q + lane, 223u);
        lrow[q] = c / 14u;
        lchk[q] = 16u * (c % 14u);
    }
    const XbView xv{reinterpret_cast<const _Float16 *>(a.xp) + 8u * pl,
                    reinterpret_cast<const _Float16 *>(a.xp + L.msum) + 8u * pl,
                    reinterpret_cast<const int *>(a.xp + L.expo)};
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds, ring = lds0 + wave * R * ISZ;
    float *const red = reinterpret_cast<float *>(lds + 16u * R * ISZ);
    // offsets are taken from w rounded down to 16 bytes (as in Q6K::load)
    const uint8_t *const w = a.w[0];
    const uint32_t wlo = (uint32_t)(uintptr_t)w & 15u;
    h4 ag[2][16];
    vi2 as[2];
    float acc[T][2];
#pragma unroll
    for (uint32_t j = 0; j < T; j++) acc[j][0] = acc[j][1] = 0.f;

    auto issue = [&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        constexpr uint32_t k = i / T, j = i % T;
        const uint32_t b = min(wave + 16u * k, nblk - 1u);
        if constexpr (j == 0u) q6kb_load_a_async(xv, b, g, ag[k % 2u], as[k % 2u]);
        const uint32_t dst = ring + (i % R) * ISZ;
#pragma unroll
        for (uint32_t q = 0; q < 4u; q++) {
            const uint32_t st = min(r0 + 16u * j + lrow[q], r1 - 1u) * rb + b * 210u;
            const uint32_t off = ((st + wlo) & ~15u) + lchk[q];
            if (q < 3u || lane < 32u) dma16s(w - wlo, off, dst + 1024u * q);
        }
    };
    unroll_for<0u, R>(issue);

    unroll_for<0u, NI>([&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        constexpr uint32_t k = i / T, j = i % T;
        vmcnt_le<P::after_item(i)>();  // (the block's A loads precede its first item)
        asm volatile("" ::: "memory");
        if constexpr (j == 0u) {
#pragma unroll
            for (uint32_t G = 0; G < 16u; G++) asm volatile("" : "+v"(ag[k % 2u][G]));
            asm volatile("" : "+v"(as[k % 2u]));
        }
        const uint32_t bw = wave + 16u * k;
        if (bw < nblk) {
            Q6KB::A x;
#pragma unroll
            for (uint32_t G = 0; G < 16u; G++) x.g[G] = ag[k % 2u][G];
            x.s = make_int2(as[k % 2u].x, as[k % 2u].y);
            const Src src{w, a.rows[0] * rb, rb, r0 + 16u * j, r1};
            Q6KB::dot_staged(lds + (ring - lds0) + (i % R) * ISZ, x, src, bw, n, g, acc[j]);
            asm volatile("" ::"v"(acc[j][0]), "v"(acc[j][1]));
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (i + R < NI) issue(std::integral_constant<uint32_t, i + R>{});
    });

    // per tile: lane (n, g) holds row n for vectors 2g and 2g + 1; the waves'
    // sums added in wave order
#pragma unroll
    for (uint32_t j = 0; j < T; j++) {
        red[(j * 16u + wave) * 128u + 2u * lane] = acc[j][0];
        red[(j * 16u + wave) * 128u + 2u * lane + 1u] = acc[j][1];
    }
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < T * 128u; q += 1024u) {
        const uint32_t j = q >> 7, l = (q >> 1) & 63u, tk = q & 1u;
        float sum = 0.f;
        for (uint32_t v = 0; v < 16u; v++) sum += red[(j * 16u + v) * 128u + 2u * l + tk];
        const uint32_t row = r0 + 16u * j + (l & 15u), t = 2u * (l >> 4) + tk;
        if (row < r1 && t < a.batch) {
            float *dst = a.y[0] + (uint64_t)t * a.ys[0] + row;
            *dst = ACC ? __fadd_rn(*dst, sum) : sum;
        }
    }
}

template <uint32_t NB, uint32_t T, uint32_t R, bool ACC>
static hipError_t launch_mvbr6_t(const MbArgs &a, uint32_t wgs, uint32_t rpw, hipStream_t s) {
    const size_t lds = MvbrPlan<NB, T, R>::lds();
    static bool granted = false;
    if (!granted) {
        if (hipFuncSetAttribute((const void *)k_mvbr6<NB, T, R, ACC>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorNotSupported;
        }
        granted = true;
    }
    k_mvbr6<NB, T, R, ACC><<<wgs, 1024, lds, s>>>(a, rpw);
    return hipGetLastError();
}

// One Q6_K matrix of rows of 33-48 blocks over 2049-4096 rows (three blocks
// per wave, one tile) or of 97-112 blocks over 4097-8192 rows (seven blocks,
// two tiles); the matrix's last block read as aligned chunks must end inside
// it (the DMA has no bounded form).
static hipError_t launch_mvbr6(const MbArgs &a, bool acc, hipStream_t s) {
    const uint32_t nblk = a.cols / 256u, rows = a.rows[0];
    const bool narrow = nblk > 32u && nblk <= 48u, wide = nblk > 96u && nblk <= 112u;
    if (a.nmat != 1u || a.cols % 256u || !(narrow || wide) || ((uintptr_t)a.w[0] & 1u))
        return hipErrorNotSupported;
    const uint32_t wgs = device_cus();
    const uint32_t rpw = (rows + wgs - 1u) / wgs;
    if (narrow ? rows <= 2048u || rpw > 16u : rows <= 4096u || rpw > 32u) return hipErrorNotSupported;
    const uint64_t rb = (uint64_t)nblk * 210u, bytes = rb * rows, wlo = (uintptr_t)a.w[0] & 15u;
    const uint64_t last = bytes - 210u;
    if (((last + wlo) & ~(uint64_t)15u) + 224u > bytes + wlo || bytes + 256u >= (1ull << 32))
        return hipErrorNotSupported;
    const uint32_t g = (rows + rpw - 1u) / rpw;
    if (wide) return acc ? launch_mvbr6_t<7, 2, 2, true>(a, g, rpw, s) : launch_mvbr6_t<7, 2, 2, false>(a, g, rpw, s);
    return acc ? launch_mvbr6_t<3, 1, 2, true>(a, g, rpw, s) : launch_mvbr6_t<3, 1, 2, false>(a, g, rpw, s);
}

// Q4KB's A operands of block b requested from inline assembly (vbs_lds_dma.h):
// the eight k-slices, the mins' sums and the two exponents.
__device__ __forceinline__ void q4kb_load_a_async(const XbView &v, uint32_t b, uint32_t g, h8 (&am)[8],
                                                  h8 &mn, vi2 &es) {
    const _Float16 *p = v.plane + 128u * (32u * b + 2u * (g & 1u));
#pragma unroll
    for (uint32_t m = 0; m < 8u; m++) {
        const uint32_t j = 4u * (m >> 2) + 2u * (g >> 1) + ((m >> 1) & 1u);
        asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(am[m]) : "v"(p + 128u * (4u * j + (m & 1u))));
    }
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(mn) : "v"(v.msum + 128u * b));
    asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(es) : "v"(v.expo + 8u * b + 2u * g));
}

// ---- ring form of the batched Q4_K launch ----------------------------------------------
// k_mvbr4: one 16-wave workgroup per CU owns T consecutive tiles (of up to three
// matrices); wave w owns blocks w, w + 16, ... (NB of them) and for each of them
// all T tiles, so a block's A operands (Q4KB's, 10 loads from inline assembly)
// serve T items. The items -- for each of the wave's blocks, its T tiles'
// 16 x 144 bytes -- come by LDS DMA into a ring of R slots, item i + R requested
// as soon as item i is computed; the next block's A operands are requested
// after the current block's last item, into the same registers. Per tile a wave
// adds its blocks in order; the waves' sums meet in LDS (the ring's space, a
// pass of up to kMvbr4Pass tiles at a time) and are added in wave order.
template <uint32_t NB, uint32_t T, uint32_t R>
struct Mvbr4Plan {
    static constexpr uint32_t NI = NB * T, ISZ = 16u * 144u;
    static_assert(R >= 1u && R <= NI, "ring");
    // Loads issued after the awaited one when item i is computed: the awaited
    // one is item i's last DMA, or for the first item of a later block that
    // block's A. Issue order: A(0), items 0 .. R - 1; after computing item s,
    // A(k) when s is the last item of block k - 1, then item s + R.
    static constexpr uint32_t wait_count(uint32_t i) {
        const bool await_a = i % T == 0u && i >= T;
        uint32_t count = 0;
        bool after = false;
        auto visit = [&](bool is_a, uint32_t idx, uint32_t n) {
            if (after)
                count += n;
            else if (await_a ? (is_a && idx == i / T) : (!is_a && idx == i))
                after = true;
        };
        visit(true, 0u, 10u);
        for (uint32_t q = 0; q < R; q++) visit(false, q, 3u);
        for (uint32_t st = 0; st < i; st++) {
            if ((st + 1u) % T == 0u && (st + 1u) / T < NB) visit(true, (st + 1u) / T, 10u);
            if (st + R < NI) visit(false, st + R, 3u);
        }
        return count;
    }
    static constexpr size_t lds() { return 16u * (size_t)R * ISZ; }
};
constexpr uint32_t kMvbr4Pass = 12;  // tiles per reduction pass (12 x 8 KB in the ring's 110 KB)

template <uint32_t NB, uint32_t T, uint32_t R, int EPI, bool RANGED = false>
__global__ __launch_bounds__(1024) void k_mvbr4(const MbArgs a) {
    using P = Mvbr4Plan<NB, T, R>;
    constexpr uint32_t NI = P::NI, ISZ = P::ISZ;
    static_assert(16u * R * ISZ >= (T < kMvbr4Pass ? T : kMvbr4Pass) * 16u * 128u * sizeof(float), "pass");
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t cols = a.cols, nblk = cols >> 8, rb = nblk * 144u;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t total = a.tile_end[a.nmat - 1u], gt0 = blockIdx.x * T;
    if (!RANGED && gt0 >= total) return;
    const XbLayout L = xb_layout(cols);
    const uint32_t pl = min(n, 2u * a.batch - 1u);
    const XbView xv{reinterpret_cast<const _Float16 *>(a.xp) + 8u * pl,
                    reinterpret_cast<const _Float16 *>(a.xp + L.msum) + 8u * pl,
                    reinterpret_cast<const int *>(a.xp + L.expo)};
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds, ring = lds0 + wave * R * ISZ;
    // RANGED: the workgroup's matrix and rows [r0, r1)
    uint32_t rm = 0, r0 = 0, r1 = 0;
    if constexpr (RANGED) {
        rm = (uint32_t)(blockIdx.x >= a.rwg_end[0]) + (uint32_t)(blockIdx.x >= a.rwg_end[1]);
        const uint32_t start = rm == 0u ? 0u : rm == 1u ? a.rwg_end[0] : a.rwg_end[1];
        const uint32_t rpw = rm == 0u ? a.rpw[0] : rm == 1u ? a.rpw[1] : a.rpw[2];
        r0 = (blockIdx.x - start) * rpw;
        r1 = min(r0 + rpw, rm == 0u ? a.rows[0] : rm == 1u ? a.rows[1] : a.rows[2]);
    }
    // tile j of the workgroup: matrix, first row and row bound (tiles past the
    // last one repeat it and are not stored; RANGED: rows past r1 re-read row
    // r1 - 1 and are not stored)
    auto tile = [&](uint32_t j, uint32_t &m, uint32_t &base, uint32_t &bound) {
        if constexpr (RANGED) {
            m = rm;
            base = r0 + 16u * j;
            bound = r1;
        } else {
            const uint32_t gt = min(gt0 + j, total - 1u);
            m = (gt >= a.tile_end[0]) + (a.nmat > 2u && gt >= a.tile_end[1]);
            base = 16u * (gt - (m == 0u ? 0u : m == 1u ? a.tile_end[0] : a.tile_end[1]));  // (no dynamic
            bound = m == 0u ? a.rows[0] : m == 1u ? a.rows[1] : a.rows[2];  // index into the arguments)
        }
    };
    // every tile's matrix and this lane's three chunk offsets in it, computed
    // before the first DMA (argument reads inside the stream would wait for it)
    const uint8_t *tw[T];
    uint32_t toff[T][3];
#pragma unroll
    for (uint32_t j = 0; j < T; j++) {
        uint32_t m, base, bound;
        tile(j, m, base, bound);
        tw[j] = m == 0u ? a.w[0] : m == 1u ? a.w[1] : a.w[2];
#pragma unroll
        for (uint32_t q = 0; q < 3u; q++) {
            const uint32_t c = min(64u * q + lane, 143u);  // chunk 9 n' + p of the tile
            toff[j][q] = min(base + c / 9u, bound - 1u) * rb + 16u * (c % 9u);
        }
    }
    auto issue = [&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        constexpr uint32_t k = i / T, j = i % T;
        const uint32_t b = min(wave + 16u * k, nblk - 1u);
        const uint32_t dst = ring + (i % R) * ISZ;
#pragma unroll
        for (uint32_t q = 0; q < 3u; q++)
            if (q < 2u || lane < 16u) dma16(tw[j] + toff[j][q] + b * 144u, dst + 1024u * q);
    };
    h8 am[8], mn;
    vi2 es;
    float acc[T][2];
#pragma unroll
    for (uint32_t j = 0; j < T; j++) acc[j][0] = acc[j][1] = 0.f;
    q4kb_load_a_async(xv, min(wave, nblk - 1u), g, am, mn, es);
    unroll_for<0u, R>(issue);

    unroll_for<0u, NI>([&](auto ic) {
        constexpr uint32_t i = decltype(ic)::value;
        constexpr uint32_t k = i / T, j = i % T;
        vmcnt_le<P::wait_count(i)>();
        asm volatile("" ::: "memory");
        if constexpr (j == 0u) {
#pragma unroll
            for (uint32_t q = 0; q < 8u; q++) asm volatile("" : "+v"(am[q]));
            asm volatile("" : "+v"(mn), "+v"(es));
        }
        const uint32_t bw = wave + 16u * k;
        if (bw < nblk) {
            Q4KB::A x;
#pragma unroll
            for (uint32_t q = 0; q < 8u; q++) x.m[q] = am[q];
            const h8 z = {};
            x.mn = g == 0u ? mn : z;
            x.s = make_int2(es.x, es.y);
            const uint8_t *row = lds + (ring - lds0) + (i % R) * ISZ + 144u * n;
            u32x4 r[3];
            r[0] = lda4(row);
            r[1] = lda4(row + 16u + 16u * g);
            r[2] = lda4(row + 80u + 16u * g);
            const Src src{a.w[0], 0u, rb, 0u, 1u};  // (Q4KB::dot reads nothing through it)
            Q4KB::dot(r, x, nullptr, src, bw, n, g, acc[j]);
            asm volatile("" ::"v"(acc[j][0]), "v"(acc[j][1]));
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (j == T - 1u && k + 1u < NB)
            q4kb_load_a_async(xv, min(wave + 16u * (k + 1u), nblk - 1u), g, am, mn, es);
        if constexpr (i + R < NI) issue(std::integral_constant<uint32_t, i + R>{});
    });

    // per tile: lane (n, g) holds row n for vectors 2g and 2g + 1; the waves'
    // sums meet in the ring's space and are added in wave order
    __syncthreads();
    float *const red = reinterpret_cast<float *>(lds);
    unroll_for<0u, (T + kMvbr4Pass - 1u) / kMvbr4Pass>([&](auto pc) {
        constexpr uint32_t j0 = decltype(pc)::value * kMvbr4Pass;
        constexpr uint32_t jn = T - j0 < kMvbr4Pass ? T - j0 : kMvbr4Pass;
#pragma unroll
        for (uint32_t jj = 0; jj < jn; jj++) {
            red[(jj * 16u + wave) * 128u + 2u * lane] = acc[j0 + jj][0];
            red[(jj * 16u + wave) * 128u + 2u * lane + 1u] = acc[j0 + jj][1];
        }
        __syncthreads();
        for (uint32_t q = threadIdx.x; q < jn * 128u; q += 1024u) {
            const uint32_t jj = q >> 7, l = (q >> 1) & 63u, tk = q & 1u;
            float sum = 0.f;
            for (uint32_t v = 0; v < 16u; v++) sum += red[(jj * 16u + v) * 128u + 2u * l + tk];
            uint32_t m, base, bound;
            tile(j0 + jj, m, base, bound);
            const uint32_t row = base + (l & 15u), t = 2u * (l >> 4) + tk;
            const bool st = (RANGED || gt0 + j0 + jj < total) && row < bound && t < a.batch;
            if constexpr (EPI == E_QKV) {
                // the RoPE partner (row ^ 1, same vector) is thread q ^ 2
                const float other = __shfl_xor(sum, 2, 64);
                if (st) {
                    const uint32_t pos = a.pos[t];
                    float v = sum;
                    if (m < 2u && pos < a.max_ctx) {
                        const float2 cs = a.rope[(uint64_t)pos * (a.hd / 2u) + (row % a.hd) / 2u];
                        const bool even = (row & 1u) == 0u;
                        const float x0 = even ? sum : other, x1 = even ? other : sum;
                        v = even ? __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y))
                                 : __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
                    }
                    if (m == 0u)
                        a.y[0][(uint64_t)t * a.ys[0] + row] = v;
                    else if (pos < a.max_ctx)  // (the host bounds every greedy run by max_ctx)
                        (m == 1u ? a.kc : a.vc)[(uint64_t)t * a.kv_seq + a.layer_off + (uint64_t)pos * a.kvd +
                                                row] = vbs_f2h(v);
                }
            } else if (st) {
                float *const y = m == 0u ? a.y[0] : m == 1u ? a.y[1] : a.y[2];
                const uint32_t ys = m == 0u ? a.ys[0] : m == 1u ? a.ys[1] : a.ys[2];
                float *dst = y + (uint64_t)t * ys + row;
                *dst = EPI == E_ACC ? __fadd_rn(*dst, sum) : sum;
            }
        }
        __syncthreads();
    });
}

template <uint32_t NB, uint32_t T, int EPI, bool RANGED = false>
static hipError_t launch_mvbr4_t(const MbArgs &a, uint32_t wgs, hipStream_t s) {
    // a wave's items all in flight when it has at most four (147 KB of LDS),
    // else three slots: four slots made the longer streams slower (70B
    // gate/up 61.6 -> 63.3-66.0 us, Q/K/V 16.8 -> 17.4-17.7 us) while the
    // four-item O launch gained (14.6 -> 14.3 us)
    constexpr uint32_t R = NB * T <= 4u ? NB * T : 3u;
    const size_t lds = Mvbr4Plan<NB, T, R>::lds();
    static bool granted = false;
    if (!granted) {
        if (hipFuncSetAttribute((const void *)k_mvbr4<NB, T, R, EPI, RANGED>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorNotSupported;
        }
        granted = true;
    }
    k_mvbr4<NB, T, R, EPI, RANGED><<<wgs, 1024, lds, s>>>(a);
    return hipGetLastError();
}

// Rows of 16 or 17-32 blocks; tiles per workgroup: the tiles per CU rounded up
// to 1, 2, 3 or 6, or 7 with as many rounds of workgroups as that takes (more
// tiles per workgroup would not fit the registers); w 16-byte aligned, 32-bit
// offsets.
static hipError_t launch_mvbr4(const MbArgs &a, int epi, hipStream_t s) {
    const uint32_t nblk = a.cols / 256u, total = a.tile_end[a.nmat - 1u], cus = device_cus();
    if (a.cols % 256u || nblk == 0u || nblk > 32u) return hipErrorNotSupported;
    for (uint32_t m = 0; m < a.nmat; m++)
        if (((uintptr_t)a.w[m] & 15u) || (uint64_t)a.rows[m] * nblk * 144u + 256u >= (1ull << 32))
            return hipErrorNotSupported;
    // Rows of 17-32 blocks where three tiles per workgroup leave CUs idle
    // (70B Q/K/V: 640 tiles, 214 workgroups): an even range of at most 48
    // rows of one matrix per workgroup (at 70B 42 rows, 246 workgroups)
    if (nblk > 16u) {
        uint32_t rows_all = 0;
        bool even = true;
        for (uint32_t m = 0; m < a.nmat; m++) {
            rows_all += a.rows[m];
            even = even && (a.rows[m] & 1u) == 0u;
        }
        // (ranges of 33-48 rows: the three tiles mostly hold the range's own rows)
        for (uint32_t rpw = ((rows_all + cus - 1u) / cus + 1u) & ~1u; even && rpw > 32u && rpw <= 48u;
             rpw += 2u) {
            MbArgs r = a;
            uint32_t wgs = 0;
            for (uint32_t m = 0; m < 3u; m++) {
                if (m < a.nmat) wgs += (a.rows[m] + rpw - 1u) / rpw;
                r.rwg_end[m] = wgs;
                r.rpw[m] = rpw;
            }
            if (wgs <= cus)
                return epi == E_QKV   ? launch_mvbr4_t<2, 3, E_QKV, true>(r, wgs, s)
                       : epi == E_ACC ? launch_mvbr4_t<2, 3, E_ACC, true>(r, wgs, s)
                                      : launch_mvbr4_t<2, 3, E_STORE, true>(r, wgs, s);
        }
    }
    const uint32_t per = (total + cus - 1u) / cus;
    const uint32_t T = per <= 1u ? 1u : per <= 2u ? 2u : per <= 3u ? 3u : per <= 6u ? 6u : 7u;
    const uint32_t wgs = (total + T - 1u) / T;
#define VBS_MVBR4(NB_, T_)                                                                  \
    return epi == E_QKV   ? launch_mvbr4_t<NB_, T_, E_QKV>(a, wgs, s)                           \
           : epi == E_ACC ? launch_mvbr4_t<NB_, T_, E_ACC>(a, wgs, s)                           \
                          : launch_mvbr4_t<NB_, T_, E_STORE>(a, wgs, s)
    if (nblk <= 16u) {
        if (T == 1u) VBS_MVBR4(1, 1);
        if (T == 2u) VBS_MVBR4(1, 2);
        if (T == 3u) VBS_MVBR4(1, 3);
        if (T == 6u) VBS_MVBR4(1, 6);
        VBS_MVBR4(1, 7);
    }
    if (T == 1u) VBS_MVBR4(2, 1);
    if (T == 2u) VBS_MVBR4(2, 2);
    if (T == 3u) VBS_MVBR4(2, 3);
    if (T == 6u) VBS_MVBR4(2, 6);
    VBS_MVBR4(2, 7);
#undef VBS_MVBR4
}

template <class T, uint32_t TPW, bool ACC>
static hipError_t launch_mvb_t(const MbArgs &a, uint32_t nw, hipStream_t s) {
    const uint32_t tiles = a.tile_end[a.nmat - 1u];
    const size_t lds = (size_t)nw * T::SCRATCH + (size_t)TPW * nw * 128u * sizeof(float);
    k_mvb<T, TPW, ACC><<<(tiles + TPW - 1u) / TPW, 64u * nw, lds, s>>>(a);
    return hipGetLastError();
}

// Tiles per workgroup and waves (measured at batch 8 on the 70B and 7B
// shapes): the A operands of a block serve every tile of a wave, so they are
// shared as widely as the grid still fills the chip. From 1024 tiles of
// rows wider than 16 blocks (70B gate/up) four tiles pair best with four
// waves; otherwise from 640 tiles (70B Q/K/V, the 7B gate and gate/up)
// three tiles and eight waves (Q4_K 10240x8192: 25.7 -> 22.6 us,
// 11008x4096: 16.1 -> 14.4 us, 22016x4096: 27.9 -> 24.4 us against four
// tiles); below that two tiles. Other splits were slower at every shape.
// Q6_K stops at two tiles (four would spill registers).
template <class T, bool ACC>
static hipError_t launch_mvb_plan(const MbArgs &a, hipStream_t s) {
    const uint32_t nblk = a.cols / 256u, tiles = a.tile_end[a.nmat - 1u];
    if constexpr (T::BYTES == 144u) {
        if (tiles >= 1024u && nblk > 16u) return launch_mvb_t<T, 4, ACC>(a, 4u, s);
        if (tiles >= 640u) return launch_mvb_t<T, 3, ACC>(a, min(8u, nblk), s);
        if (tiles >= 256u) return launch_mvb_t<T, 2, ACC>(a, min(8u, nblk), s);
    } else {
        if (tiles >= 512u) return launch_mvb_t<T, 2, ACC>(a, nblk > 64u ? 8u : min(4u, nblk), s);
    }
    return launch_mvb_t<T, 1, ACC>(a, min(8u, nblk), s);
}

// ---- attention merge into the prepared form ------------------------------------------
// The batched decoder's attention merge (head_dim 128, the matrix-core chunk
// kernel's partials) writing O's prepared x directly: workgroup (pair p,
// sequence t) merges q heads 2p and 2p + 1 -- block p of the attention output
// -- as k_attn_merge_h128 does (four waves per head, the same vbs_attn_common.h
// pieces), then one wave prepares the block with xprep_block: the values and
// the prepared bytes equal the merge launch followed by k_xprep_b's.
__global__ __launch_bounds__(512) void k_attn_merge_prep(const float *__restrict__ part,
                                                         uint8_t *__restrict__ xp, uint32_t stride_chunks,
                                                         const uint32_t *__restrict__ pos_dev,
                                                         uint32_t nkh, uint64_t part_bstride,
                                                         uint32_t cols, uint32_t target) {
    __shared__ float2 red[2][kMergeRes][64];
    __shared__ float4 outv[64];
    const uint32_t pb = blockIdx.x, bz = blockIdx.y, lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t hh = wave / kMergeRes, r = wave % kMergeRes, h = 2u * pb + hh;
    part += bz * part_bstride;
    const uint32_t nc = mfma_chunks(pos_dev[bz] + 1u, nkh, target);  // seq = pos + 1
    const float *ph = part + (uint64_t)h * stride_chunks * kPartRow;
    float2 av[kMergeBatch];
    merge_residue_load(ph, nc, r, lane, av);
    const MergeStats st = merge_stats(ph, nc, lane, merge_ml_load(ph, nc, lane));
    red[hh][r][lane] = merge_residue_sum(ph, nc, st, r, lane, av);
    __syncthreads();
    if (r == 0u) {
        float2 a[kMergeRes];
#pragma unroll
        for (uint32_t k = 0; k < kMergeRes; k++) a[k] = red[hh][k][lane];
        reinterpret_cast<float2 *>(outv)[64u * hh + lane] = merge_finish(a, st.L);
    }
    __syncthreads();
    if (wave == 0u) {
        const float4 x = outv[lane];
        const float v[4] = {x.x, x.y, x.z, x.w};
        xprep_block(v, lane, bz, pb, cols, xp);
    }
}

hipError_t launch_attn_merge_prep(const float *part, uint8_t *xp, uint32_t stride_chunks,
                                  const uint32_t *pos_dev, uint32_t nqh, uint32_t nkh,
                                  uint64_t part_bstride, uint32_t batch, hipStream_t s) {
    if (nqh % 2u || batch == 0 || batch > kBatchMax || !pos_dev) return hipErrorNotSupported;
    k_attn_merge_prep<<<dim3(nqh / 2u, batch), 512, 0, s>>>(part, xp, stride_chunks, pos_dev, nkh,
                                                           part_bstride, nqh * 128u,
                                                           attn_batch_target(batch));
    return hipGetLastError();
}

size_t xprep_bytes(uint32_t cols) { return xb_layout(cols).bytes; }

hipError_t launch_xprep(int mode, const float *x, const float *x2, uint32_t xs,
                        const float *norm_w, float eps, uint32_t cols, uint32_t batch, uint8_t *xp,
                        hipStream_t s) {
    if (batch == 0 || batch > kBatchMax || cols % 256u || cols / 256u > 128u) return hipErrorNotSupported;
    const dim3 grid((cols / 256u + 3u) / 4u, batch);
    if (mode == XP_NORM)
        k_xprep_b<XP_NORM><<<grid, 256, 0, s>>>(x, x2, xs, norm_w, eps, cols, xp);
    else if (mode == XP_SILU)
        k_xprep_b<XP_SILU><<<grid, 256, 0, s>>>(x, x2, xs, norm_w, eps, cols, xp);
    else
        k_xprep_b<XP_PLAIN><<<grid, 256, 0, s>>>(x, x2, xs, norm_w, eps, cols, xp);
    return hipGetLastError();
}

hipError_t launch_mvb(int type, uint32_t nmat, const uint8_t *const w[], const uint32_t rows[],
                      float *const y[], const uint32_t ys[], int accumulate, const uint8_t *xp,
                      uint32_t cols, uint32_t batch, hipStream_t s) {
    if (nmat == 0 || nmat > 3u || batch == 0 || batch > kBatchMax) return hipErrorNotSupported;
    MbArgs a{};
    uint32_t tiles = 0;
    for (uint32_t m = 0; m < nmat; m++) {
        // (x is read from the prepared planes; any 4-byte aligned pointer passes the check)
        if (rows[m] == 0 || !mv_fits(type, w[m], reinterpret_cast<const float *>(xp), cols, rows[m]))
            return hipErrorNotSupported;
        a.w[m] = w[m];
        a.y[m] = y[m];
        a.ys[m] = ys[m];
        a.rows[m] = rows[m];
        tiles += (rows[m] + 15u) / 16u;
        a.tile_end[m] = tiles;
    }
    a.nmat = nmat;
    a.xp = xp;
    a.cols = cols;
    a.batch = batch;
    {
        const hipError_t e = type == kQ6_K ? launch_mvbr6(a, accumulate != 0, s)
                                           : launch_mvbr4(a, accumulate ? E_ACC : E_STORE, s);
        if (e != hipErrorNotSupported) return e;
    }
    if (type == kQ4_K)
        return accumulate ? launch_mvb_plan<Q4KB, true>(a, s) : launch_mvb_plan<Q4KB, false>(a, s);
    return accumulate ? launch_mvb_plan<Q6KB, true>(a, s) : launch_mvb_plan<Q6KB, false>(a, s);
}

hipError_t launch_mvb_qkv(int type, const uint8_t *const w[3], const uint32_t rows[3], float *q,
                          uint32_t q_stride, const uint8_t *xp, uint32_t cols, uint32_t batch,
                          const float2 *rope, const uint32_t *pos, uint16_t *kc, uint16_t *vc,
                          uint64_t kv_seq, uint64_t layer_off, uint32_t hd, uint32_t kvd,
                          uint32_t max_ctx, hipStream_t s) {
    if (type != kQ4_K || batch == 0 || batch > kBatchMax || hd == 0u || (hd & 1u))
        return hipErrorNotSupported;
    MbArgs a{};
    uint32_t tiles = 0;
    for (uint32_t m = 0; m < 3u; m++) {
        if (rows[m] == 0 || rows[m] % 16u ||
            !mv_fits(type, w[m], reinterpret_cast<const float *>(xp), cols, rows[m]))
            return hipErrorNotSupported;
        a.w[m] = w[m];
        a.rows[m] = rows[m];
        tiles += rows[m] / 16u;
        a.tile_end[m] = tiles;
    }
    a.y[0] = q;
    a.ys[0] = q_stride;
    a.nmat = 3;
    a.xp = xp;
    a.cols = cols;
    a.batch = batch;
    a.rope = rope;
    a.pos = pos;
    a.kc = kc;
    a.vc = vc;
    a.kv_seq = kv_seq;
    a.layer_off = layer_off;
    a.hd = hd;
    a.kvd = kvd;
    a.max_ctx = max_ctx;
    return launch_mvbr4(a, E_QKV, s);
}

hipError_t launch_kq_linear_batch(int type, const uint8_t *w, const float *x, uint32_t xs, float *y,
                                  uint32_t ys, uint32_t cols, uint32_t rows, uint32_t batch,
                                  hipStream_t s) {
    if (batch == 0 || batch > kBatchMax || rows == 0 || !mv_fits(type, w, x, cols, rows))
        return hipErrorNotSupported;
    hipError_t why;
    uint8_t *xp = static_cast<uint8_t *>(rt_scratch(xb_layout(cols).bytes, s, &why));
    if (!xp) return why;
    hipError_t e = launch_xprep(XP_PLAIN, x, nullptr, xs, nullptr, 0.f, cols, batch, xp, s);
    if (e != hipSuccess) return e;
    const uint8_t *wm[1] = {w};
    float *ym[1] = {y};
    const uint32_t rm[1] = {rows}, ysm[1] = {ys};
    return launch_mvb(type, 1, wm, rm, ym, ysm, 0, xp, cols, batch, s);
}

hipError_t launch_linear_batch_multi(int type, uint32_t n_mat, const uint8_t *const w[],
                                     const uint32_t rows[], const float *x, uint32_t xs,
                                     float *const y[], const uint32_t ys[], uint32_t cols,
                                     uint32_t batch, hipStream_t s) {
    if (n_mat == 0 || n_mat > 3u) return hipErrorInvalidValue;
    if (batch == 0) return hipSuccess;
    bool mfma = type == kQ4_K || type == kQ6_K;
    for (uint32_t m = 0; m < n_mat && mfma; m++)
        mfma = rows[m] != 0 && mv_fits(type, w[m], x, cols, rows[m]);
    if (!mfma) {
        for (uint32_t m = 0; m < n_mat; m++) {
            const hipError_t e = launch_linear_batch(type, w[m], x, xs, y[m], ys[m], cols, rows[m],
                                                     batch, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    hipError_t why;
    uint8_t *xp = static_cast<uint8_t *>(rt_scratch(xb_layout(cols).bytes, s, &why));
    if (!xp) return why;
    for (uint32_t b0 = 0; b0 < batch; b0 += kBatchMax) {
        const uint32_t nb = min(kBatchMax, batch - b0);
        hipError_t e = launch_xprep(XP_PLAIN, x + (uint64_t)b0 * xs, nullptr, xs, nullptr, 0.f, cols,
                                    nb, xp, s);
        if (e != hipSuccess) return e;
        float *yb[3];
        for (uint32_t m = 0; m < n_mat; m++) yb[m] = y[m] + (uint64_t)b0 * ys[m];
        e = launch_mvb(type, n_mat, w, rows, yb, ys, 0, xp, cols, nb, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace vbs
