// vbs_internal.h — launchers shared between the runtime (vbs_gfx950_rt.hip)
// and the kernel translation units. Every launcher enqueues on `s` and
// returns hipSuccess or the launch error; argument validation is done by the
// C-ABI entry points before any launcher runs.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vbs {

// Row stride in bytes of a packed row of `cols` elements (src/vbs_gguf.c:12-40).
uint64_t row_bytes(int type, uint32_t cols);
// Elements per block of `type`, 0 if not a hot-path type.
uint32_t block_elems(int type);

// Device scratch owned by the runtime, at least `bytes` long. It only grows;
// a replaced buffer stays allocated until the process ends, so graphs
// captured with it stay valid. NULL with *why set when it cannot grow:
// hipErrorStreamCaptureUnsupported while `s` is being captured (growing
// allocates), hipErrorOutOfMemory otherwise.
void *rt_scratch(size_t bytes, hipStream_t s, hipError_t *why);

// The library's stream, and the last-error writer of the C ABI.
hipStream_t rt_stream();
int rt_fail(const char *fmt, ...);
int rt_hip_ok(hipError_t e, const char *what);
bool rt_ready();

// Q4_K / Q6_K matvecs on the matrix cores (x is prepared inside the kernel);
// launch_kq_linear also takes Q4_0 / Q4_1 / Q8_0 (eight blocks per unit of
// 256 columns); hipErrorNotSupported outside their shape/alignment range.
hipError_t launch_kq_linear(int type, const uint8_t *w, const float *x, float *y, uint32_t cols,
                            uint32_t rows, int accumulate, hipStream_t s);
// The Q4_0 / Q4_1 / Q8_0 part of launch_kq_linear.
hipError_t launch_blk_linear(int type, const uint8_t *w, const float *x, float *y, uint32_t cols,
                             uint32_t rows, int accumulate, hipStream_t s);
// y = W * rms_norm(x, norm_w) (the norm as k_rms_norm computes it).
hipError_t launch_kq_norm_linear(int type, const uint8_t *w, const float *x, const float *norm_w,
                                 float eps, float *y, uint32_t cols, uint32_t rows,
                                 hipStream_t s);
// The f32 vectors a grouped launch also stores, for the backend shim's
// grouped ops (each may be NULL): the normalised x, and the rows of the
// first (q; gate) and second and third (k roped, v; up) matrices.
struct GroupOut {
    float *xn = nullptr, *k = nullptr, *v = nullptr, *gate = nullptr, *up = nullptr;
};
// Matrices q, k, v (roles role0 .. role0 + n_mat - 1, same type and cols) of
// rms_norm(x) in one launch (norm_w may be NULL): q roped into `q`, k roped
// and v stored as f16 at position *pos of the caches (offset kv_layer).
hipError_t launch_kq_qkv(int type, const uint8_t *const w[3], uint32_t n_mat, uint32_t role0,
                         const float *x, const float *norm_w, float eps, uint32_t cols,
                         const uint32_t rows[3], float *q, uint16_t *kc, uint16_t *vc,
                         uint64_t kv_layer, uint32_t kvd, const float2 *rope,
                         const uint32_t *pos, uint32_t hd, hipStream_t s,
                         const GroupOut &out = GroupOut{});
// hid = silu(Wg * rms_norm(x)) * (Wu * rms_norm(x)) in one launch.
hipError_t launch_kq_silu(int type, const uint8_t *wg, const uint8_t *wu, const float *x,
                          const float *norm_w, float eps, uint32_t cols, uint32_t rows,
                          float *hid, hipStream_t s, const GroupOut &out = GroupOut{});

// Batched matrix-core matvecs in two steps: x of up to 8 vectors prepared
// once (XP_PLAIN: x; XP_NORM: rms_norm(x) * norm_w; XP_SILU: silu(x) * x2,
// all at row stride xs) into xprep_bytes(cols) of device memory, then
// launch_mvb for 1-3 matrices of one K-quant type over it (y = W x, or
// y += W x with `accumulate`); hipErrorNotSupported (nothing launched)
// outside the matrix-core shape range.
enum : int { XP_PLAIN = 0, XP_NORM = 1, XP_SILU = 2 };
size_t xprep_bytes(uint32_t cols);
hipError_t launch_xprep(int mode, const float *x, const float *x2, uint32_t xs,
                        const float *norm_w, float eps, uint32_t cols, uint32_t batch, uint8_t *xp,
                        hipStream_t s);
hipError_t launch_mvb(int type, uint32_t nmat, const uint8_t *const w[], const uint32_t rows[],
                      float *const y[], const uint32_t ys[], int accumulate, const uint8_t *xp,
                      uint32_t cols, uint32_t batch, hipStream_t s);
// The head_dim-128 merge of the batched attention partials (chunk stride
// attn_max_chunks(max_seq, nkh), part_bstride floats per sequence, the split
// of attn_batch_target(batch) that launch_attention_batch used) written as
// O's prepared x (xprep layout, nqh x 128 columns), pairs of q heads per block.
hipError_t launch_attn_merge_prep(const float *part, uint8_t *xp, uint32_t stride_chunks,
                                  const uint32_t *pos_dev, uint32_t nqh, uint32_t nkh,
                                  uint64_t part_bstride, uint32_t batch, hipStream_t s);
uint32_t attention_chunk_stride(uint32_t max_seq, uint32_t nkh);
// The batched decoder's Q/K/V launch with the RoPE and the f16 cache store of
// every sequence in its epilogue (q, k, v of Q4_K, rows of 16-row multiples, at
// most 32 blocks; hipErrorNotSupported otherwise): q rows to q + t q_stride,
// k and v rows to kc / vc + t kv_seq + layer_off + pos[t] kvd.
hipError_t launch_mvb_qkv(int type, const uint8_t *const w[3], const uint32_t rows[3], float *q,
                          uint32_t q_stride, const uint8_t *xp, uint32_t cols, uint32_t batch,
                          const float2 *rope, const uint32_t *pos, uint16_t *kc, uint16_t *vc,
                          uint64_t kv_seq, uint64_t layer_off, uint32_t hd, uint32_t kvd,
                          uint32_t max_ctx, hipStream_t s);
// Y[t] = W * X[t] for t < batch <= 8 (Q4_K / Q6_K) on the f16 matrix cores,
// W read once; x prepared into the runtime scratch first. hipErrorNotSupported
// (before anything is launched) outside the matrix-core shape range.
hipError_t launch_kq_linear_batch(int type, const uint8_t *w, const float *x, uint32_t xs, float *y,
                                  uint32_t ys, uint32_t cols, uint32_t rows, uint32_t batch,
                                  hipStream_t s);

struct MvArgs;
// Q4_K matvec with each workgroup's whole row range in flight (rows of 16
// blocks, 4096-12288 rows, 16-byte aligned w and x); hipErrorNotSupported
// outside that range (k_mvf then runs). Bit-identical to k_mvf. `extra`
// (may be NULL) brings the backend shim's fused neighbours: norm_w / eps /
// xn for an RMSNorm in front (not with accumulate), ycopy with accumulate.
hipError_t launch_q4k_mvl(const uint8_t *w, const float *x, float *y, uint32_t cols, uint32_t rows,
                          int accumulate, hipStream_t s, const MvArgs *extra = nullptr);
// The ring variant (vbs_kern_mvl.hip) for Q6_K rows of 33-48 blocks over
// 2049-4096 rows (7B down) and of 97-112 blocks over 4097-8192 rows (70B
// down); hipErrorNotSupported elsewhere. ycopy (accumulate only, may be
// NULL) also receives each row value before it is added.
hipError_t launch_q6k_mvr(const uint8_t *w, const float *x, float *y, uint32_t cols, uint32_t rows,
                          int accumulate, hipStream_t s, float *ycopy = nullptr);
// A decode step's O projection with the attention merge in front, in one
// launch (k_mvl_attn, vbs_kern_mvl.hip): y += W attn, W Q4_K of rows of 16
// blocks (cols = 4096 = nqh x 128), attn the head_dim-128 merge of the
// partials launch_attention_chunks wrote (stride_chunks per q head, the
// sequence length pos[0] + 1 read on the device), bit-identical to
// launch_attention's merge followed by launch_q4k_mvl. 8 nqh workgroups of
// rpw <= 16 rows. The heads travel between the workgroups of an XCD through
// mbuf ([8][cols] floats) and mflag (attn_o_flag_words(cols) words, cleared
// by the chunk launch before it); spin bounds each workgroup's wait for them,
// after which it merges every head itself (fallbacks, if not NULL, counts
// those workgroups). attn, if not NULL, also receives the merged vector.
constexpr uint32_t kAttnOXcds = 8;
struct AttnOArgs {
    const uint8_t *w;
    float *y;
    uint32_t rows, cols, rpw;
    const float *part;
    uint32_t stride_chunks, nkh;
    const uint32_t *pos;
    float *attn, *mbuf;
    uint32_t *mflag;
    uint32_t spin;
    uint32_t *fallbacks;
};
// One flag per (XCD, head), each on a 128-byte line of its own (polls of one
// line by many workgroups' atomics would queue behind each other in the L2).
constexpr uint32_t kAttnOFlagStride = 32;
inline uint32_t attn_o_flags(uint32_t cols) { return kAttnOXcds * (cols / 128u); }
inline uint32_t attn_o_flag_words(uint32_t cols) { return attn_o_flags(cols) * kAttnOFlagStride; }
size_t attn_o_exchange_bytes(uint32_t cols);
hipError_t launch_q4k_mvl_attn(const AttnOArgs &a, hipStream_t s);
// The linear op fused with its neighbours in the bridge's op sequence (the
// backend shim's dispatch path, vbs_gfx950_linear_fused): norm_w / eps / xn
// (RMSNorm in front, the normalised x stored to xn), ycopy (y = y + W x, W x
// also stored to ycopy), rope / pos / hd (the result rotated at the device
// position *pos, as the ROTARY op after it), gate_in / hid (hid =
// silu(gate_in) * W x, the ACTIVATION op after the up matvec), kin / kc / vc
// / kv_off (the CACHE op after the V matvec: f16(W x) to vc and f16(kin) to
// kc at kv_off). Q4_K and Q6_K only; hipErrorNotSupported (nothing launched)
// outside the combinations and shapes the fused kernels take.
struct LinJoin {
    const float *norm_w = nullptr;
    float eps = 0.f;
    float *xn = nullptr, *ycopy = nullptr;
    const float2 *rope = nullptr;
    const uint32_t *pos = nullptr;
    uint32_t hd = 0;
    const float *gate_in = nullptr, *kin = nullptr;
    float *hid = nullptr;
    uint16_t *kc = nullptr, *vc = nullptr;
    uint64_t kv_off = 0;
};
hipError_t launch_kq_linear_fused(int type, const uint8_t *w, const float *x, float *y, uint32_t cols,
                                  uint32_t rows, const LinJoin &j, hipStream_t s);
// Specialised Q4_K matvec; hipErrorNotSupported when the shape/alignment is
// outside its range (the generic kernel then runs).
hipError_t launch_q4k_fast(const uint8_t *w, const float *x, float *y, uint32_t cols,
                           uint32_t rows, int accumulate, hipStream_t s);

hipError_t launch_linear(int type, const uint8_t *w, const float *x, float *y, uint32_t cols,
                         uint32_t rows, int accumulate, hipStream_t s);
hipError_t launch_linear_batch(int type, const uint8_t *w, const float *x, uint32_t x_stride,
                               float *y, uint32_t y_stride, uint32_t cols, uint32_t rows,
                               uint32_t batch, hipStream_t s);
// n_mat (<= 3) matrices of one type over the same vectors: x prepared once per
// eight vectors and one matrix-core launch for Q4_K / Q6_K, else n_mat
// launch_linear_batch calls.
hipError_t launch_linear_batch_multi(int type, uint32_t n_mat, const uint8_t *const w[],
                                     const uint32_t rows[], const float *x, uint32_t xs,
                                     float *const y[], const uint32_t ys[], uint32_t cols,
                                     uint32_t batch, hipStream_t s);
hipError_t launch_dequant_rows(int type, const uint8_t *w, const uint32_t *ids, uint32_t token,
                               uint32_t n_rows, uint32_t dim, float *out, hipStream_t s);
hipError_t launch_rms_norm(const float *in, const float *w, float *out, uint32_t n, float eps,
                           hipStream_t s);
hipError_t launch_rope(float *x, uint32_t head_dim, uint32_t n_heads, const float *cs,
                       hipStream_t s);
hipError_t launch_cache_store(const float *k, const float *v, uint16_t *kc, uint16_t *vc,
                              uint64_t base, uint32_t kv_dim, hipStream_t s);
// Split-sequence attention. With pos_dev the sequence length is read on the
// device (pos + 1) and seq_len only sizes the grid; `part` may be NULL (then
// the runtime scratch holds the per-chunk partials).
size_t attention_partial_bytes(uint32_t max_seq, uint32_t nqh, uint32_t nkh, uint32_t hd);
hipError_t launch_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                            uint32_t seq_len, const uint32_t *pos_dev, float *part,
                            uint64_t layer_off, uint32_t nqh, uint32_t nkh, uint32_t hd,
                            float scale, hipStream_t s);
// Its matrix-core chunk launch alone (head_dim 128, group <= 8, 16-byte
// aligned q and caches; hipErrorNotSupported otherwise), the partials in
// `part` (attention_chunk_stride(seq_len, nkh) chunks per q head) for a merge
// by the launch after it (launch_q4k_mvl_attn), the words clear[i stride]
// for i < nclear zeroed for that launch.
hipError_t launch_attention_chunks(const float *q, const uint16_t *kc, const uint16_t *vc,
                                   uint32_t seq_len, const uint32_t *pos_dev, float *part,
                                   uint64_t layer_off, uint32_t nqh, uint32_t nkh, uint32_t hd,
                                   float scale, uint32_t *clear, uint32_t nclear, uint32_t stride,
                                   hipStream_t s);
// The same for `batch` sequences with their own caches and positions:
// sequence b reads q + b q_stride, writes out + b q_stride, uses the caches at
// + b kv_stride elements, the position pos_dev[b] and the partials at
// part + b * attention_partial_bytes(max_seq, ...) bytes. With out NULL only the
// matrix-core chunk launch runs (attn_mfma_batch_fits; hipErrorNotSupported
// otherwise) and the caller merges the partials (launch_attn_merge_prep).
bool attn_mfma_batch_fits(const float *q, const uint16_t *kc, const uint16_t *vc, uint32_t nqh,
                          uint32_t nkh, uint32_t hd, uint32_t q_stride, uint64_t kv_stride);
hipError_t launch_attention_batch(const float *q, const uint16_t *kc, const uint16_t *vc,
                                  float *out, uint32_t max_seq, const uint32_t *pos_dev,
                                  float *part, uint64_t layer_off, uint32_t nqh, uint32_t nkh,
                                  uint32_t hd, float scale, uint32_t batch, uint32_t q_stride,
                                  uint64_t kv_stride, hipStream_t s);
hipError_t launch_silu_mul(const float *g, const float *u, float *out, uint32_t n,
                           hipStream_t s);
// XOR of the 32-bit words of p[0, bytes) (bytes a multiple of 16, p 16-byte
// aligned) as checksum_partials(bytes) partial words: 16 per workgroup, one per
// wave, each the XOR of that wave's interleaved 1 KB runs of the workgroup's
// span. `variant` selects the shape (0 the default; 1 two 8-wave workgroups
// per CU, 8 partials each; 2 register loads instead of LDS DMA).
uint32_t checksum_partials(uint64_t bytes, int variant = 0);
hipError_t launch_checksum(const uint8_t *p, uint64_t bytes, uint32_t *partials, int variant,
                           hipStream_t s);
hipError_t launch_add(const float *a, const float *b, float *out, uint32_t n, hipStream_t s);

}  // namespace vbs
