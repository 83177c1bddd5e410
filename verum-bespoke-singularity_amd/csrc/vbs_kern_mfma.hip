// vbs_kern_mfma.hip — launchers of the batch-1 matrix-core matvec (k_mvf,
// vbs_mfma.h) for Q4_K and Q6_K: plain and accumulating matvecs, the RMSNorm
// prologue, and the fused Q/K/V + RoPE + KV store and gate/up + SiLU launches
// of the graph decoder. The 32-element block types are launched from
// vbs_kern_mfma_blk.hip, the batched kernels live in vbs_kern_mfma_batch.hip.
#include "vbs_mfma.h"

namespace vbs {

template <bool NORM, int EPI>
static hipError_t launch_type(int type, const MvArgs &a, hipStream_t s) {
    return type == kQ4_K ? launch_plan<Q4K, NORM, EPI>(a, s) : launch_plan<Q6K, NORM, EPI>(a, s);
}

hipError_t launch_kq_linear(int type, const uint8_t *w, const float *x, float *y, uint32_t cols,
                            uint32_t rows, int accumulate, hipStream_t s) {
    if (rows == 0) return hipErrorNotSupported;
    if (mv_fits_blk(type, w, x, cols, rows))
        return launch_blk_linear(type, w, x, y, cols, rows, accumulate, s);
    if (!mv_fits(type, w, x, cols, rows)) return hipErrorNotSupported;
    {
        const hipError_t e = type == kQ4_K ? launch_q4k_mvl(w, x, y, cols, rows, accumulate, s)
                                           : launch_q6k_mvr(w, x, y, cols, rows, accumulate, s);
        if (e != hipErrorNotSupported) return e;
    }
    MvArgs a{};
    a.w[0] = w;
    a.y[0] = y;
    a.rows[0] = rows;
    a.nmat = 1;
    a.cols = cols;
    a.x = x;
    set_tiles(a);
    return accumulate ? launch_type<false, E_ACC>(type, a, s) : launch_type<false, E_STORE>(type, a, s);
}

hipError_t launch_kq_norm_linear(int type, const uint8_t *w, const float *x, const float *norm_w,
                                 float eps, float *y, uint32_t cols, uint32_t rows,
                                 hipStream_t s) {
    if (rows == 0 || !mv_fits(type, w, x, cols, rows)) return hipErrorNotSupported;
    MvArgs a{};
    a.w[0] = w;
    a.y[0] = y;
    a.rows[0] = rows;
    a.nmat = 1;
    a.cols = cols;
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    set_tiles(a);
    return launch_type<true, E_STORE>(type, a, s);
}

hipError_t launch_kq_linear_fused(int type, const uint8_t *w, const float *x, float *y, uint32_t cols,
                                  uint32_t rows, const LinJoin &j, hipStream_t s) {
    if (rows == 0 || !mv_fits(type, w, x, cols, rows)) return hipErrorNotSupported;
    const bool store_join = j.hid || j.kin;
    const int n_after = (j.ycopy != nullptr) + (j.rope != nullptr) + (int)store_join;
    if (n_after > 1 || (j.hid && j.kin) || (j.norm_w && (j.ycopy || store_join)) ||
        (!j.norm_w && !n_after))
        return hipErrorNotSupported;
    MvArgs a{};
    a.w[0] = w;
    a.y[0] = y;
    a.rows[0] = rows;
    a.nmat = 1;
    a.cols = cols;
    a.x = x;
    a.norm_w = j.norm_w;
    a.eps = j.eps;
    a.xn = j.xn;
    if (j.rope) {  // the q path of E_QKV: the row value rotated at *pos, stored as f32
        if ((rows & 1u) || (j.hd & 1u) || !j.hd || rows % j.hd) return hipErrorNotSupported;
        a.rope = j.rope;
        a.pos = j.pos;
        a.hd = j.hd;
        a.role0 = 0;
        if (type == kQ4_K) {
            const hipError_t e = launch_q4k_mvl_qkv(a, s);
            if (e != hipErrorNotSupported) return e;
        }
        set_tiles(a);
        return a.norm_w ? launch_type<true, E_QKV>(type, a, s) : launch_type<false, E_QKV>(type, a, s);
    }
    a.gate_in = j.gate_in;
    a.hid = j.hid;
    a.kin = j.kin;
    a.kc = j.kc;
    a.vc = j.vc;
    a.kv_layer = j.kv_off;
    if (j.norm_w || store_join) {  // E_STORE with the RMSNorm in front or a store join after
        if (type == kQ4_K) {
            const hipError_t e = launch_q4k_mvl(w, x, y, cols, rows, 0, s, &a);
            if (e != hipErrorNotSupported) return e;
        }
        set_tiles(a);
        return j.norm_w ? launch_type<true, E_STORE>(type, a, s) : launch_type<false, E_STORE>(type, a, s);
    }
    a.ycopy = j.ycopy;
    {
        const hipError_t e = type == kQ4_K ? launch_q4k_mvl(w, x, y, cols, rows, 1, s, &a)
                                           : launch_q6k_mvr(w, x, y, cols, rows, 1, s, j.ycopy);
        if (e != hipErrorNotSupported) return e;
    }
    set_tiles(a);
    return launch_type<false, E_ACC>(type, a, s);
}

hipError_t launch_kq_qkv(int type, const uint8_t *const wqkv[3], uint32_t n_mat, uint32_t role0,
                         const float *x, const float *norm_w, float eps, uint32_t cols,
                         const uint32_t rows[3], float *q, uint16_t *kc, uint16_t *vc,
                         uint64_t kv_layer, uint32_t kvd, const float2 *rope,
                         const uint32_t *pos, uint32_t hd, hipStream_t s, const GroupOut &out) {
    if (n_mat == 0 || n_mat > 3u || role0 + n_mat > 3u || (hd & 1u)) return hipErrorNotSupported;
    MvArgs a{};
    for (uint32_t m = 0; m < n_mat; m++) {
        if (!mv_fits(type, wqkv[m], x, cols, rows[m]) || rows[m] == 0 || (n_mat > 1u && rows[m] % 16u))
            return hipErrorNotSupported;
        a.w[m] = wqkv[m];
        a.rows[m] = rows[m];
    }
    a.y[0] = q;
    a.nmat = n_mat;
    a.role0 = role0;
    a.cols = cols;
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.rope = rope;
    a.pos = pos;
    a.hd = hd;
    a.kvd = kvd;
    a.kc = kc;
    a.vc = vc;
    a.kv_layer = kv_layer;
    a.xn = out.xn;
    a.kout = out.k;
    a.vout = out.v;
    if (type == kQ4_K) {
        const hipError_t e = launch_q4k_mvl_qkv(a, s);
        if (e != hipErrorNotSupported) return e;
    }
    set_tiles(a);
    return norm_w ? launch_type<true, E_QKV>(type, a, s) : launch_type<false, E_QKV>(type, a, s);
}

hipError_t launch_kq_silu(int type, const uint8_t *wg, const uint8_t *wu, const float *x,
                          const float *norm_w, float eps, uint32_t cols, uint32_t rows,
                          float *hid, hipStream_t s, const GroupOut &out) {
    if (rows == 0 || rows % 16u || !mv_fits(type, wg, x, cols, rows) || !mv_fits(type, wu, x, cols, rows))
        return hipErrorNotSupported;
    MvArgs a{};
    a.w[0] = wg;
    a.w[1] = wu;
    a.y[0] = hid;
    a.rows[0] = a.rows[1] = rows;
    a.nmat = 2;
    a.cols = cols;
    a.x = x;
    a.norm_w = norm_w;
    a.eps = eps;
    a.xn = out.xn;
    a.gout = out.gate;
    a.uout = out.up;
    set_tiles(a);
    return norm_w ? launch_type<true, E_SILU>(type, a, s) : launch_type<false, E_SILU>(type, a, s);
}


}  // namespace vbs
