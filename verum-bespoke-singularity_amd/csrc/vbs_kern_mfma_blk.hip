// vbs_kern_mfma_blk.hip — the batch-1 matrix-core matvec (k_mvf, vbs_mfma.h)
// for the 32-element block types Q4_0, Q4_1 and Q8_0 (plain and accumulating
// launches), in a translation unit of its own so it compiles in parallel.
#include "vbs_mfma.h"

namespace vbs {

hipError_t launch_blk_linear(int type, const uint8_t *w, const float *x, float *y, uint32_t cols,
                             uint32_t rows, int accumulate, hipStream_t s) {
    if (rows == 0 || !mv_fits_blk(type, w, x, cols, rows)) return hipErrorNotSupported;
    MvArgs a{};
    a.w[0] = w;
    a.y[0] = y;
    a.rows[0] = rows;
    a.nmat = 1;
    a.cols = cols;
    a.x = x;
    set_tiles(a);
    if (type == kQ4_0)
        return accumulate ? launch_plan<Q40, false, E_ACC>(a, s) : launch_plan<Q40, false, E_STORE>(a, s);
    if (type == kQ4_1)
        return accumulate ? launch_plan<Q41, false, E_ACC>(a, s) : launch_plan<Q41, false, E_STORE>(a, s);
    return accumulate ? launch_plan<Q80, false, E_ACC>(a, s) : launch_plan<Q80, false, E_STORE>(a, s);
}

}  // namespace vbs
