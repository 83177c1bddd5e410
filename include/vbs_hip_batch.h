/* vbs_hip_batch.h — versioned batched-linear extension of the gfx950 HIP
 * backend shim (libvbs_backend_gfx950.so).
 *
 * vbs_backend_ops_t has no batched matvec: the reference's token loop runs one
 * token at a time (src/vbs_specializer.c:353-357), and dispatch_linear_tile
 * (include/vbs_backend.h:80-84) takes one x. This extension is the batched
 * counterpart of that slot for callers that decode several sequences over
 * one copy of the weights: no counterpart in the reference; its oracle is
 * `batch` independent vbs_host_linear_tile calls (src/vbs_host_math.h:223-267).
 *
 * Callers find it with dlsym on the backend library and check
 * vbs_hip_linear_batch_version() before use.
 */
#ifndef VBS_GFX950_HIP_BATCH_H
#define VBS_GFX950_HIP_BATCH_H

#include "vbs_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

#define VBS_HIP_LINEAR_BATCH_VERSION 1u

uint32_t vbs_hip_linear_batch_version(void);

/* Y[b * y_stride + r] = sum_c deq(W[r, c]) * X[b * x_stride + c] for r < rows,
 * b < batch (1..16), with the weights resident (convention A: w's
 * internal_handle holds the packed tensor) and the pipeline from
 * compile_linear_pipeline. The weights are read once for all vectors; each
 * vector's result equals a dispatch_linear_tile of that vector to the
 * linear's tolerance. Returns false with the reason in vbs_hip_last_error()
 * on a bad argument or device failure; nothing is launched then. */
bool vbs_hip_dispatch_linear_batch(vbs_device_t *dev, void *pipeline, vbs_buffer_t *w,
                                   vbs_buffer_t *x, uint32_t x_stride, vbs_buffer_t *y,
                                   uint32_t y_stride, uint32_t cols, uint32_t rows,
                                   uint32_t batch);

#ifdef __cplusplus
}
#endif

#endif
