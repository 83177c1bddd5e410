/* vbs_hot_abi.h — binary-compatible restatement of the reference's CPU
 * hot-kernel module ABI, version 1, and the two exports a module provides.
 *
 *   VBS_HOT_ABI_VERSION, vbs_hot_kernels_t   include/vbs_hotpath.h:36-57
 *   vbs_hot_abi_version, vbs_hot_kernels     src/hotkernels/vbs_hot_ref.c:11-12,
 *                                            looked up by vbs_hot_load
 *                                            (src/vbs_hotpath.c:78-109)
 *
 * lib/libvbs_hot_gfx950.so is such a module: the five matvecs of the table run
 * on the gfx950 device library, bit-identical to the reference's built-in
 * kernels. Define VBS_ABI_USE_REFERENCE_HEADERS to take the table type from
 * the reference's own vbs_hotpath.h instead.
 */
#ifndef VBS_GFX950_HOT_ABI_H
#define VBS_GFX950_HOT_ABI_H

#ifdef VBS_ABI_USE_REFERENCE_HEADERS
#include "vbs_hotpath.h"
#else

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VBS_HOT_ABI_VERSION 1

typedef struct {
    uint32_t abi_version;
    const char *name;
    void (*matvec_q8_0)(const uint8_t *w, size_t rows, size_t cols, const int8_t *xq,
                        const float *qd, float *y);
    void (*matvec_q4_0)(const uint8_t *w, size_t rows, size_t cols, const int8_t *xq,
                        const float *qd, float *y);
    void (*matvec_q4_1)(const uint8_t *w, size_t rows, size_t cols, const int8_t *xq,
                        const float *qd, const float *qsum, float *y);
    void (*matvec_f32)(const float *w, size_t rows, size_t cols, const float *x, float *y);
    void (*matvec_f16)(const uint16_t *w, size_t rows, size_t cols, const float *x, float *y);
} vbs_hot_kernels_t;

#ifdef __cplusplus
}
#endif
#endif /* VBS_ABI_USE_REFERENCE_HEADERS */

#ifdef __cplusplus
extern "C" {
#endif

/* Module exports (replace src/hotkernels/vbs_hot_ref.c:11-12). */
uint32_t vbs_hot_abi_version(void);
const vbs_hot_kernels_t *vbs_hot_kernels(void);

/* Why the last call failed ("ok" after a successful one). The table's
 * functions return nothing, so a failed call (no device, out of device
 * memory, a HIP error) fills y with NaN and leaves its reason here. No
 * counterpart in the reference: its kernels cannot fail. */
const char *vbs_hot_gfx950_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
