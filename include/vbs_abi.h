/* vbs_abi.h — binary-compatible restatement of the Verum backend boundary.
 *
 * The gfx950 backend is a drop-in for the reference's HIP backend, so every
 * type that crosses the boundary must have the reference's exact layout and
 * enumerator values. This header restates only those types; it is written
 * for this build and carries no code from the reference.
 *
 *   vbs_ggml_type_t       include/vbs_gguf.h:13-48   (GGUF tensor type ids)
 *   vbs_block_geometry_t  include/vbs_gguf.h:50-53
 *   vbs_op_kind_t         include/vbs_graph.h:11-23
 *   vbs_backend_type_t    include/vbs_backend.h:13-19
 *   vbs_device_t          include/vbs_backend.h:24-30
 *   vbs_buffer_t          include/vbs_backend.h:32-37
 *   vbs_arg_t             include/vbs_backend.h:48-54
 *   vbs_prim_pipeline_t   include/vbs_backend.h:59-62
 *   vbs_backend_ops_t     include/vbs_backend.h:64-99
 *
 * When the shim is linked into the reference tree, the reference's own
 * headers provide these definitions and this file is not included (the
 * include guard names differ, so define VBS_ABI_USE_REFERENCE_HEADERS to
 * pull the reference headers instead).
 */
#ifndef VBS_GFX950_ABI_H
#define VBS_GFX950_ABI_H

#ifdef VBS_ABI_USE_REFERENCE_HEADERS
#include "vbs_backend.h"
#include "vbs_backend_select.h"
#else

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    VBS_GGML_TYPE_F32 = 0,
    VBS_GGML_TYPE_F16 = 1,
    VBS_GGML_TYPE_Q4_0 = 2,
    VBS_GGML_TYPE_Q4_1 = 3,
    VBS_GGML_TYPE_Q5_0 = 6,
    VBS_GGML_TYPE_Q5_1 = 7,
    VBS_GGML_TYPE_Q8_0 = 8,
    VBS_GGML_TYPE_Q8_1 = 9,
    VBS_GGML_TYPE_Q2_K = 10,
    VBS_GGML_TYPE_Q3_K = 11,
    VBS_GGML_TYPE_Q4_K = 12,
    VBS_GGML_TYPE_Q5_K = 13,
    VBS_GGML_TYPE_Q6_K = 14,
    VBS_GGML_TYPE_Q8_K = 15,
    VBS_GGML_TYPE_IQ2_XXS = 16,
    VBS_GGML_TYPE_IQ2_XS = 17,
    VBS_GGML_TYPE_IQ3_XXS = 18,
    VBS_GGML_TYPE_IQ1_S = 19,
    VBS_GGML_TYPE_IQ4_NL = 20,
    VBS_GGML_TYPE_IQ3_S = 21,
    VBS_GGML_TYPE_IQ2_S = 22,
    VBS_GGML_TYPE_IQ4_XS = 23,
    VBS_GGML_TYPE_I8 = 24,
    VBS_GGML_TYPE_I16 = 25,
    VBS_GGML_TYPE_I32 = 26,
    VBS_GGML_TYPE_I64 = 27,
    VBS_GGML_TYPE_F64 = 28,
    VBS_GGML_TYPE_IQ1_M = 29,
    VBS_GGML_TYPE_BF16 = 30,
    VBS_GGML_TYPE_TQ1_0 = 34,
    VBS_GGML_TYPE_TQ2_0 = 35,
    VBS_GGML_TYPE_MXFP4 = 39,
    VBS_GGML_TYPE_LNS8 = 40,
    VBS_GGML_TYPE_I8G = 100
} vbs_ggml_type_t;

typedef struct {
    uint32_t elements_per_block;
    uint32_t bytes_per_block;
} vbs_block_geometry_t;

typedef enum {
    VBS_OP_EMBEDDING,
    VBS_OP_LINEAR,
    VBS_OP_NORMALIZE,
    VBS_OP_ATTENTION,
    VBS_OP_ROTARY,
    VBS_OP_ACTIVATION,
    VBS_OP_ELEMENTWISE,
    VBS_OP_STATE_SPACE,
    VBS_OP_CONVOLUTION,
    VBS_OP_CACHE,
    VBS_OP_PROJECTION
} vbs_op_kind_t;

typedef enum {
    VBS_BACKEND_METAL,
    VBS_BACKEND_CUDA,
    VBS_BACKEND_HIP,
    VBS_BACKEND_CPU,
    VBS_BACKEND_VULKAN
} vbs_backend_type_t;

typedef struct vbs_device vbs_device_t;
typedef struct vbs_buffer vbs_buffer_t;

struct vbs_device {
    char name[128];
    vbs_backend_type_t type;
    uint64_t max_working_set_bytes;
    uint64_t max_buffer_bytes;
    void *internal_handle;
};

struct vbs_buffer {
    void *internal_handle; /* device pointer */
    void *host_ptr;        /* pinned host shadow (may be NULL for bridge wrappers) */
    size_t size;
    vbs_device_t *device;
};

typedef enum { VBS_ARG_BUFFER = 0, VBS_ARG_SCALAR = 1 } vbs_arg_tag_t;

typedef struct {
    vbs_arg_tag_t tag;
    const void *value; /* BUFFER: device pointer. SCALAR: address of the value. */
    size_t size;       /* SCALAR: byte size of the value. BUFFER: 0. */
} vbs_arg_t;

typedef struct {
    void *native;
    vbs_op_kind_t kind;
} vbs_prim_pipeline_t;

typedef struct vbs_backend_ops {
    bool (*init)(void);
    size_t (*get_device_count)(void);
    vbs_device_t *(*get_device)(size_t index);

    vbs_buffer_t *(*alloc_buffer)(vbs_device_t *dev, size_t bytes, bool shared);
    void (*free_buffer)(vbs_buffer_t *buf);
    bool (*copy_to_device)(vbs_buffer_t *dst, const void *src, size_t bytes);
    bool (*copy_to_host)(void *dst, const vbs_buffer_t *src, size_t bytes);

    void *(*compile_linear_pipeline)(vbs_device_t *dev, vbs_ggml_type_t type, char *err_buf, size_t err_cap);
    void *(*compile_embed_pipeline)(vbs_device_t *dev, vbs_ggml_type_t type, char *err_buf, size_t err_cap);
    void *(*compile_primitive_pipeline)(vbs_device_t *dev, vbs_op_kind_t kind, char *err_buf, size_t err_cap);

    bool (*dispatch_linear_tile)(vbs_device_t *dev, void *pipeline,
                                 vbs_buffer_t *weight_private, vbs_buffer_t *weight_stage,
                                 size_t copied_bytes, vbs_buffer_t *input, vbs_buffer_t *output,
                                 uint32_t cols, uint32_t rows, uint32_t col_offset,
                                 uint32_t row_offset, bool accumulate);

    bool (*dispatch_primitive)(vbs_device_t *dev, void *pipeline, const vbs_arg_t *args,
                               size_t n_args, size_t grid_x, size_t block_x);

    void (*synchronize_device)(vbs_device_t *dev);

    bool (*launch_persistent_kernel)(vbs_device_t *dev, void *pipeline,
                                     vbs_buffer_t *control_buffer);
} vbs_backend_ops_t;

/* The table this backend exports, under the reference's symbol name
 * (include/vbs_backend.h:102), and its last-error accessor
 * (include/vbs_backend_select.h:41). */
extern const vbs_backend_ops_t g_vbs_hip_backend;
const char *vbs_hip_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* VBS_ABI_USE_REFERENCE_HEADERS */
#endif /* VBS_GFX950_ABI_H */
