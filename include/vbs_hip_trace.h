/* vbs_hip_trace.h — dispatch trace of the gfx950 HIP backend shim
 * (libvbs_backend_gfx950.so).
 *
 * The reference counts and times every call of its CPU hot-kernel table
 * (src/vbs_hotpath.c:142-151, read back through vbs_hot_counters,
 * src/vbs_hotpath.c:72-76); its GPU backends have no timing at all. The shim
 * keeps the same kind of counters for the ops table, switched on by the
 * environment when the backend initialises:
 *
 *   VBS_TRACE=1  count the table's calls per op kind and the device launches
 *                they became per launch kind (an op may be held back and
 *                issued inside another op's launch), and write one line per
 *                launch: "vbs_trace <kind> <shape>";
 *   VBS_TRACE=2  the same, and synchronize after every launch so that each
 *                line and the counters carry the launch's wall time (this
 *                serialises the device work: a measuring mode, not a
 *                production one).
 *
 * The lines go to stderr, or are appended to the file $VBS_TRACE_FILE names.
 * Unset or 0: nothing is counted or written.
 */
#ifndef VBS_GFX950_HIP_TRACE_H
#define VBS_GFX950_HIP_TRACE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Kinds: the table's op kinds and the launch kinds of the shim. */
enum {
    VBS_HIP_TRACE_EMBEDDING = 0,
    VBS_HIP_TRACE_NORMALIZE,
    VBS_HIP_TRACE_ROTARY,
    VBS_HIP_TRACE_CACHE,
    VBS_HIP_TRACE_ATTENTION,
    VBS_HIP_TRACE_ACTIVATION,
    VBS_HIP_TRACE_ELEMENTWISE,
    VBS_HIP_TRACE_LINEAR,        /* dispatch_linear_tile; a matvec launch */
    VBS_HIP_TRACE_LINEAR_BATCH,  /* vbs_hip_dispatch_linear_batch */
    VBS_HIP_TRACE_LINEAR_JOINED, /* launch: a matvec with its neighbours */
    VBS_HIP_TRACE_QKV_GROUP,     /* launch: the q / k / v run in one */
    VBS_HIP_TRACE_FFN_GROUP,     /* launch: the gate / up run in one */
    VBS_HIP_TRACE_KINDS
};

typedef struct {
    uint64_t calls;    /* table calls of this op kind */
    uint64_t launches; /* device launches of this kind */
    uint64_t ns;       /* their wall time (VBS_TRACE=2 only) */
} vbs_hip_trace_counter_t;

/* The trace level the shim read at init (0, 1 or 2). */
int vbs_hip_trace_level(void);
void vbs_hip_trace_counters(vbs_hip_trace_counter_t out[VBS_HIP_TRACE_KINDS]);
void vbs_hip_trace_reset(void);

#ifdef __cplusplus
}
#endif

#endif
