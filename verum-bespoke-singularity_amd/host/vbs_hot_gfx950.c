/* vbs_hot_gfx950.c — a CPU hot-kernel module (ABI v1) whose five matvecs run
 * on the MI355X through the gfx950 device library.
 *
 * The reference's CPU model reaches its quantised matvecs only through the
 * swappable table of include/vbs_hotpath.h; vbs_hot_load() accepts any module
 * that exports vbs_hot_abi_version() == 1 and a complete vbs_hot_kernels()
 * table (src/vbs_hotpath.c:78-109). This is such a module. Each call copies
 * the host weights, activations and scales into a device workspace, runs
 * vbs_gfx950_hot_matvec (same float order as src/hotkernels/
 * vbs_hot_ref_impl.h:49-129, so y is bit-identical to the built-in table) and
 * copies y back.
 *
 * It is a parity adapter, not a fast path: the ABI hands over host pointers,
 * so every call moves the whole weight matrix over PCIe. Two departures from
 * the ABI text (include/vbs_hotpath.h:15-16), both forced by a device behind
 * it: the module keeps one device context and a workspace that grows to the
 * largest call (never shrinks), and the device is opened on the first call,
 * not at load, so a forked verification child (src/vbs_loop.c) starts clean.
 * A call that cannot run fills y with NaN and records why
 * (vbs_hot_gfx950_last_error). Single-threaded callers only, as the CPU
 * model is (src/vbs_hotpath.c:1-7).
 *
 * Device library search: $VBS_GFX950_LIB, libvbs_gfx950.so next to this
 * module, then the loader's default path.
 */
#ifndef _GNU_SOURCE
#define _GNU_SOURCE
#endif
#include "vbs_hot_abi.h"
#include "vbs_gfx950.h"

#include <dlfcn.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q8_0 = 8 };

static struct {
    void *handle;
    int (*abi_version)(void);
    int (*init)(void);
    const char *(*last_error)(void);
    void *(*alloc)(size_t);
    int (*free)(void *);
    int (*copy_h2d)(void *, const void *, size_t);
    int (*copy_d2h)(void *, const void *, size_t);
    int (*hot_matvec)(int, const void *, uint32_t, uint32_t, const void *, const float *,
                      const float *, float *);
} g_lib;

static int g_state; /* 0 not opened yet, 1 ready, -1 failed for good */
static char g_err[512] = "ok";
static uint8_t *g_ws;
static size_t g_ws_bytes;

static void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

const char *vbs_hot_gfx950_last_error(void) { return g_err; }

static void *open_device_lib(void) {
    const char *env = getenv("VBS_GFX950_LIB");
    if (env && *env) return dlopen(env, RTLD_NOW | RTLD_LOCAL);
    Dl_info info;
    if (dladdr((void *)&open_device_lib, &info) && info.dli_fname) {
        char path[1100];
        snprintf(path, sizeof(path), "%s", info.dli_fname);
        char *slash = strrchr(path, '/');
        if (slash) {
            snprintf(slash + 1, sizeof(path) - (size_t)(slash + 1 - path), "libvbs_gfx950.so");
            void *h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
            if (h) return h;
        }
    }
    return dlopen("libvbs_gfx950.so", RTLD_NOW | RTLD_LOCAL);
}

static int device_ready(void) {
    if (g_state) return g_state > 0;
    g_state = -1;
    g_lib.handle = open_device_lib();
    if (!g_lib.handle) {
        set_err("gfx950 device library not found: %s", dlerror());
        return 0;
    }
#define BIND(field, sym)                                                   \
    do {                                                                   \
        *(void **)(&g_lib.field) = dlsym(g_lib.handle, sym);               \
        if (!g_lib.field) {                                                \
            set_err("device library lacks %s", sym);                       \
            return 0;                                                      \
        }                                                                  \
    } while (0)
    BIND(abi_version, "vbs_gfx950_abi_version");
    BIND(init, "vbs_gfx950_init");
    BIND(last_error, "vbs_gfx950_last_error");
    BIND(alloc, "vbs_gfx950_alloc");
    BIND(free, "vbs_gfx950_free");
    BIND(copy_h2d, "vbs_gfx950_copy_h2d");
    BIND(copy_d2h, "vbs_gfx950_copy_d2h");
    BIND(hot_matvec, "vbs_gfx950_hot_matvec");
#undef BIND
    if (g_lib.abi_version() != VBS_GFX950_ABI_VERSION) {
        set_err("device library ABI %d, module built for %d", g_lib.abi_version(),
                VBS_GFX950_ABI_VERSION);
        return 0;
    }
    if (!g_lib.init()) {
        set_err("gfx950 init: %s", g_lib.last_error());
        return 0;
    }
    g_state = 1;
    return 1;
}

static size_t up256(size_t n) { return (n + 255u) & ~(size_t)255u; }

static uint8_t *workspace(size_t bytes) {
    if (bytes <= g_ws_bytes) return g_ws;
    if (g_ws) g_lib.free(g_ws);
    g_ws = NULL;
    g_ws_bytes = 0;
    size_t want = bytes + bytes / 4;
    g_ws = (uint8_t *)g_lib.alloc(want);
    if (!g_ws) return NULL;
    g_ws_bytes = want;
    return g_ws;
}

/* One table call: stage w, activations and scales, run, fetch y. `cols` is
 * already cut to whole blocks for the quantised types (the reference reads
 * cols/32 blocks and ignores any tail). */
static void run(int type, const void *w, size_t wbytes, size_t rows, size_t cols,
                const void *act, size_t abytes, const float *qd, const float *qsum, size_t nblk,
                float *y) {
    if (rows == 0) return;
    const char *why = NULL;
    if (rows > 0x7FFFFFFFu || cols > 0xFFFFFFFFu) why = "shape beyond 2^31 rows / 2^32 columns";
    else if (!device_ready()) why = g_err;
    if (!why) {
        size_t o_act = up256(wbytes), o_qd = o_act + up256(abytes);
        size_t o_qs = o_qd + up256(nblk * 4), o_y = o_qs + up256(nblk * 4);
        uint8_t *ws = workspace(o_y + rows * 4);
        if (!ws) why = "device workspace allocation failed";
        else if ((wbytes && !g_lib.copy_h2d(ws, w, wbytes)) ||
                 (abytes && !g_lib.copy_h2d(ws + o_act, act, abytes)) ||
                 (qd && nblk && !g_lib.copy_h2d(ws + o_qd, qd, nblk * 4)) ||
                 (qsum && nblk && !g_lib.copy_h2d(ws + o_qs, qsum, nblk * 4)) ||
                 !g_lib.hot_matvec(type, ws, (uint32_t)rows, (uint32_t)cols, ws + o_act,
                                   (const float *)(ws + o_qd), (const float *)(ws + o_qs),
                                   (float *)(ws + o_y)) ||
                 !g_lib.copy_d2h(y, ws + o_y, rows * 4))
            why = g_lib.last_error();
    }
    if (why) {
        if (why != g_err) set_err("%s", why);
        for (size_t r = 0; r < rows; r++) y[r] = NAN;
        return;
    }
    set_err("ok");
}

static void hot_q8_0(const uint8_t *w, size_t rows, size_t cols, const int8_t *xq,
                     const float *qd, float *y) {
    size_t nb = cols / 32;
    run(T_Q8_0, w, rows * nb * 34, rows, nb * 32, xq, nb * 32, qd, NULL, nb, y);
}

static void hot_q4_0(const uint8_t *w, size_t rows, size_t cols, const int8_t *xq,
                     const float *qd, float *y) {
    size_t nb = cols / 32;
    run(T_Q4_0, w, rows * nb * 18, rows, nb * 32, xq, nb * 32, qd, NULL, nb, y);
}

static void hot_q4_1(const uint8_t *w, size_t rows, size_t cols, const int8_t *xq,
                     const float *qd, const float *qsum, float *y) {
    size_t nb = cols / 32;
    run(T_Q4_1, w, rows * nb * 20, rows, nb * 32, xq, nb * 32, qd, qsum, nb, y);
}

static void hot_f32(const float *w, size_t rows, size_t cols, const float *x, float *y) {
    run(T_F32, w, rows * cols * 4, rows, cols, x, cols * 4, NULL, NULL, 0, y);
}

static void hot_f16(const uint16_t *w, size_t rows, size_t cols, const float *x, float *y) {
    run(T_F16, w, rows * cols * 2, rows, cols, x, cols * 4, NULL, NULL, 0, y);
}

static const vbs_hot_kernels_t g_table = {
    VBS_HOT_ABI_VERSION, "gfx950-hip", hot_q8_0, hot_q4_0, hot_q4_1, hot_f32, hot_f16,
};

uint32_t vbs_hot_abi_version(void) { return VBS_HOT_ABI_VERSION; }
const vbs_hot_kernels_t *vbs_hot_kernels(void) { return &g_table; }
