/* vbs_backend_gfx950.c — Verum's HIP backend slot (g_vbs_hip_backend) on the
 * MI355X device library libvbs_gfx950.so.
 *
 * Drop-in for src/vbs_backend_hip.c: same exported symbols
 * (g_vbs_hip_backend, vbs_hip_last_error), same vbs_backend_ops_t contract,
 * same "init fails -> false + reason -> selection falls through to the CPU"
 * behaviour (src/vbs_backend_select.c:42-58). What changes is underneath: the
 * reference dlopens libamdhip64 and host-stages every op through
 * src/vbs_host_math.h; this shim dlopens the gfx950 library, checks its ABI
 * version and every entry point (as vbs_hot_load does,
 * src/vbs_hotpath.c:78-109), and forwards each op to a device kernel.
 *
 * Library search order: $VBS_GFX950_LIB, then libvbs_gfx950.so next to this
 * shim, then the loader's default search path.
 *
 * C11, no HIP headers: the shim only sees the C ABI of include/vbs_gfx950.h.
 */
#ifndef _GNU_SOURCE
#define _GNU_SOURCE
#endif
#include "vbs_abi.h"
#include "vbs_gfx950.h"
#include "vbs_hip_batch.h"
#include "vbs_hip_trace.h"

#include <dlfcn.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ---- the device library's entry points -------------------------------- */

typedef struct {
    void *handle;
    char path[1200];
    int (*abi_version)(void);
    int (*init)(void);
    const char *(*last_error)(void);
    int (*device_count)(void);
    int (*device_info)(int, char *, size_t, uint64_t *, uint64_t *);
    void *(*alloc)(size_t);
    int (*free)(void *);
    void *(*host_alloc)(size_t);
    int (*host_free)(void *);
    int (*copy_h2d)(void *, const void *, size_t);
    int (*copy_d2h)(void *, const void *, size_t);
    int (*synchronize)(void);
    int (*linear_supported)(int);
    int (*linear)(int, const void *, const float *, float *, uint32_t, uint32_t, uint32_t,
                  uint32_t, int);
    int (*linear_batch)(int, const void *, const float *, uint32_t, float *, uint32_t, uint32_t,
                        uint32_t, uint32_t);
    int (*embed)(int, const void *, uint32_t, float *, uint32_t);
    int (*rms_norm)(const float *, const float *, float *, uint32_t, float);
    int (*rope)(float *, uint32_t, uint32_t, uint32_t, float);
    int (*cache_store)(const float *, const float *, uint16_t *, uint16_t *, uint32_t, uint32_t,
                       uint32_t, uint32_t);
    int (*attention)(const float *, const uint16_t *, const uint16_t *, float *, uint32_t,
                     uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, float);
    int (*silu_mul)(const float *, const float *, float *, uint32_t);
    int (*add)(const float *, const float *, float *, uint32_t);
    int (*linear_fused)(int, const void *, const float *, float *, uint32_t, uint32_t,
                        const vbs_gfx950_linear_join_t *);
    int (*qkv_fused)(int, const void *, const void *, const void *, const float *, uint32_t,
                     uint32_t, uint32_t, const float *, float, float *, float *, float *, float *,
                     uint32_t, uint32_t, float, uint16_t *, uint16_t *, uint32_t, uint32_t);
    int (*gate_up_fused)(int, const void *, const void *, const float *, uint32_t, uint32_t,
                         const float *, float, float *, float *, float *, float *);
} gfx950_lib_t;

static gfx950_lib_t g_lib;
static bool flush_pending(void); /* issues the held-back op, if any (below) */
static int g_probed, g_ready;
static char g_err[512] = "not probed yet";
static vbs_device_t g_device;

static void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

/* A device-library failure: keep its reason. */
static bool lib_fail(const char *what) {
    set_err("%s: %s", what, g_lib.last_error ? g_lib.last_error() : "unknown");
    return false;
}

const char *vbs_hip_last_error(void) { return g_err; }

/* Path of the device library in use ("" before a successful init). Lets a
 * caller confirm which native library is serving the backend. */
const char *vbs_gfx950_shim_library_path(void) { return g_ready ? g_lib.path : ""; }

static void *open_lib(void) {
    const char *env = getenv("VBS_GFX950_LIB");
    if (env && *env) {
        void *h = dlopen(env, RTLD_NOW | RTLD_LOCAL);
        if (h) snprintf(g_lib.path, sizeof(g_lib.path), "%s", env);
        else set_err("cannot load %s: %s", env, dlerror());
        return h;
    }
    Dl_info info;
    if (dladdr((void *)&open_lib, &info) && info.dli_fname) {
        char dir[1024];
        snprintf(dir, sizeof(dir), "%s", info.dli_fname);
        char *slash = strrchr(dir, '/');
        if (slash) {
            *slash = '\0';
            char cand[1100];
            snprintf(cand, sizeof(cand), "%s/libvbs_gfx950.so", dir);
            void *h = dlopen(cand, RTLD_NOW | RTLD_LOCAL);
            if (h) {
                snprintf(g_lib.path, sizeof(g_lib.path), "%s", cand);
                return h;
            }
        }
    }
    void *h = dlopen("libvbs_gfx950.so", RTLD_NOW | RTLD_LOCAL);
    if (h) snprintf(g_lib.path, sizeof(g_lib.path), "libvbs_gfx950.so");
    else set_err("gfx950 device library not found (libvbs_gfx950.so): %s", dlerror());
    return h;
}

/* ---- dispatch trace (include/vbs_hip_trace.h) ---------------------------- */
static int g_trace;
static FILE *g_trace_out;
static vbs_hip_trace_counter_t g_tc[VBS_HIP_TRACE_KINDS];
static const char *const k_trace_name[VBS_HIP_TRACE_KINDS] = {
    "embedding",  "normalize",   "rotary", "cache",        "attention",     "activation",
    "elementwise", "linear", "linear_batch", "linear_joined", "qkv_group", "ffn_group"};

static uint64_t now_ns(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

static void trace_init(void) {
    const char *e = getenv("VBS_TRACE");
    g_trace = e ? atoi(e) : 0;
    g_trace = g_trace < 0 ? 0 : g_trace > 2 ? 2 : g_trace;
    if (!g_trace) return;
    const char *f = getenv("VBS_TRACE_FILE");
    g_trace_out = f && *f ? fopen(f, "a") : NULL;
    if (g_trace_out) setvbuf(g_trace_out, NULL, _IOLBF, 0);  /* whole lines, as they come */
    else g_trace_out = stderr;
}

static void trace_call(int kind) {
    if (g_trace) g_tc[kind].calls++;
}

static uint64_t trace_t0(void) { return g_trace > 1 ? now_ns() : 0; }

/* After a device-library call that returned r (1: it launched): counts the
 * launch, at level 2 waits for it and adds its wall time, and writes its
 * line. Returns r (0 if the wait failed). */
static int trace_launch(int kind, uint64_t t0, int r, const char *fmt, ...) {
    if (!g_trace || r != 1) return r;
    char desc[192];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(desc, sizeof(desc), fmt, ap);
    va_end(ap);
    g_tc[kind].launches++;
    if (g_trace > 1) {
        if (!g_lib.synchronize()) return 0;
        const uint64_t dt = now_ns() - t0;
        g_tc[kind].ns += dt;
        fprintf(g_trace_out, "vbs_trace %s %s %.2f us\n", k_trace_name[kind], desc, (double)dt * 1e-3);
    } else {
        fprintf(g_trace_out, "vbs_trace %s %s\n", k_trace_name[kind], desc);
    }
    return r;
}

int vbs_hip_trace_level(void) { return g_trace; }

void vbs_hip_trace_counters(vbs_hip_trace_counter_t out[VBS_HIP_TRACE_KINDS]) {
    memcpy(out, g_tc, sizeof(g_tc));
}

void vbs_hip_trace_reset(void) { memset(g_tc, 0, sizeof(g_tc)); }

static bool gfx950_init(void) {
    if (g_probed) return g_ready != 0;
    g_probed = 1;
    trace_init();
    memset(&g_lib, 0, sizeof(g_lib));
    g_lib.handle = open_lib();
    if (!g_lib.handle) return false;

#define BIND(field, sym)                                                       \
    do {                                                                       \
        *(void **)(&g_lib.field) = dlsym(g_lib.handle, sym);                   \
        if (!g_lib.field) {                                                    \
            set_err("%s lacks %s", g_lib.path, sym);                           \
            dlclose(g_lib.handle);                                             \
            g_lib.handle = NULL;                                               \
            return false;                                                      \
        }                                                                      \
    } while (0)
    BIND(abi_version, "vbs_gfx950_abi_version");
    BIND(init, "vbs_gfx950_init");
    BIND(last_error, "vbs_gfx950_last_error");
    BIND(device_count, "vbs_gfx950_device_count");
    BIND(device_info, "vbs_gfx950_device_info");
    BIND(alloc, "vbs_gfx950_alloc");
    BIND(free, "vbs_gfx950_free");
    BIND(host_alloc, "vbs_gfx950_host_alloc");
    BIND(host_free, "vbs_gfx950_host_free");
    BIND(copy_h2d, "vbs_gfx950_copy_h2d");
    BIND(copy_d2h, "vbs_gfx950_copy_d2h");
    BIND(synchronize, "vbs_gfx950_synchronize");
    BIND(linear_supported, "vbs_gfx950_linear_supported");
    BIND(linear, "vbs_gfx950_linear");
    BIND(linear_batch, "vbs_gfx950_linear_batch");
    BIND(embed, "vbs_gfx950_embed");
    BIND(rms_norm, "vbs_gfx950_rms_norm");
    BIND(rope, "vbs_gfx950_rope");
    BIND(cache_store, "vbs_gfx950_cache_store");
    BIND(attention, "vbs_gfx950_attention");
    BIND(silu_mul, "vbs_gfx950_silu_mul");
    BIND(add, "vbs_gfx950_add");
    BIND(linear_fused, "vbs_gfx950_linear_fused");
    BIND(qkv_fused, "vbs_gfx950_qkv_fused");
    BIND(gate_up_fused, "vbs_gfx950_gate_up_fused");
#undef BIND

    int ver = g_lib.abi_version();
    if (ver != VBS_GFX950_ABI_VERSION) {
        set_err("%s has ABI version %d, this backend needs %d", g_lib.path, ver,
                VBS_GFX950_ABI_VERSION);
        dlclose(g_lib.handle);
        g_lib.handle = NULL;
        return false;
    }
    if (!g_lib.init()) return lib_fail("gfx950 init");
    if (g_lib.device_count() < 1) {
        set_err("gfx950 library reports no device");
        return false;
    }
    memset(&g_device, 0, sizeof(g_device));
    uint64_t total = 0, free_b = 0;
    char name[128] = {0};
    if (!g_lib.device_info(0, name, sizeof(name), &total, &free_b)) return lib_fail("device info");
    snprintf(g_device.name, sizeof(g_device.name), "%s", name);
    g_device.type = VBS_BACKEND_HIP;
    g_device.max_working_set_bytes = total;
    g_device.max_buffer_bytes = total;
    g_device.internal_handle = NULL;
    g_ready = 1;
    set_err("ok");
    return true;
}

static size_t gfx950_get_device_count(void) { return g_ready ? 1 : 0; }

static vbs_device_t *gfx950_get_device(size_t i) { return (g_ready && i == 0) ? &g_device : NULL; }

/* Device memory plus a host shadow: pinned for staging windows (shared),
 * lazily committed calloc otherwise, as the reference provides host_ptr for
 * every buffer (src/vbs_backend_hip.c:241) and the slice executor and the
 * backend self-test write tiles through it. */
typedef struct {
    vbs_buffer_t pub;
    int pinned;
} gfx950_buffer_t;

static vbs_buffer_t *gfx950_alloc_buffer(vbs_device_t *dev, size_t bytes, bool shared) {
    if (!g_ready) { set_err("alloc_buffer before a successful init"); return NULL; }
    if (bytes == 0) bytes = 1;
    gfx950_buffer_t *b = (gfx950_buffer_t *)calloc(1, sizeof(*b));
    if (!b) return NULL;
    b->pub.internal_handle = g_lib.alloc(bytes);
    if (!b->pub.internal_handle) { lib_fail("alloc_buffer"); free(b); return NULL; }
    if (shared) {
        b->pub.host_ptr = g_lib.host_alloc(bytes);
        b->pinned = b->pub.host_ptr != NULL;
    }
    if (!b->pub.host_ptr) b->pub.host_ptr = calloc(1, bytes);
    b->pub.size = bytes;
    b->pub.device = dev;
    return &b->pub;
}

static void gfx950_free_buffer(vbs_buffer_t *buf) {
    if (!buf) return;
    if (g_ready) (void)flush_pending();
    gfx950_buffer_t *b = (gfx950_buffer_t *)buf;
    if (g_ready) g_lib.free(buf->internal_handle);
    if (b->pinned) g_lib.host_free(buf->host_ptr);
    else free(buf->host_ptr);
    free(b);
}

static bool gfx950_copy_to_device(vbs_buffer_t *dst, const void *src, size_t bytes) {
    if (!g_ready || !dst || !src) return false;
    if (!flush_pending()) return false;
    return g_lib.copy_h2d(dst->internal_handle, src, bytes) ? true : lib_fail("copy_to_device");
}

/* Waits for all earlier work: the bridge reads logits without a prior
 * synchronize (src/vbs_specializer_bridge.c:201-206). */
static bool gfx950_copy_to_host(void *dst, const vbs_buffer_t *src, size_t bytes) {
    if (!g_ready || !dst || !src) return false;
    if (!flush_pending()) return false;
    return g_lib.copy_d2h(dst, src->internal_handle, bytes) ? true : lib_fail("copy_to_host");
}

/* ---- held-back ops --------------------------------------------------------
 * The bridge issues each token step as ~16 ops per layer (NORMALIZE, LINEAR,
 * ROTARY, ..., src/vbs_specializer.c:270-349), and at this size each
 * separate launch costs about as much as its work. The shim therefore holds
 * back a NORMALIZE and the resident LINEARs that read its output, each with
 * a ROTARY of its own output, and issues them with the op that ends the run:
 *   NORMALIZE, LINEAR q, ROTARY, LINEAR k, ROTARY, LINEAR v, CACHE
 *                                   -> one launch (vbs_gfx950_qkv_fused)
 *   NORMALIZE, LINEAR gate, LINEAR up, ACTIVATION
 *                                   -> one launch (vbs_gfx950_gate_up_fused)
 * and otherwise each held LINEAR with its neighbours in one launch
 * (vbs_gfx950_linear_fused):
 *   the NORMALIZE before it                       -> RMSNorm + matvec
 *   a ROTARY of its output (in place)             -> matvec + RoPE
 *   an ELEMENTWISE a = a + its output             -> matvec + add
 *   a CACHE with its output as V                  -> matvec + f16 K/V store
 *   an ACTIVATION with its output as up           -> matvec + SiLU gate
 * Each result is bit-identical to the ops run one by one, and every buffer the
 * ops write is written (the normalised x, each linear's own output). Any other
 * op, copy, free or synchronize first issues what is held, in order, so the
 * ordering the caller sees is the one it asked for; an error of a held op is
 * reported by the call that issues it. An op joins the held run only if it
 * writes no buffer that a held op reads or writes (the checks compare buffer
 * addresses: the bridge's buffers never partly overlap). One host thread
 * drives the table (as the reference assumes, src/vbs_hotpath.c:3-5). */
typedef struct {
    int type;                        /* LINEAR (convention A, no offsets) */
    const void *w;
    const float *x;
    float *y;
    uint32_t cols, rows;
    int rope;                        /* a ROTARY of y held behind it */
    uint32_t pos, hd, nh;
    float theta;
} held_linear_t;

typedef struct {
    int has_norm;                    /* a NORMALIZE, in front of linear 0 if any */
    const float *n_in, *n_w;
    float *n_out;
    uint32_t n_dim;
    float n_eps;
    int n_lin;                       /* LINEARs held, in issue order, all reading lin[0].x */
    held_linear_t lin[3];
} pending_t;

static pending_t g_pend;

static void drop_pending(void) { memset(&g_pend, 0, sizeof(g_pend)); }

static bool run_norm(const pending_t *p) {
    const uint64_t t0 = trace_t0();
    return trace_launch(VBS_HIP_TRACE_NORMALIZE, t0,
                        g_lib.rms_norm(p->n_in, p->n_w, p->n_out, p->n_dim, p->n_eps), "%u", p->n_dim)
               ? true
               : lib_fail("normalize");
}

static const char *type_name(vbs_ggml_type_t t);

/* A held linear's one-launch form, traced. */
static int linear_fused_traced(const held_linear_t *l, const float *x, const vbs_gfx950_linear_join_t *j) {
    const uint64_t t0 = trace_t0();
    return trace_launch(VBS_HIP_TRACE_LINEAR_JOINED, t0,
                        g_lib.linear_fused(l->type, l->w, x, l->y, l->cols, l->rows, j),
                        "%s %ux%u%s%s%s%s%s", type_name((vbs_ggml_type_t)l->type), l->rows, l->cols,
                        j->norm_w ? " +norm" : "", j->rope ? " +rope" : "", j->acc ? " +add" : "",
                        j->gate ? " +silu" : "", j->k_row ? " +cache" : "");
}

static int rope_traced(const held_linear_t *l) {
    const uint64_t t0 = trace_t0();
    return trace_launch(VBS_HIP_TRACE_ROTARY, t0, g_lib.rope(l->y, l->pos, l->hd, l->nh, l->theta),
                        "%ux%u pos %u", l->nh, l->hd, l->pos);
}

/* Held linear i with what it carries (the RMSNorm in front of linear 0, its
 * ROTARY) and the op `j` names after it (acc, gate or k_row; or none), in one
 * launch where a fused kernel takes them, else one by one without the op `j`
 * names: *done tells the caller whether that op was part of the launch. */
static bool issue_linear(const pending_t *p, int i, vbs_gfx950_linear_join_t *j, bool *done) {
    const held_linear_t *l = &p->lin[i];
    const bool norm = i == 0 && p->has_norm;
    const bool after = j->acc || j->gate || j->k_row;
    *done = false;
    if (norm) {
        j->norm_w = p->n_w;
        j->norm_eps = p->n_eps;
        j->x_normed = p->n_out;
    }
    if (l->rope) {
        j->rope = 1;
        j->pos = l->pos;
        j->head_dim = l->hd;
        j->theta = l->theta;
    }
    if (norm || l->rope || after) {
        int r = linear_fused_traced(l, norm ? p->n_in : l->x, j);
        if (r == 1) {
            *done = after;
            return true;
        }
        if (r == 0) return lib_fail("linear tile (fused)");
        if (norm && (l->rope || after)) { /* the RMSNorm + matvec alone, then the RoPE */
            vbs_gfx950_linear_join_t n = {0};
            n.norm_w = p->n_w;
            n.norm_eps = p->n_eps;
            n.x_normed = p->n_out;
            r = linear_fused_traced(l, p->n_in, &n);
            if (r == 0) return lib_fail("linear tile (fused)");
            if (r == 1) {
                if (l->rope && !rope_traced(l)) return lib_fail("rotary");
                return true;
            }
        }
    }
    if (norm && !run_norm(p)) return false;
    const uint64_t t0 = trace_t0();
    if (!trace_launch(VBS_HIP_TRACE_LINEAR, t0,
                      g_lib.linear(l->type, l->w, l->x, l->y, l->cols, l->rows, 0, 0, 0), "%s %ux%u",
                      type_name((vbs_ggml_type_t)l->type), l->rows, l->cols))
        return lib_fail("linear tile");
    if (l->rope && !rope_traced(l)) return lib_fail("rotary");
    return true;
}

static bool flush_pending(void) {
    const pending_t p = g_pend;
    drop_pending();
    if (p.n_lin == 0) return p.has_norm ? run_norm(&p) : true;
    for (int i = 0; i < p.n_lin; i++) {
        vbs_gfx950_linear_join_t j = {0};
        bool done;
        if (!issue_linear(&p, i, &j, &done)) return false;
    }
    return true;
}

/* The last held linear joined with the op `j` names after it, the held ops
 * before it issued first; *done as in issue_linear. */
static bool issue_last_with(vbs_gfx950_linear_join_t *j, bool *done) {
    const pending_t p = g_pend;
    drop_pending();
    *done = false;
    for (int i = 0; i + 1 < p.n_lin; i++) {
        vbs_gfx950_linear_join_t none = {0};
        bool d;
        if (!issue_linear(&p, i, &none, &d)) return false;
    }
    return issue_linear(&p, p.n_lin - 1, j, done);
}

/* Whether buffer b is one that a held op reads or writes. */
static bool touches_held(const void *b) {
    const pending_t *h = &g_pend;
    if (h->has_norm && (b == (const void *)h->n_in || b == (const void *)h->n_out)) return true;
    for (int i = 0; i < h->n_lin; i++)
        if (b == (const void *)h->lin[i].x || b == (const void *)h->lin[i].y) return true;
    return false;
}

/* A convention-A LINEAR: joins the held run (the NORMALIZE it reads, or the
 * q / k / v and gate / up runs above) or starts a new one. */
static bool hold_linear(const held_linear_t *n) {
    pending_t *h = &g_pend;
    if (h->n_lin > 0 && h->n_lin < 3 && n->x == h->lin[0].x && n->type == h->lin[0].type &&
        n->cols == h->lin[0].cols && !touches_held(n->y)) {
        bool all_roped = true;
        for (int i = 0; i < h->n_lin; i++) all_roped = all_roped && h->lin[i].rope;
        const bool ffn = h->n_lin == 1 && !h->lin[0].rope && n->rows == h->lin[0].rows;
        if (all_roped || ffn) {
            h->lin[h->n_lin++] = *n;
            return true;
        }
    }
    if (h->n_lin == 0 && h->has_norm && n->x == h->n_out && n->cols == h->n_dim &&
        h->n_in != (const float *)h->n_out && (const float *)n->y != h->n_in &&
        n->y != h->n_out) {
        h->lin[0] = *n;
        h->n_lin = 1;
        return true;
    }
    if (!flush_pending()) return false;
    g_pend.lin[0] = *n;
    g_pend.n_lin = 1;
    return true;
}

/* ---- pipelines ---------------------------------------------------------- */

typedef struct {
    vbs_ggml_type_t type;
} gfx950_linear_pipe_t;

typedef struct {
    vbs_prim_pipeline_t base; /* .native = this struct, .kind = op kind */
    vbs_ggml_type_t type;     /* EMBEDDING table type */
} gfx950_prim_pipe_t;

static const char *type_name(vbs_ggml_type_t t) {
    switch (t) {
        case VBS_GGML_TYPE_F32: return "F32";
        case VBS_GGML_TYPE_F16: return "F16";
        case VBS_GGML_TYPE_Q4_0: return "Q4_0";
        case VBS_GGML_TYPE_Q4_1: return "Q4_1";
        case VBS_GGML_TYPE_Q8_0: return "Q8_0";
        case VBS_GGML_TYPE_Q4_K: return "Q4_K";
        case VBS_GGML_TYPE_Q6_K: return "Q6_K";
        case VBS_GGML_TYPE_LNS8: return "LNS8";
        default: return "unsupported";
    }
}

static void *gfx950_compile_linear_pipeline(vbs_device_t *dev, vbs_ggml_type_t type, char *err,
                                            size_t cap) {
    (void)dev;
    if (!g_ready || !g_lib.linear_supported((int)type)) {
        if (err && cap)
            snprintf(err, cap, "gfx950 backend: no linear kernel for weight type %d", (int)type);
        return NULL;
    }
    gfx950_linear_pipe_t *p = (gfx950_linear_pipe_t *)malloc(sizeof(*p));
    if (p) p->type = type;
    return p;
}

static gfx950_prim_pipe_t *prim_pipe(vbs_op_kind_t kind, vbs_ggml_type_t type) {
    gfx950_prim_pipe_t *p = (gfx950_prim_pipe_t *)malloc(sizeof(*p));
    if (!p) return NULL;
    p->base.native = p;
    p->base.kind = kind;
    p->type = type;
    return p;
}

static void *gfx950_compile_embed_pipeline(vbs_device_t *dev, vbs_ggml_type_t type, char *err,
                                           size_t cap) {
    (void)dev;
    if (!g_ready || !g_lib.linear_supported((int)type)) {
        if (err && cap)
            snprintf(err, cap, "gfx950 backend: no embedding kernel for weight type %d", (int)type);
        return NULL;
    }
    return prim_pipe(VBS_OP_EMBEDDING, type);
}

static void *gfx950_compile_primitive_pipeline(vbs_device_t *dev, vbs_op_kind_t kind, char *err,
                                               size_t cap) {
    (void)dev;
    switch (kind) {
        case VBS_OP_EMBEDDING: /* F32 table, as in the reference */
        case VBS_OP_NORMALIZE:
        case VBS_OP_ROTARY:
        case VBS_OP_CACHE:
        case VBS_OP_ATTENTION:
        case VBS_OP_ACTIVATION:
        case VBS_OP_ELEMENTWISE:
            if (g_ready) return prim_pipe(kind, VBS_GGML_TYPE_F32);
            /* fall through */
        default:
            if (err && cap)
                snprintf(err, cap, "gfx950 backend: no primitive kernel for op kind %d", (int)kind);
            return NULL;
    }
}

/* ---- dispatch ----------------------------------------------------------- */

static uint64_t packed_row_bytes(vbs_ggml_type_t t, uint32_t cols) {
    switch (t) {
        case VBS_GGML_TYPE_F32: return 4ull * cols;
        case VBS_GGML_TYPE_F16: return 2ull * cols;
        case VBS_GGML_TYPE_Q4_0: return 18ull * (cols / 32u);
        case VBS_GGML_TYPE_Q4_1: return 20ull * (cols / 32u);
        case VBS_GGML_TYPE_Q8_0: return 34ull * (cols / 32u);
        case VBS_GGML_TYPE_Q4_K: return 144ull * (cols / 256u);
        case VBS_GGML_TYPE_Q6_K: return 210ull * (cols / 256u);
        case VBS_GGML_TYPE_LNS8: return 36ull * (cols / 32u);
        default: return 0;
    }
}

/* Two calling conventions (src/vbs_backend_hip.c:346-394):
 *  A (bridge, resident): ws == NULL, wp->internal_handle is the packed tensor.
 *  B (slice executor, staged): ws->host_ptr holds a packed tile; it is
 *    uploaded into the private device buffer wp and computed there.
 * Offsets index x and y; accumulate adds into y. */
static bool gfx950_dispatch_linear_tile(vbs_device_t *dev, void *pipeline, vbs_buffer_t *wp,
                                        vbs_buffer_t *ws, size_t copied_bytes, vbs_buffer_t *in,
                                        vbs_buffer_t *out, uint32_t cols, uint32_t rows,
                                        uint32_t col_off, uint32_t row_off, bool accumulate) {
    (void)dev;
    gfx950_linear_pipe_t *p = (gfx950_linear_pipe_t *)pipeline;
    if (!g_ready || !p || !wp || !in || !out) return false;
    trace_call(VBS_HIP_TRACE_LINEAR);
    uint64_t need = packed_row_bytes(p->type, cols) * rows;
    if (ws && ws->host_ptr) {
        size_t n = copied_bytes ? copied_bytes : (size_t)need;
        if (n < need) {
            set_err("linear tile: staged %zu bytes, %s %ux%u needs %llu", n, type_name(p->type),
                    rows, cols, (unsigned long long)need);
            return false;
        }
        if ((ws->size && ws->size < need) || (wp->size && wp->size < need)) {
            set_err("linear tile: window smaller than the %llu-byte tile", (unsigned long long)need);
            return false;
        }
        if (!flush_pending()) return false;
        if (!g_lib.copy_h2d(wp->internal_handle, ws->host_ptr, (size_t)need))
            return lib_fail("linear tile upload");
    }
    const float *x = (const float *)in->internal_handle;
    float *y = (float *)out->internal_handle;
    if (!ws && !col_off && !row_off && !accumulate && need && wp->internal_handle && x && y &&
        (const float *)y != x) {
        /* convention A, the bridge's resident matvec: held back for the next op */
        held_linear_t n = {0};
        n.type = (int)p->type;
        n.w = wp->internal_handle;
        n.x = x;
        n.y = y;
        n.cols = cols;
        n.rows = rows;
        return hold_linear(&n);
    }
    if (!flush_pending()) return false;
    const uint64_t t0 = trace_t0();
    if (!trace_launch(VBS_HIP_TRACE_LINEAR, t0,
                      g_lib.linear((int)p->type, wp->internal_handle, x, y, cols, rows, col_off,
                                   row_off, accumulate ? 1 : 0),
                      "%s %ux%u at %u,%u%s%s", type_name(p->type), rows, cols, row_off, col_off,
                      accumulate ? " +acc" : "", ws ? " staged" : ""))
        return lib_fail("linear tile");
    return true;
}

/* ---- batched linear (extension, include/vbs_hip_batch.h) ------------------ */

uint32_t vbs_hip_linear_batch_version(void) { return VBS_HIP_LINEAR_BATCH_VERSION; }

bool vbs_hip_dispatch_linear_batch(vbs_device_t *dev, void *pipeline, vbs_buffer_t *w,
                                   vbs_buffer_t *x, uint32_t x_stride, vbs_buffer_t *y,
                                   uint32_t y_stride, uint32_t cols, uint32_t rows,
                                   uint32_t batch) {
    (void)dev;
    gfx950_linear_pipe_t *p = (gfx950_linear_pipe_t *)pipeline;
    if (!g_ready) {
        set_err("linear batch before a successful init");
        return false;
    }
    trace_call(VBS_HIP_TRACE_LINEAR_BATCH);
    if (!p || !w || !x || !y || !w->internal_handle || !x->internal_handle || !y->internal_handle) {
        set_err("linear batch: null pipeline or buffer");
        return false;
    }
    if (batch == 0 || batch > 16u) {
        set_err("linear batch: batch %u outside 1..16", batch);
        return false;
    }
    if (x_stride < cols || y_stride < rows) {
        set_err("linear batch: strides %u/%u below cols/rows %u/%u", x_stride, y_stride, cols,
                rows);
        return false;
    }
    const uint64_t need_w = packed_row_bytes(p->type, cols) * rows;
    const uint64_t need_x = 4ull * ((uint64_t)(batch - 1u) * x_stride + cols);
    const uint64_t need_y = 4ull * ((uint64_t)(batch - 1u) * y_stride + rows);
    if ((w->size && w->size < need_w) || (x->size && x->size < need_x) ||
        (y->size && y->size < need_y)) {
        set_err("linear batch: a buffer is smaller than %s %ux%u at batch %u needs",
                type_name(p->type), rows, cols, batch);
        return false;
    }
    if (!flush_pending()) return false;
    const uint64_t t0 = trace_t0();
    if (!trace_launch(VBS_HIP_TRACE_LINEAR_BATCH, t0,
                      g_lib.linear_batch((int)p->type, w->internal_handle,
                                         (const float *)x->internal_handle, x_stride,
                                         (float *)y->internal_handle, y_stride, cols, rows, batch),
                      "%s %ux%u x%u", type_name(p->type), rows, cols, batch))
        return lib_fail("linear batch");
    return true;
}

static bool arg_ok(const vbs_arg_t *a, vbs_arg_tag_t tag) {
    if (a->tag != tag) return false;
    if (tag == VBS_ARG_SCALAR) return a->value && a->size == 4;
    return a->value != NULL;
}

#define BUF(i) ((void *)args[i].value)
#define U32(i) (*(const uint32_t *)args[i].value)
#define F32(i) (*(const float *)args[i].value)

/* Canonical bridge argument order (include/vbs_specializer_bridge.h:44-53).
 * grid_x/block_x are launch hints for other backends; gfx950 kernels size
 * their own grids. */
static bool gfx950_dispatch_primitive(vbs_device_t *dev, void *pipeline, const vbs_arg_t *args,
                                      size_t n_args, size_t grid_x, size_t block_x) {
    (void)dev; (void)grid_x; (void)block_x;
    gfx950_prim_pipe_t *pp = (gfx950_prim_pipe_t *)pipeline;
    if (!g_ready || !pp || !args) return false;
    static const char *const sig[] = {
        [VBS_OP_EMBEDDING] = "BSBS", [VBS_OP_NORMALIZE] = "BBBSS", [VBS_OP_ROTARY] = "BSSSS",
        [VBS_OP_CACHE] = "BBBBSSSS", [VBS_OP_ATTENTION] = "BBBBSSSSSSS",
        [VBS_OP_ACTIVATION] = "BBBS", [VBS_OP_ELEMENTWISE] = "BBBS",
    };
    if ((unsigned)pp->base.kind >= sizeof(sig) / sizeof(sig[0]) || !sig[pp->base.kind]) {
        set_err("dispatch_primitive: op kind %d has no kernel", (int)pp->base.kind);
        return false;
    }
    const char *s = sig[pp->base.kind];
    if (n_args != strlen(s)) {
        set_err("dispatch_primitive: op kind %d takes %zu arguments, got %zu", (int)pp->base.kind,
                strlen(s), n_args);
        return false;
    }
    for (size_t i = 0; i < n_args; i++) {
        if (!arg_ok(&args[i], s[i] == 'B' ? VBS_ARG_BUFFER : VBS_ARG_SCALAR)) {
            set_err("dispatch_primitive: op kind %d argument %zu is malformed", (int)pp->base.kind, i);
            return false;
        }
    }
    static const int trace_kind[] = {
        [VBS_OP_EMBEDDING] = VBS_HIP_TRACE_EMBEDDING, [VBS_OP_NORMALIZE] = VBS_HIP_TRACE_NORMALIZE,
        [VBS_OP_ROTARY] = VBS_HIP_TRACE_ROTARY,       [VBS_OP_CACHE] = VBS_HIP_TRACE_CACHE,
        [VBS_OP_ATTENTION] = VBS_HIP_TRACE_ATTENTION, [VBS_OP_ACTIVATION] = VBS_HIP_TRACE_ACTIVATION,
        [VBS_OP_ELEMENTWISE] = VBS_HIP_TRACE_ELEMENTWISE,
    };
    const int tk = trace_kind[pp->base.kind];
    trace_call(tk);
    /* held itself (NORMALIZE, ROTARY), or issued with the held run */
    if (pp->base.kind == VBS_OP_NORMALIZE && BUF(0) != BUF(2)) {
        if (!flush_pending()) return false;
        g_pend.has_norm = 1;
        g_pend.n_in = (const float *)BUF(0);
        g_pend.n_w = (const float *)BUF(1);
        g_pend.n_out = (float *)BUF(2);
        g_pend.n_dim = U32(3);
        g_pend.n_eps = F32(4);
        return true;
    }
    if (g_pend.n_lin > 0) {
        const pending_t *h = &g_pend;
        const held_linear_t *last = &h->lin[h->n_lin - 1];
        vbs_gfx950_linear_join_t j = {0};
        bool joined = false, done = false;
        switch (pp->base.kind) {
            case VBS_OP_ROTARY: /* (x, pos, head_dim, n_heads, theta), x the last output */
                if (!last->rope && (float *)BUF(0) == last->y &&
                    (uint64_t)U32(2) * U32(3) == last->rows) {
                    held_linear_t *l = &g_pend.lin[h->n_lin - 1];
                    l->rope = 1;
                    l->pos = U32(1);
                    l->hd = U32(2);
                    l->nh = U32(3);
                    l->theta = F32(4);
                    return true;
                }
                break;
            case VBS_OP_ELEMENTWISE: /* (a, b, out, n): a = a + the last output */
                if (!last->rope && BUF(1) == last->y && BUF(2) == BUF(0) && BUF(0) != last->y &&
                    (const float *)BUF(0) != last->x && U32(3) == last->rows) {
                    j.acc = (float *)BUF(0);
                    joined = true;
                }
                break;
            case VBS_OP_CACHE: { /* (k, v, kc, vc, pos, layer, max_ctx, kv_dim) */
                const uint32_t pos = U32(4), layer = U32(5), mc = U32(6), kvd = U32(7);
                const held_linear_t *q = &h->lin[0], *k = &h->lin[1], *v = &h->lin[2];
                if (touches_held(BUF(2)) || touches_held(BUF(3))) break;  /* the caches */
                if (h->n_lin == 3 && q->rope && k->rope && !v->rope && BUF(0) == k->y &&
                    BUF(1) == v->y && kvd == k->rows && kvd == v->rows && pos < mc &&
                    q->pos == pos && k->pos == pos && q->hd == k->hd && q->theta == k->theta) {
                    /* NORMALIZE, q, ROTARY, k, ROTARY, v, CACHE in one launch */
                    const uint64_t t0 = trace_t0();
                    const int r = trace_launch(
                        VBS_HIP_TRACE_QKV_GROUP, t0,
                        g_lib.qkv_fused(q->type, q->w, k->w, v->w, h->has_norm ? h->n_in : q->x,
                                        q->cols, q->rows, kvd, h->has_norm ? h->n_w : NULL,
                                        h->n_eps, h->has_norm ? h->n_out : NULL, q->y, k->y, v->y,
                                        pos, q->hd, q->theta, (uint16_t *)BUF(2),
                                        (uint16_t *)BUF(3), layer, mc),
                        "%s %u+%u+%ux%u%s pos %u", type_name((vbs_ggml_type_t)q->type), q->rows,
                        kvd, kvd, q->cols, h->has_norm ? " +norm" : "", pos);
                    if (r == 1) {
                        drop_pending();
                        return true;
                    }
                    if (r == 0) {
                        drop_pending();
                        return lib_fail("q/k/v (grouped)");
                    }
                }
                if (!last->rope && BUF(1) == last->y && BUF(0) != last->y && kvd == last->rows &&
                    pos < mc) {
                    j.k_row = (const float *)BUF(0);
                    j.kc = (uint16_t *)BUF(2);
                    j.vc = (uint16_t *)BUF(3);
                    j.kv_off = ((uint64_t)layer * mc + pos) * kvd;
                    joined = true;
                }
                break;
            }
            case VBS_OP_ACTIVATION: { /* (gate, up, out, n) */
                const held_linear_t *g = &h->lin[0], *u = &h->lin[1];
                const void *out = BUF(2);
                if (h->n_lin == 2 && !g->rope && !u->rope && BUF(0) == g->y && BUF(1) == u->y &&
                    U32(3) == g->rows && U32(3) == u->rows && !touches_held(out)) {
                    /* NORMALIZE, gate, up, ACTIVATION in one launch */
                    const uint64_t t0 = trace_t0();
                    const int r = trace_launch(
                        VBS_HIP_TRACE_FFN_GROUP, t0,
                        g_lib.gate_up_fused(g->type, g->w, u->w, h->has_norm ? h->n_in : g->x,
                                            g->cols, g->rows, h->has_norm ? h->n_w : NULL,
                                            h->n_eps, h->has_norm ? h->n_out : NULL, g->y, u->y,
                                            (float *)out),
                        "%s 2x%ux%u%s", type_name((vbs_ggml_type_t)g->type), g->rows, g->cols,
                        h->has_norm ? " +norm" : "");
                    if (r == 1) {
                        drop_pending();
                        return true;
                    }
                    if (r == 0) {
                        drop_pending();
                        return lib_fail("gate/up (grouped)");
                    }
                }
                if (!last->rope && BUF(1) == last->y && BUF(0) != last->y && out != last->y &&
                    out != BUF(0) && out != (const void *)last->x && U32(3) == last->rows) {
                    j.gate = (const float *)BUF(0);
                    j.hidden = (float *)out;
                    joined = true;
                }
                break;
            }
            default:
                break;
        }
        if (joined) {
            if (!issue_last_with(&j, &done)) return false;
            if (done) return true;  /* else: the held ops ran alone, this one follows */
        }
    }
    if (!flush_pending()) return false;
    int ok = 0;
    const uint64_t t0 = trace_t0();
    switch (pp->base.kind) {
        case VBS_OP_EMBEDDING:
            ok = g_lib.embed((int)pp->type, BUF(0), U32(1), (float *)BUF(2), U32(3));
            break;
        case VBS_OP_NORMALIZE:
            ok = g_lib.rms_norm((const float *)BUF(0), (const float *)BUF(1), (float *)BUF(2), U32(3),
                                F32(4));
            break;
        case VBS_OP_ROTARY:
            ok = g_lib.rope((float *)BUF(0), U32(1), U32(2), U32(3), F32(4));
            break;
        case VBS_OP_CACHE:
            ok = g_lib.cache_store((const float *)BUF(0), (const float *)BUF(1), (uint16_t *)BUF(2),
                                   (uint16_t *)BUF(3), U32(4), U32(5), U32(6), U32(7));
            break;
        case VBS_OP_ATTENTION:
            ok = g_lib.attention((const float *)BUF(0), (const uint16_t *)BUF(1),
                                 (const uint16_t *)BUF(2), (float *)BUF(3), U32(4), U32(5), U32(6),
                                 U32(7), U32(8), U32(9), F32(10));
            break;
        case VBS_OP_ACTIVATION:
            ok = g_lib.silu_mul((const float *)BUF(0), (const float *)BUF(1), (float *)BUF(2), U32(3));
            break;
        case VBS_OP_ELEMENTWISE:
            ok = g_lib.add((const float *)BUF(0), (const float *)BUF(1), (float *)BUF(2), U32(3));
            break;
        default:
            break;
    }
    if (g_trace) {
        char d[96];
        switch (pp->base.kind) {
            case VBS_OP_EMBEDDING: snprintf(d, sizeof(d), "%s token %u dim %u", type_name(pp->type), U32(1), U32(3)); break;
            case VBS_OP_NORMALIZE: snprintf(d, sizeof(d), "%u", U32(3)); break;
            case VBS_OP_ROTARY: snprintf(d, sizeof(d), "%ux%u pos %u", U32(3), U32(2), U32(1)); break;
            case VBS_OP_CACHE: snprintf(d, sizeof(d), "%u pos %u layer %u", U32(7), U32(4), U32(5)); break;
            case VBS_OP_ATTENTION:
                snprintf(d, sizeof(d), "seq %u layer %u heads %u/%u hd %u", U32(4), U32(5), U32(7), U32(8), U32(9));
                break;
            default: snprintf(d, sizeof(d), "%u", U32(3)); break;
        }
        ok = trace_launch(tk, t0, ok, "%s", d);
    }
    return ok ? true : lib_fail("dispatch_primitive");
}

#undef BUF
#undef U32
#undef F32

static void gfx950_synchronize(vbs_device_t *dev) {
    (void)dev;
    if (g_ready && flush_pending() && !g_lib.synchronize()) lib_fail("synchronize");
}

const vbs_backend_ops_t g_vbs_hip_backend = {
    .init = gfx950_init,
    .get_device_count = gfx950_get_device_count,
    .get_device = gfx950_get_device,
    .alloc_buffer = gfx950_alloc_buffer,
    .free_buffer = gfx950_free_buffer,
    .copy_to_device = gfx950_copy_to_device,
    .copy_to_host = gfx950_copy_to_host,
    .compile_linear_pipeline = gfx950_compile_linear_pipeline,
    .compile_embed_pipeline = gfx950_compile_embed_pipeline,
    .compile_primitive_pipeline = gfx950_compile_primitive_pipeline,
    .dispatch_linear_tile = gfx950_dispatch_linear_tile,
    .dispatch_primitive = gfx950_dispatch_primitive,
    .synchronize_device = gfx950_synchronize,
    .launch_persistent_kernel = NULL,
};
