// vbs_gfx950_rt.hip — runtime and C-ABI entry points of libvbs_gfx950.so
// (declared in include/vbs_gfx950.h).
//
// One device, one in-order stream. Entry points validate their arguments on
// the host (types, shapes, null pointers, head/group limits) before anything
// is launched, record the reason of any failure in a last-error string and
// return 0; nothing aborts across the C ABI.
#include <math.h>
#include <stdarg.h>
#include <vector>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <thread>

#include "vbs_dev_common.h"
#include "vbs_gfx950.h"
#include "vbs_internal.h"

// Partial results of vbs_gfx950_attention_noalloc: a fixed device array, so
// that entry point allocates nothing. Its device address is looked up once,
// at vbs_gfx950_init with the library's device current; host code uses only
// that address (the array's name is a host-side stand-in). Every call on the
// device shares it, and calls that overlap on the device would race; the
// library orders all its work on one stream, so its own calls never overlap.
constexpr size_t kNoAllocScratchBytes = 8u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxRetired = 48;

struct Runtime {
    bool probed = false;
    bool ready = false;
    int device = -1;
    hipStream_t stream = nullptr;
    char name[128] = {0};
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    void *retired[kMaxRetired] = {nullptr};  // superseded scratch buffers, kept (see rt_scratch)
    int n_retired = 0;
    void *noalloc_scratch = nullptr;  // device address of `scratch` on the library's device
};

Runtime g_rt;
char g_err[512] = "not initialised";

int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return 0;
}

int hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return 1;
    return fail("%s: %s", what, hipGetErrorString(e));
}

bool ready_or_fail() {
    if (g_rt.ready) return true;
    if (!g_rt.probed) vbs_gfx950_init();
    if (!g_rt.ready) {
        if (!g_rt.probed) fail("vbs_gfx950_init has not succeeded");
        return false;
    }
    return true;
}

}  // namespace

namespace vbs {

uint32_t block_elems(int type) {
    switch (type) {
        case kF32: case kF16: return 1;
        case kQ4_0: case kQ4_1: case kQ8_0: case kLNS8: return 32;
        case kQ4_K: case kQ6_K: return 256;
        default: return 0;
    }
}

uint64_t row_bytes(int type, uint32_t cols) {
    switch (type) {
        case kF32: return 4ull * cols;
        case kF16: return 2ull * cols;
        case kQ4_0: return 18ull * (cols / 32u);
        case kQ4_1: return 20ull * (cols / 32u);
        case kQ8_0: return 34ull * (cols / 32u);
        case kQ4_K: return 144ull * (cols / 256u);
        case kQ6_K: return 210ull * (cols / 256u);
        case kLNS8: return 36ull * (cols / 32u);
        default: return 0;
    }
}

// The scratch only grows, and a buffer that a larger one replaces stays
// allocated until the process ends: a graph captured from the library's
// stream keeps the address it was captured with, and a replay after a larger
// call must still find valid memory there. Every growth at least doubles the
// size, so the retired buffers together are smaller than the live one (and
// 48 retirements are more than any 64-bit size allows). Growing allocates,
// which a stream under capture must not do: such a call fails with
// hipErrorStreamCaptureUnsupported and nothing is launched; one uncaptured
// call of the same size first sizes the scratch for later captures.
void *rt_scratch(size_t bytes, hipStream_t s, hipError_t *why) {
    *why = hipSuccess;
    if (bytes <= g_rt.scratch_bytes) return g_rt.scratch;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        *why = hipErrorStreamCaptureUnsupported;
        return nullptr;
    }
    if (g_rt.n_retired == kMaxRetired) {
        *why = hipErrorOutOfMemory;
        return nullptr;
    }
    size_t want = bytes < 2 * g_rt.scratch_bytes ? 2 * g_rt.scratch_bytes : bytes;
    want = want < (1u << 20) ? (1u << 20) : want;
    want = (want + 4095u) & ~(size_t)4095u;
    void *p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
        (void)hipGetLastError();
        *why = hipErrorOutOfMemory;
        return nullptr;
    }
    if (g_rt.scratch) g_rt.retired[g_rt.n_retired++] = g_rt.scratch;
    g_rt.scratch = p;
    g_rt.scratch_bytes = want;
    return p;
}

hipStream_t rt_stream() { return g_rt.stream; }



int rt_fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return 0;
}

int rt_hip_ok(hipError_t e, const char *what) { return hip_ok(e, what); }

bool rt_ready() { return ready_or_fail(); }

}  // namespace vbs

using namespace vbs;

extern "C" {

int vbs_gfx950_abi_version(void) { return VBS_GFX950_ABI_VERSION; }

const char *vbs_gfx950_last_error(void) { return g_err; }

int vbs_gfx950_init(void) {
    if (g_rt.probed) return g_rt.ready ? 1 : 0;
    g_rt.probed = true;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0)
        return fail("no AMD GPU visible to the HIP runtime (%s)",
                    e == hipSuccess ? "0 devices" : hipGetErrorString(e));
    int chosen = -1;
    for (int i = 0; i < count && chosen < 0; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) != hipSuccess) continue;
        if (strncmp(p.gcnArchName, "gfx950", 6) == 0) {
            chosen = i;
            snprintf(g_rt.name, sizeof(g_rt.name), "AMD %s (%s, %d CUs)", p.name, p.gcnArchName,
                     p.multiProcessorCount);
        }
    }
    if (chosen < 0) return fail("no gfx950 (MI355X) device among %d visible GPUs", count);
    if (!hip_ok(hipSetDevice(chosen), "hipSetDevice")) return 0;
    if (!hip_ok(hipStreamCreateWithFlags(&g_rt.stream, hipStreamNonBlocking), "hipStreamCreate"))
        return 0;
    if (!hip_ok(hipGetSymbolAddress(&g_rt.noalloc_scratch, HIP_SYMBOL(scratch)),
                "hipGetSymbolAddress(scratch)"))
        return 0;
    if (!hip_ok(hipDeviceSynchronize(), "init")) return 0;
    g_rt.device = chosen;
    g_rt.ready = true;
    snprintf(g_err, sizeof(g_err), "ok");
    return 1;
}

int vbs_gfx950_device_count(void) { return g_rt.ready ? 1 : 0; }

int vbs_gfx950_device_info(int index, char *name, size_t cap, uint64_t *total, uint64_t *free_b) {
    if (!ready_or_fail()) return 0;
    if (index != 0) return fail("device index %d out of range (1 device)", index);
    if (name && cap) snprintf(name, cap, "%s", g_rt.name);
    size_t fr = 0, tot = 0;
    if (!hip_ok(hipMemGetInfo(&fr, &tot), "hipMemGetInfo")) return 0;
    if (total) *total = tot;
    if (free_b) *free_b = fr;
    return 1;
}

void *vbs_gfx950_alloc(size_t bytes) {
    if (!ready_or_fail()) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
        fail("hipMalloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

int vbs_gfx950_free(void *p) {
    if (!p) return 1;
    if (!ready_or_fail()) return 0;
    (void)hipStreamSynchronize(g_rt.stream);
    return hip_ok(hipFree(p), "hipFree");
}

void *vbs_gfx950_host_alloc(size_t bytes) {
    if (!ready_or_fail()) return nullptr;
    void *p = nullptr;
    if (hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault) != hipSuccess) {
        fail("hipHostMalloc(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

int vbs_gfx950_host_free(void *p) {
    if (!p) return 1;
    if (!ready_or_fail()) return 0;
    (void)hipStreamSynchronize(g_rt.stream);
    return hip_ok(hipHostFree(p), "hipHostFree");
}

// Pageable host memory reaches the device through two pinned staging
// buffers: while the DMA engine copies chunk k out of one, host threads fill
// the other with chunk k+1. (The runtime's own path for pageable sources ran
// at about half the pinned DMA rate on MI355X hosts: 28.8 vs 57.6 GB/s.)
constexpr size_t kStageChunk = 32u << 20;
constexpr size_t kStagedMin = 16u << 20;
constexpr unsigned kCopyThreads = 8;

struct Staging {
    void *buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool tried = false, ok = false;
    std::mutex lock;  // one staged copy at a time (the buffers are shared)
};
static Staging g_stage;

static bool staging_ready() {  // called with g_stage.lock held
    if (g_stage.tried) return g_stage.ok;
    g_stage.tried = true;
    for (int i = 0; i < 2; i++) {
        if (hipHostMalloc(&g_stage.buf[i], kStageChunk, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&g_stage.done[i], hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            return false;  // the direct path stays in use
        }
    }
    g_stage.ok = true;
    return true;
}

static bool host_pinned(const void *p) {
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();  // pageable memory: not known to the runtime
        return false;
    }
    return a.type == hipMemoryTypeHost;
}

// memcpy split over up to kCopyThreads host threads (page-aligned slices).
static void parallel_copy(void *dst, const void *src, size_t n) {
    unsigned nt = std::thread::hardware_concurrency();
    nt = nt == 0 ? 1 : nt > kCopyThreads ? kCopyThreads : nt;
    if (nt == 1 || n < (4u << 20)) {
        memcpy(dst, src, n);
        return;
    }
    const size_t per = ((n + nt - 1) / nt + 4095u) & ~(size_t)4095u;
    std::thread th[kCopyThreads];
    unsigned used = 0;
    for (unsigned t = 1; t < nt && per * t < n; t++) {
        const size_t off = per * t, len = n - off < per ? n - off : per;
        try {
            th[used] = std::thread([=] { memcpy((char *)dst + off, (const char *)src + off, len); });
            used++;
        } catch (...) {  // no thread to spare: copy the rest here (no exception leaves the C ABI)
            memcpy((char *)dst + off, (const char *)src + off, n - off);
            break;
        }
    }
    memcpy(dst, src, n < per ? n : per);
    for (unsigned i = 0; i < used; i++) th[i].join();
}

static int copy_h2d_staged(void *dst, const void *src, size_t bytes) {
    const char *s = (const char *)src;
    char *d = (char *)dst;
    int ok = 1;
    for (size_t off = 0, k = 0; off < bytes && ok; k++) {
        const int slot = (int)(k & 1u);
        const size_t n = bytes - off < kStageChunk ? bytes - off : kStageChunk;
        if (k >= 2) ok = hip_ok(hipEventSynchronize(g_stage.done[slot]), "copy_h2d");
        if (!ok) break;
        parallel_copy(g_stage.buf[slot], s + off, n);
        ok = hip_ok(hipMemcpyAsync(d + off, g_stage.buf[slot], n, hipMemcpyHostToDevice,
                                   g_rt.stream), "copy_h2d") &&
             hip_ok(hipEventRecord(g_stage.done[slot], g_rt.stream), "copy_h2d");
        off += n;
    }
    // every staged chunk has left its buffer before the buffers are reused
    const hipError_t e = hipStreamSynchronize(g_rt.stream);
    return ok && hip_ok(e, "copy_h2d");
}

static int copy_sync(void *dst, const void *src, size_t bytes, hipMemcpyKind kind,
                     const char *what) {
    if (!ready_or_fail()) return 0;
    if (bytes == 0) return 1;
    if (!dst || !src) return fail("%s: null pointer", what);
    if (!hip_ok(hipMemcpyAsync(dst, src, bytes, kind, g_rt.stream), what)) return 0;
    return hip_ok(hipStreamSynchronize(g_rt.stream), what);
}

int vbs_gfx950_copy_h2d(void *dst, const void *src, size_t bytes) {
    if (bytes >= kStagedMin && dst && src && ready_or_fail() && !host_pinned(src)) {
        std::lock_guard<std::mutex> hold(g_stage.lock);
        if (staging_ready()) return copy_h2d_staged(dst, src, bytes);
    }
    return copy_sync(dst, src, bytes, hipMemcpyHostToDevice, "copy_h2d");
}
int vbs_gfx950_copy_d2h(void *dst, const void *src, size_t bytes) {
    return copy_sync(dst, src, bytes, hipMemcpyDeviceToHost, "copy_d2h");
}
int vbs_gfx950_copy_d2d(void *dst, const void *src, size_t bytes) {
    if (!ready_or_fail()) return 0;
    if (bytes == 0) return 1;
    if (!dst || !src) return fail("copy_d2d: null pointer");
    return hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_rt.stream),
                  "copy_d2d");
}

int vbs_gfx950_synchronize(void) {
    if (!ready_or_fail()) return 0;
    return hip_ok(hipStreamSynchronize(g_rt.stream), "synchronize");
}

void *vbs_gfx950_stream(void) { return g_rt.ready ? (void *)g_rt.stream : nullptr; }

int vbs_gfx950_linear_supported(int type) { return block_elems(type) != 0; }

int vbs_gfx950_linear(int type, const void *w, const float *x, float *y, uint32_t cols,
                      uint32_t rows, uint32_t col_off, uint32_t row_off, int accumulate) {
    if (!ready_or_fail()) return 0;
    uint32_t e = block_elems(type);
    if (!e) return fail("linear: no gfx950 kernel for weight type %d", type);
    if (cols % e) return fail("linear: cols %u is not a multiple of the block size %u", cols, e);
    if (!w || !x || !y) return fail("linear: null pointer");
    return hip_ok(launch_linear(type, (const uint8_t *)w, x + col_off, y + row_off, cols, rows,
                                accumulate, g_rt.stream),
                  "linear");
}

// RoPE rows of the fused linear: (cos, sin) of every pair angle for positions
// [0, n_pos) at one (theta, head_dim), computed with the host libm as
// vbs_gfx950_rope does, and the positions 0 .. n_pos - 1 themselves (the
// kernels read the position through a device pointer). Rebuilt, twice as
// long, when a call needs a later position; the previous tables are freed
// after the stream drains (this path is never captured).
struct RopeRows {
    float theta = 0.f;
    uint32_t hd = 0, n_pos = 0;
    float2 *tab = nullptr;
    uint32_t *pos = nullptr;
};
static RopeRows g_rope;

static bool rope_rows(float theta, uint32_t hd, uint32_t pos) {
    if (g_rope.tab && g_rope.theta == theta && g_rope.hd == hd && pos < g_rope.n_pos) return true;
    uint32_t n = 4096;
    while (n <= pos) n *= 2u;
    if (g_rope.tab && g_rope.theta == theta && g_rope.hd == hd && n < 2u * g_rope.n_pos)
        n = 2u * g_rope.n_pos;
    const uint32_t pairs = hd / 2u;
    std::vector<float2> tab((size_t)n * pairs);
    std::vector<uint32_t> ids(n);
    for (uint32_t p = 0; p < n; p++) {
        ids[p] = p;
        for (uint32_t pr = 0; pr < pairs; pr++) {
            const float angle = (float)p * powf(theta, -(float)(2u * pr) / (float)hd);
            tab[(size_t)p * pairs + pr] = make_float2(cosf(angle), sinf(angle));
        }
    }
    float2 *t = nullptr;
    uint32_t *ip = nullptr;
    if (hipMalloc(&t, tab.size() * sizeof(float2)) != hipSuccess ||
        hipMalloc(&ip, ids.size() * sizeof(uint32_t)) != hipSuccess ||
        hipMemcpyAsync(t, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice,
                       g_rt.stream) != hipSuccess ||
        hipMemcpyAsync(ip, ids.data(), ids.size() * sizeof(uint32_t), hipMemcpyHostToDevice,
                       g_rt.stream) != hipSuccess ||
        hipStreamSynchronize(g_rt.stream) != hipSuccess) {
        if (t) (void)hipFree(t);
        if (ip) (void)hipFree(ip);
        return false;
    }
    if (g_rope.tab) (void)hipFree(g_rope.tab);
    if (g_rope.pos) (void)hipFree(g_rope.pos);
    g_rope = RopeRows{theta, hd, n, t, ip};
    return true;
}

int vbs_gfx950_linear_fused(int type, const void *w, const float *x, float *y, uint32_t cols,
                            uint32_t rows, const vbs_gfx950_linear_join_t *join) {
    if (!ready_or_fail()) return 0;
    if (!w || !x || !y || !join) return fail("linear_fused: null pointer");
    const vbs_gfx950_linear_join_t &jn = *join;
    if ((jn.norm_w != nullptr) != (jn.x_normed != nullptr))
        return fail("linear_fused: the RMSNorm needs both its weights and its output");
    if ((jn.gate != nullptr) != (jn.hidden != nullptr))
        return fail("linear_fused: the activation needs both its gate and its output");
    if ((jn.k_row != nullptr) != (jn.kc != nullptr) || (jn.k_row != nullptr) != (jn.vc != nullptr))
        return fail("linear_fused: the cache store needs the k row and both caches");
    if (type != kQ4_K && type != kQ6_K) return 2;
    if (cols % 256u || rows == 0) return 2;
    const int n_after = (jn.acc != nullptr) + (jn.rope != 0) + (jn.gate != nullptr) +
                        (jn.k_row != nullptr);
    if (n_after > 1 || (!n_after && !jn.norm_w)) return 2;
    if (jn.norm_w && n_after && !jn.rope) return 2;
    LinJoin lj;
    lj.norm_w = jn.norm_w;
    lj.eps = jn.norm_eps;
    lj.xn = jn.x_normed;
    if (jn.rope) {
        if (jn.head_dim == 0 || (jn.head_dim & 3u) || jn.head_dim > 256u || rows % jn.head_dim)
            return 2;
        if (!rope_rows(jn.theta, jn.head_dim, jn.pos))
            return fail("linear_fused: RoPE table allocation failed");
        lj.rope = g_rope.tab;
        lj.pos = g_rope.pos + jn.pos;
        lj.hd = jn.head_dim;
    }
    lj.gate_in = jn.gate;
    lj.hid = jn.hidden;
    lj.kin = jn.k_row;
    lj.kc = jn.kc;
    lj.vc = jn.vc;
    lj.kv_off = jn.kv_off;
    // with the add, the kernels accumulate into acc and copy the row values to y
    float *dst = y;
    if (jn.acc) {
        dst = jn.acc;
        lj.ycopy = y;
    }
    const hipError_t e = launch_kq_linear_fused(type, (const uint8_t *)w, x, dst, cols, rows, lj,
                                                g_rt.stream);
    if (e == hipErrorNotSupported) return 2;
    return hip_ok(e, "linear_fused");
}

int vbs_gfx950_qkv_fused(int type, const void *wq, const void *wk, const void *wv, const float *x,
                         uint32_t cols, uint32_t q_rows, uint32_t kv_rows, const float *norm_w,
                         float eps, float *x_normed, float *q, float *k, float *v, uint32_t pos,
                         uint32_t head_dim, float theta, uint16_t *kc, uint16_t *vc,
                         uint32_t layer, uint32_t max_ctx) {
    if (!ready_or_fail()) return 0;
    if (!wq || !wk || !wv || !x || !q || !k || !v || !kc || !vc)
        return fail("qkv_fused: null pointer");
    if ((norm_w != nullptr) != (x_normed != nullptr))
        return fail("qkv_fused: the RMSNorm needs both its weights and its output");
    if (pos >= max_ctx) return fail("qkv_fused: pos %u >= max_ctx %u", pos, max_ctx);
    if (type != kQ4_K && type != kQ6_K) return 2;
    if (cols % 256u || q_rows == 0 || kv_rows == 0 || q_rows % 16u || kv_rows % 16u) return 2;
    if (head_dim == 0 || (head_dim & 3u) || head_dim > 256u || q_rows % head_dim ||
        kv_rows % head_dim)
        return 2;
    if (!rope_rows(theta, head_dim, pos)) return fail("qkv_fused: RoPE table allocation failed");
    const uint8_t *w[3] = {(const uint8_t *)wq, (const uint8_t *)wk, (const uint8_t *)wv};
    const uint32_t rows[3] = {q_rows, kv_rows, kv_rows};
    GroupOut out;
    out.xn = x_normed;
    out.k = k;
    out.v = v;
    const hipError_t e = launch_kq_qkv(type, w, 3, 0, x, norm_w, eps, cols, rows, q, kc, vc,
                                       (uint64_t)layer * max_ctx * kv_rows, kv_rows, g_rope.tab,
                                       g_rope.pos + pos, head_dim, g_rt.stream, out);
    if (e == hipErrorNotSupported) return 2;
    return hip_ok(e, "qkv_fused");
}

int vbs_gfx950_gate_up_fused(int type, const void *wg, const void *wu, const float *x,
                             uint32_t cols, uint32_t rows, const float *norm_w, float eps,
                             float *x_normed, float *gate, float *up, float *hidden) {
    if (!ready_or_fail()) return 0;
    if (!wg || !wu || !x || !gate || !up || !hidden) return fail("gate_up_fused: null pointer");
    if ((norm_w != nullptr) != (x_normed != nullptr))
        return fail("gate_up_fused: the RMSNorm needs both its weights and its output");
    if (type != kQ4_K && type != kQ6_K) return 2;
    if (cols % 256u || rows == 0 || rows % 16u) return 2;
    GroupOut out;
    out.xn = x_normed;
    out.gate = gate;
    out.up = up;
    const hipError_t e = launch_kq_silu(type, (const uint8_t *)wg, (const uint8_t *)wu, x, norm_w,
                                        eps, cols, rows, hidden, g_rt.stream, out);
    if (e == hipErrorNotSupported) return 2;
    return hip_ok(e, "gate_up_fused");
}

int vbs_gfx950_linear_batch(int type, const void *w, const float *x, uint32_t x_stride, float *y,
                            uint32_t y_stride, uint32_t cols, uint32_t rows, uint32_t batch) {
    if (!ready_or_fail()) return 0;
    uint32_t e = block_elems(type);
    if (!e) return fail("linear_batch: no gfx950 kernel for weight type %d", type);
    if (cols % e) return fail("linear_batch: cols %u not a multiple of %u", cols, e);
    if (batch > 16) return fail("linear_batch: batch %u exceeds 16", batch);
    if (x_stride < cols || y_stride < rows) return fail("linear_batch: stride smaller than row");
    if (!w || !x || !y) return fail("linear_batch: null pointer");
    return hip_ok(launch_linear_batch(type, (const uint8_t *)w, x, x_stride, y, y_stride, cols,
                                      rows, batch, g_rt.stream),
                  "linear_batch");
}

int vbs_gfx950_linear_batch_multi(int type, uint32_t n_mat, const void *const *w,
                                  const uint32_t *rows, const float *x, uint32_t x_stride,
                                  float *const *y, const uint32_t *y_stride, uint32_t cols,
                                  uint32_t batch) {
    if (!ready_or_fail()) return 0;
    uint32_t e = block_elems(type);
    if (!e) return fail("linear_batch_multi: no gfx950 kernel for weight type %d", type);
    if (cols % e) return fail("linear_batch_multi: cols %u not a multiple of %u", cols, e);
    if (n_mat == 0 || n_mat > 3) return fail("linear_batch_multi: %u matrices (1-3)", n_mat);
    if (batch > 16) return fail("linear_batch_multi: batch %u exceeds 16", batch);
    if (!w || !rows || !x || !y || !y_stride) return fail("linear_batch_multi: null pointer");
    if (x_stride < cols) return fail("linear_batch_multi: x stride smaller than a row");
    const uint8_t *wm[3];
    float *ym[3];
    uint32_t rm[3], ysm[3];
    for (uint32_t m = 0; m < n_mat; m++) {
        if (!w[m] || !y[m]) return fail("linear_batch_multi: null pointer for matrix %u", m);
        if (y_stride[m] < rows[m]) return fail("linear_batch_multi: y stride of matrix %u smaller than its rows", m);
        wm[m] = (const uint8_t *)w[m];
        ym[m] = y[m];
        rm[m] = rows[m];
        ysm[m] = y_stride[m];
    }
    return hip_ok(launch_linear_batch_multi(type, n_mat, wm, rm, x, x_stride, ym, ysm, cols, batch,
                                            g_rt.stream),
                  "linear_batch_multi");
}

int vbs_gfx950_embed(int type, const void *w, uint32_t token, float *out, uint32_t dim) {
    if (!ready_or_fail()) return 0;
    uint32_t e = block_elems(type);
    if (!e) return fail("embed: no gfx950 kernel for weight type %d", type);
    if (dim % e) return fail("embed: dim %u not a multiple of the block size %u", dim, e);
    if (!w || !out) return fail("embed: null pointer");
    if (token == 0xFFFFFFFFu) return fail("embed: token id out of range");
    return hip_ok(launch_dequant_rows(type, (const uint8_t *)w, nullptr, token, 1, dim, out,
                                      g_rt.stream),
                  "embed");
}

int vbs_gfx950_dequant_rows(int type, const void *w, const uint32_t *ids, uint32_t n_rows,
                            uint32_t dim, float *out) {
    if (!ready_or_fail()) return 0;
    uint32_t e = block_elems(type);
    if (!e) return fail("dequant_rows: no decoder for weight type %d", type);
    if (dim % e) return fail("dequant_rows: dim %u not a multiple of %u", dim, e);
    if (n_rows > 65535u) return fail("dequant_rows: at most 65535 rows per call");
    if (!w || !out) return fail("dequant_rows: null pointer");
    return hip_ok(launch_dequant_rows(type, (const uint8_t *)w, ids, 0xFFFFFFFFu, n_rows, dim,
                                      out, g_rt.stream),
                  "dequant_rows");
}

int vbs_gfx950_rms_norm(const float *in, const float *w, float *out, uint32_t dim, float eps) {
    if (!ready_or_fail()) return 0;
    if (!in || !w || !out) return fail("rms_norm: null pointer");
    return hip_ok(launch_rms_norm(in, w, out, dim, eps, g_rt.stream), "rms_norm");
}

int vbs_gfx950_rope(float *x, uint32_t pos, uint32_t head_dim, uint32_t n_heads, float theta) {
    if (!ready_or_fail()) return 0;
    if (!x || head_dim == 0 || n_heads == 0) return fail("rope: null pointer or empty shape");
    if (head_dim > 512) return fail("rope: head_dim %u exceeds 512", head_dim);
    // Pair angles with the host libm, exactly as src/vbs_host_math.h:43-44.
    float cs[512];
    for (uint32_t i = 0; i + 1 < head_dim; i += 2) {
        float angle = (float)pos * powf(theta, -(float)i / (float)head_dim);
        cs[i] = cosf(angle);
        cs[i + 1] = sinf(angle);
    }
    return hip_ok(launch_rope(x, head_dim, n_heads, cs, g_rt.stream), "rope");
}

int vbs_gfx950_cache_store(const float *k, const float *v, uint16_t *kc, uint16_t *vc,
                           uint32_t pos, uint32_t layer, uint32_t max_ctx, uint32_t kv_dim) {
    if (!ready_or_fail()) return 0;
    if (!k || !v || !kc || !vc) return fail("cache_store: null pointer");
    if (pos >= max_ctx) return fail("cache_store: pos %u >= max_ctx %u", pos, max_ctx);
    uint64_t base = ((uint64_t)layer * max_ctx + pos) * kv_dim;
    return hip_ok(launch_cache_store(k, v, kc, vc, base, kv_dim, g_rt.stream), "cache_store");
}

// Argument checks shared by both attention entry points; 0 with the reason set.
static int attention_args_ok(const char *who, const float *q, const uint16_t *kc,
                             const uint16_t *vc, const float *out, uint32_t seq_len,
                             uint32_t max_ctx, uint32_t nqh, uint32_t nkh, uint32_t hd) {
    if (!q || !kc || !vc || !out) return fail("%s: null pointer", who);
    if (seq_len == 0 || nqh == 0 || nkh == 0 || hd == 0) return fail("%s: empty shape", who);
    if (seq_len > max_ctx) return fail("%s: seq_len %u > max_ctx %u", who, seq_len, max_ctx);
    if (nqh % nkh) return fail("%s: %u q heads not a multiple of %u kv heads", who, nqh, nkh);
    if (nqh / nkh > 16) return fail("%s: group size %u exceeds 16", who, nqh / nkh);
    if (hd > 256 || (hd & 1u)) return fail("%s: head_dim %u must be even and <= 256", who, hd);
    return 1;
}

int vbs_gfx950_attention(const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                         uint32_t seq_len, uint32_t layer, uint32_t max_ctx, uint32_t nqh,
                         uint32_t nkh, uint32_t hd, float scale) {
    if (!ready_or_fail()) return 0;
    if (!attention_args_ok("attention", q, kc, vc, out, seq_len, max_ctx, nqh, nkh, hd)) return 0;
    uint64_t layer_off = (uint64_t)layer * max_ctx * nkh * hd;
    return hip_ok(launch_attention(q, kc, vc, out, seq_len, nullptr, nullptr, layer_off, nqh, nkh,
                                   hd, scale, g_rt.stream),
                  "attention");
}

int vbs_gfx950_attention_noalloc(const float *q, const uint16_t *kc, const uint16_t *vc,
                                 float *out, uint32_t seq_len, uint32_t layer, uint32_t max_ctx,
                                 uint32_t nqh, uint32_t nkh, uint32_t hd, float scale) {
    if (!ready_or_fail()) return 0;
    if (!attention_args_ok("attention_noalloc", q, kc, vc, out, seq_len, max_ctx, nqh, nkh, hd))
        return 0;
    const size_t need = attention_partial_bytes(seq_len, nqh, nkh, hd);
    if (need > kNoAllocScratchBytes)
        return fail("attention_noalloc: %zu bytes of partial results (seq_len %u, %u q heads, "
                    "%u kv heads, head_dim %u) exceed its fixed %zu-byte scratch",
                    need, seq_len, nqh, nkh, hd, kNoAllocScratchBytes);
    // every partial the merge reads is written by the same call's chunk
    // kernels first, so the scratch needs no clearing between calls
    uint64_t layer_off = (uint64_t)layer * max_ctx * nkh * hd;
    return hip_ok(launch_attention(q, kc, vc, out, seq_len, nullptr,
                                   static_cast<float *>(g_rt.noalloc_scratch), layer_off, nqh,
                                   nkh, hd, scale, g_rt.stream),
                  "attention_noalloc");
}

uint32_t vbs_gfx950_checksum_partials(size_t bytes) { return checksum_partials(bytes); }

uint32_t vbs_gfx950_checksum_variant_partials(size_t bytes, int variant) {
    return variant >= 0 && variant <= 2 ? checksum_partials(bytes, variant) : 0u;
}

int vbs_gfx950_checksum_variant(const void *p, size_t bytes, uint32_t *partials, int variant) {
    if (!ready_or_fail()) return 0;
    if (variant < 0 || variant > 2) return fail("checksum: variant %d outside 0..2", variant);
    if (bytes == 0) return 1;
    if (!p || !partials) return fail("checksum: null pointer");
    if ((bytes & 15u) || ((uintptr_t)p & 15u))
        return fail("checksum: region must be 16-byte aligned and a multiple of 16 bytes");
    return hip_ok(launch_checksum(static_cast<const uint8_t *>(p), bytes, partials, variant,
                                  g_rt.stream),
                  "checksum");
}

int vbs_gfx950_checksum(const void *p, size_t bytes, uint32_t *partials) {
    return vbs_gfx950_checksum_variant(p, bytes, partials, 0);
}

int vbs_gfx950_silu_mul(const float *g, const float *u, float *out, uint32_t n) {
    if (!ready_or_fail()) return 0;
    if (!g || !u || !out) return fail("silu_mul: null pointer");
    return hip_ok(launch_silu_mul(g, u, out, n, g_rt.stream), "silu_mul");
}

int vbs_gfx950_add(const float *a, const float *b, float *out, uint32_t n) {
    if (!ready_or_fail()) return 0;
    if (!a || !b || !out) return fail("add: null pointer");
    return hip_ok(launch_add(a, b, out, n, g_rt.stream), "add");
}

}  // extern "C"
