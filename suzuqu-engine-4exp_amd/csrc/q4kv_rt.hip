/*
 * q4kv_rt.hip -- device runtime shim for the QSA KV-cache path.
 *
 * Restates the part of the reference's runtime the KV path needs
 * (src/q4_rocm.cu:30-330, 6218-6227, 8162-8250, 8418-8430): one compute
 * stream, malloc/free/copies ordered on that stream, the device decode
 * position, stream capture into hipGraphs, plus pinned host buffers and
 * event timing used by the restore path and the benchmark.
 */
#include <hip/hip_runtime.h>
#include <stdlib.h>
#include <string.h>

#include "q4kv_internal.h"

extern "C" {
#include "q4kv.h"
}

hipStream_t q4kv_stream = nullptr;
int q4kv_ok = 0;
int q4kv_capturing = 0;
int32_t *q4kv_pos_d = nullptr;
float *q4kv_part = nullptr;
size_t q4kv_part_cap = 0;

/* Pinned staging ring for position pushes: a slot is rewritten only after the
 * copy that last read it has completed (its event), so pushes never block on
 * the whole stream. */
#define POS_SLOTS 16
static int32_t *g_pos_h = nullptr;
static hipEvent_t g_pos_ev[POS_SLOTS];
static int g_pos_used[POS_SLOTS];
static unsigned g_pos_next = 0;
static hipStream_t g_own_stream = nullptr; /* the stream q4_hip_init created */
static uint32_t g_last_graph_nodes = 0;

/* Split-KV partials: 8M floats (32 MiB) covers e.g. 64 sequences x 2 KV
 * heads x 33 splits x 8 heads x 258 floats. Calls needing more fall back to
 * fewer splits (q4kv_attn.hip), so this is a performance, not a correctness,
 * bound. */
#define Q4KV_PART_FLOATS (8u << 20)

/* Copy ordered after the compute stream's work: with a non-blocking stream a
 * legacy-stream hipMemcpy would not wait for queued kernels. Inside a capture
 * it becomes a memcpy node (as src/q4_rocm.cu:207-214). */
static bool sync_copy(void *dst, const void *src, size_t n, hipMemcpyKind kind) {
    if (hipMemcpyAsync(dst, src, n, kind, q4kv_stream) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (q4kv_capturing) return true;
    return hipStreamSynchronize(q4kv_stream) == hipSuccess;
}

/* Releases whatever q4_hip_init had allocated (every handle may be null). */
static void release_all(void) {
    if (q4kv_stream) (void)hipStreamSynchronize(q4kv_stream);
    if (q4kv_part) (void)hipFree(q4kv_part);
    if (q4kv_pos_d) (void)hipFree(q4kv_pos_d);
    if (g_pos_h) (void)hipHostFree(g_pos_h);
    for (int i = 0; i < POS_SLOTS; i++) {
        if (g_pos_ev[i]) (void)hipEventDestroy(g_pos_ev[i]);
        g_pos_ev[i] = nullptr;
        g_pos_used[i] = 0;
    }
    if (g_own_stream) (void)hipStreamDestroy(g_own_stream);
    g_own_stream = nullptr;
    q4kv_part = nullptr;
    q4kv_part_cap = 0;
    q4kv_pos_d = nullptr;
    g_pos_h = nullptr;
    q4kv_stream = nullptr;
    (void)hipGetLastError();
}

extern "C" bool q4_hip_init(void) {
    if (q4kv_ok) return true;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return false;
    }
    if (hipSetDevice(0) != hipSuccess) return false;
    /* on any failure below, everything allocated so far is released, so a
     * later retry starts clean */
    bool ok = hipStreamCreateWithFlags(&q4kv_stream, hipStreamNonBlocking) == hipSuccess;
    if (ok) g_own_stream = q4kv_stream;
    else q4kv_stream = nullptr;
    ok = ok && hipMalloc((void **)&q4kv_pos_d, sizeof(int32_t)) == hipSuccess;
    ok = ok && hipHostMalloc((void **)&g_pos_h, POS_SLOTS * sizeof(int32_t),
                             hipHostMallocDefault) == hipSuccess;
    for (int i = 0; ok && i < POS_SLOTS; i++) {
        ok = hipEventCreateWithFlags(&g_pos_ev[i], hipEventDisableTiming) == hipSuccess;
        g_pos_used[i] = 0;
    }
    if (ok) {
        *g_pos_h = 0;
        ok = hipMemcpy(q4kv_pos_d, g_pos_h, sizeof(int32_t), hipMemcpyHostToDevice) ==
             hipSuccess;
    }
    if (ok) {
        if (hipMalloc((void **)&q4kv_part, (size_t)Q4KV_PART_FLOATS * sizeof(float)) ==
            hipSuccess)
            q4kv_part_cap = Q4KV_PART_FLOATS;
        else {
            (void)hipGetLastError();
            q4kv_part = nullptr;
            q4kv_part_cap = 0;
        }
    }
    ok = ok && q4kv_scratch_init();
    if (!ok) {
        release_all();
        return false;
    }
    q4kv_ok = 1;
    return true;
}

extern "C" void q4_hip_shutdown(void) {
    if (!q4kv_ok) return;
    (void)q4kv_flush();
    release_all();
    q4kv_ok = 0;
}

extern "C" bool q4_hip_ok(void) { return q4kv_ok != 0; }

/* Enqueue all library work on the caller's stream (e.g. the engine's
 * compute stream, so its producers and these kernels stay ordered); NULL
 * returns to the library's own stream. Not while capturing. */
extern "C" bool q4kv_use_stream(void *stream) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || q4kv_capturing) return false;
    (void)hipStreamSynchronize(q4kv_stream);
    q4kv_stream = stream ? (hipStream_t)stream : g_own_stream;
    return true;
}

extern "C" void *q4_hip_malloc(size_t n) {
    if (!q4kv_ok || n == 0) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, n) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}

extern "C" void q4_hip_free(void *p) {
    (void)q4kv_flush();
    if (p) (void)hipFree(p);
}

extern "C" bool q4_hip_h2d(void *d, const void *h, size_t n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d || !h || n == 0) return false;
    return sync_copy(d, h, n, hipMemcpyHostToDevice);
}

extern "C" bool q4_hip_d2h(void *h, const void *d, size_t n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d || !h || n == 0) return false;
    return sync_copy(h, d, n, hipMemcpyDeviceToHost);
}

extern "C" bool q4_hip_h2d_async(void *d, const void *h, uint64_t n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d || !h || !n) return false;
    return hipMemcpyAsync(d, h, (size_t)n, hipMemcpyHostToDevice, q4kv_stream) ==
           hipSuccess;
}

extern "C" bool q4_hip_d2h_async(void *h, const void *d, uint64_t n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d || !h || !n) return false;
    return hipMemcpyAsync(h, d, (size_t)n, hipMemcpyDeviceToHost, q4kv_stream) ==
           hipSuccess;
}

/* f32 KV width store (src/q4_rocm.cu:5667-5670): a device-to-device copy
 * ordered on the compute stream that returns once it has landed, as the
 * reference's does; inside a capture it becomes a copy node. */
extern "C" bool q4_hip_copy(float *d, const float *s, uint64_t n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d || !s || !n) return false;
    return sync_copy(d, s, (size_t)n * sizeof(float), hipMemcpyDeviceToDevice);
}

extern "C" bool q4_hip_stream_sync(void) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok) return false;
    return hipStreamSynchronize(q4kv_stream) == hipSuccess;
}

extern "C" void q4_hip_sync(void) {
    (void)q4kv_flush();
    if (q4kv_ok) (void)hipDeviceSynchronize();
}

extern "C" void q4_hip_clear(void) { (void)hipGetLastError(); }

/* Pinned host memory for the session restore path (hipHostMalloc; existing
 * allocations are never registered). */
extern "C" void *q4_hip_host_alloc(size_t n) {
    if (!q4kv_ok || !n) return nullptr;
    void *p = nullptr;
    if (hipHostMalloc(&p, n, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}

extern "C" void q4_hip_host_free(void *p) {
    (void)q4kv_flush();
    if (p) (void)hipHostFree(p);
}

/* ---- device decode position (src/q4_rocm.cu:6218-6227) ---- */
extern "C" void q4_hip_pos_push(int32_t pos) {
    (void)q4kv_flush();
    if (!q4kv_pos_d || !g_pos_h || !q4kv_stream) return;
    const unsigned i = g_pos_next++ % POS_SLOTS;
    if (g_pos_used[i] && !q4kv_capturing) (void)hipEventSynchronize(g_pos_ev[i]);
    g_pos_h[i] = pos;
    (void)hipMemcpyAsync(q4kv_pos_d, g_pos_h + i, sizeof(int32_t), hipMemcpyHostToDevice,
                         q4kv_stream);
    if (!q4kv_capturing) {
        (void)hipEventRecord(g_pos_ev[i], q4kv_stream);
        g_pos_used[i] = 1;
    }
}
extern "C" int q4_hip_capturing(void) { return q4kv_capturing; }
extern "C" int q4_hip_pos_dev_ok(void) { return q4kv_pos_d != nullptr && g_pos_h != nullptr; }

/* ---- graph capture (src/q4_rocm.cu:8162-8245) ---- */
extern "C" int q4_hip_graph_begin(void) {
    if (!q4kv_ok || q4kv_capturing) return 0;
    /* an append held before the capture runs eagerly, outside the graph */
    if (!q4kv_flush()) return 0;
    if (hipStreamBeginCapture(q4kv_stream, hipStreamCaptureModeThreadLocal) !=
        hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    q4kv_capturing = 1;
    return 1;
}

extern "C" void *q4_hip_graph_end(void) {
    if (!q4kv_capturing) return nullptr;
    /* an append held inside the capture becomes a node of the graph */
    const bool flushed = q4kv_flush();
    q4kv_capturing = 0;
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture(q4kv_stream, &g) != hipSuccess || !g || !flushed) {
        (void)hipGetLastError();
        if (g) (void)hipGraphDestroy(g);
        /* A failed end can leave the stream in capture state, which fails
         * every later launch on it (the engine then re-runs the step
         * eagerly: src/q4_fwd.c:1336-1347). Replace such a stream: the
         * library's own is recreated; an adopted caller stream is dropped
         * for a new library stream. */
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(q4kv_stream, &cs) == hipSuccess &&
            cs != hipStreamCaptureStatusNone) {
            hipStream_t ns = nullptr;
            if (q4kv_stream == g_own_stream) (void)hipStreamDestroy(g_own_stream);
            g_own_stream = nullptr;
            if (hipStreamCreateWithFlags(&ns, hipStreamNonBlocking) == hipSuccess) {
                g_own_stream = q4kv_stream = ns;
                Q4KV_ERR("graph end: the stream was left capturing; replaced it");
            } else {
                q4kv_stream = nullptr;
                q4kv_ok = 0;
                Q4KV_ERR("graph end: the stream was left capturing and no new one could be made");
            }
        }
        (void)hipGetLastError();
        return nullptr;
    }
    size_t nn = 0;
    (void)hipGraphGetNodes(g, nullptr, &nn);
    g_last_graph_nodes = (uint32_t)nn;
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    (void)hipGraphUpload(ex, q4kv_stream);
    return (void *)ex;
}

extern "C" uint32_t q4_hip_graph_nodes(void *exec) {
    (void)exec;
    return g_last_graph_nodes;
}

extern "C" bool q4_hip_graph_launch(void *exec) {
    Q4KV_FLUSH_OR_FAIL();
    if (!exec) return false;
    return hipGraphLaunch((hipGraphExec_t)exec, q4kv_stream) == hipSuccess;
}

extern "C" void q4_hip_graph_free(void *exec) {
    (void)q4kv_flush();
    if (exec) (void)hipGraphExecDestroy((hipGraphExec_t)exec);
}

/* ---- event timing on the compute stream (benchmark support) ---- */
#define Q4KV_TIMERS 8
static hipEvent_t g_ev0[Q4KV_TIMERS], g_ev1[Q4KV_TIMERS];
static int g_ev_made[Q4KV_TIMERS];

extern "C" bool q4kv_timer_begin(int slot) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || slot < 0 || slot >= Q4KV_TIMERS) return false;
    if (!g_ev_made[slot]) {
        if (hipEventCreate(&g_ev0[slot]) != hipSuccess ||
            hipEventCreate(&g_ev1[slot]) != hipSuccess)
            return false;
        g_ev_made[slot] = 1;
    }
    return hipEventRecord(g_ev0[slot], q4kv_stream) == hipSuccess;
}

extern "C" double q4kv_timer_end_ms(int slot) {
    if (!q4kv_flush()) return -1;
    if (!q4kv_ok || slot < 0 || slot >= Q4KV_TIMERS || !g_ev_made[slot]) return -1.0;
    if (hipEventRecord(g_ev1[slot], q4kv_stream) != hipSuccess) return -1.0;
    if (hipEventSynchronize(g_ev1[slot]) != hipSuccess) return -1.0;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, g_ev0[slot], g_ev1[slot]) != hipSuccess) return -1.0;
    return (double)ms;
}

extern "C" int q4kv_device_info(char *name, int name_len, int *n_cu, int *clock_khz) {
    if (!q4kv_ok) return -1;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, 0) != hipSuccess) return -1;
    if (name && name_len > 0) {
        strncpy(name, p.gcnArchName, (size_t)name_len - 1);
        name[name_len - 1] = 0;
    }
    if (n_cu) *n_cu = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    return 0;
}
