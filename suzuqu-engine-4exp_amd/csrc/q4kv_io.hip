/*
 * q4kv_io.hip -- streamed session-image I/O between a file and device memory.
 *
 * The reference stages the K/V image sections through one pageable 16 MiB
 * buffer, synchronously: read, copy, read, copy (src/q4_fwd.c:2275-2294,
 * 2393-2470). Here a pipe of Q4KV_PIPE_NBUF pinned buffers moves the bytes
 * on the library stream with one event per buffer, so the file read of
 * chunk i+1 overlaps the DMA of chunk i (restore), and the device-to-host
 * copy of chunk i+1 overlaps the file write of chunk i (save). Pinned
 * buffers are allocated (hipHostMalloc), never registered.
 */
#include <hip/hip_runtime.h>
#include <errno.h>
#include <stdlib.h>
#include <unistd.h>

#include <thread>

#include "q4kv_internal.h"

extern "C" {
#include "q4kv.h"
}

#define Q4KV_PIPE_NBUF 3
/* threads per chunk of file I/O: one thread's pread/pwrite through the page
 * cache is memcpy-bound well below the host link */
#define Q4KV_PIPE_IO_THREADS 4
#define Q4KV_PIPE_IO_MIN (4u << 20) /* smaller chunks stay on one thread */

struct q4kv_pipe {
    uint8_t *buf[Q4KV_PIPE_NBUF];
    hipEvent_t ev[Q4KV_PIPE_NBUF];
    /* save: the file range each in-flight buffer still has to be written to */
    int fd[Q4KV_PIPE_NBUF];
    uint64_t off[Q4KV_PIPE_NBUF], len[Q4KV_PIPE_NBUF];
    bool busy[Q4KV_PIPE_NBUF];
    size_t chunk;
    unsigned next;
    bool failed;
};

static bool read_full(int fd, uint8_t *p, uint64_t n, uint64_t off) {
    while (n) {
        const ssize_t r = pread(fd, p, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        p += r;
        off += (uint64_t)r;
        n -= (uint64_t)r;
    }
    return true;
}

static bool write_full(int fd, const uint8_t *p, uint64_t n, uint64_t off) {
    while (n) {
        const ssize_t r = pwrite(fd, p, n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        p += r;
        off += (uint64_t)r;
        n -= (uint64_t)r;
    }
    return true;
}

/* n bytes at file offset off, split into Q4KV_PIPE_IO_THREADS contiguous
 * parts moved concurrently (the calling thread takes the first part). */
template <bool READ>
static bool io_par(int fd, uint8_t *p, uint64_t n, uint64_t off) {
    if (n < Q4KV_PIPE_IO_MIN)
        return READ ? read_full(fd, p, n, off) : write_full(fd, p, n, off);
    const uint64_t part = (n / Q4KV_PIPE_IO_THREADS + 4095u) & ~(uint64_t)4095u;
    bool ok[Q4KV_PIPE_IO_THREADS];
    std::thread th[Q4KV_PIPE_IO_THREADS];
    for (int t = 1; t < Q4KV_PIPE_IO_THREADS; t++) {
        const uint64_t b = part * t, e = b + part < n ? b + part : n;
        ok[t] = true;
        if (b >= n) continue;
        try {
            th[t] = std::thread([=, &ok] {
                ok[t] = READ ? read_full(fd, p + b, e - b, off + b)
                             : write_full(fd, p + b, e - b, off + b);
            });
        } catch (...) { /* no thread: this part runs here */
            ok[t] = READ ? read_full(fd, p + b, e - b, off + b)
                         : write_full(fd, p + b, e - b, off + b);
        }
    }
    ok[0] = READ ? read_full(fd, p, part < n ? part : n, off)
                 : write_full(fd, p, part < n ? part : n, off);
    bool all = ok[0];
    for (int t = 1; t < Q4KV_PIPE_IO_THREADS; t++) {
        if (th[t].joinable()) th[t].join();
        all = all && ok[t];
    }
    return all;
}

/* Wait for buffer i's copy; for a pending save, write its bytes out. */
static bool retire(q4kv_pipe *p, unsigned i) {
    if (!p->busy[i]) return true;
    p->busy[i] = false;
    if (hipEventSynchronize(p->ev[i]) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (p->fd[i] >= 0 && !io_par<false>(p->fd[i], p->buf[i], p->len[i], p->off[i])) return false;
    return true;
}

extern "C" q4kv_pipe *q4kv_pipe_open(size_t chunk) {
    if (!q4kv_flush()) return nullptr;
    if (!q4kv_ok || chunk == 0) return nullptr;
    q4kv_pipe *p = (q4kv_pipe *)calloc(1, sizeof(q4kv_pipe));
    if (!p) return nullptr;
    p->chunk = chunk;
    for (int i = 0; i < Q4KV_PIPE_NBUF; i++) {
        p->fd[i] = -1;
        if (hipHostMalloc((void **)&p->buf[i], chunk, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&p->ev[i], hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            q4kv_pipe_close(p);
            return nullptr;
        }
    }
    return p;
}

extern "C" bool q4kv_pipe_finish(q4kv_pipe *p) {
    Q4KV_FLUSH_OR_FAIL();
    if (!p) return false;
    bool ok = !p->failed;
    for (unsigned k = 0; k < Q4KV_PIPE_NBUF; k++)
        ok = retire(p, (p->next + k) % Q4KV_PIPE_NBUF) && ok; /* oldest first */
    p->failed = false;
    return ok;
}

extern "C" void q4kv_pipe_close(q4kv_pipe *p) {
    (void)q4kv_flush();
    if (!p) return;
    (void)q4kv_pipe_finish(p);
    for (int i = 0; i < Q4KV_PIPE_NBUF; i++) {
        if (p->buf[i]) (void)hipHostFree(p->buf[i]);
        if (p->ev[i]) (void)hipEventDestroy(p->ev[i]);
    }
    free(p);
}

extern "C" bool q4kv_pipe_file_to_dev(q4kv_pipe *p, int fd, uint64_t off, void *dst,
                                      uint64_t n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!p || fd < 0 || !dst || p->failed) return false;
    uint8_t *d = (uint8_t *)dst;
    for (uint64_t o = 0; o < n; o += p->chunk) {
        const uint64_t len = n - o < p->chunk ? n - o : p->chunk;
        const unsigned i = p->next++ % Q4KV_PIPE_NBUF;
        if (!retire(p, i) || !io_par<true>(fd, p->buf[i], len, off + o) ||
            hipMemcpyAsync(d + o, p->buf[i], len, hipMemcpyHostToDevice, q4kv_stream) !=
                hipSuccess ||
            hipEventRecord(p->ev[i], q4kv_stream) != hipSuccess) {
            (void)hipGetLastError();
            p->failed = true;
            return false;
        }
        p->fd[i] = -1;
        p->busy[i] = true;
    }
    return true;
}

extern "C" bool q4kv_pipe_dev_to_file(q4kv_pipe *p, int fd, uint64_t off, const void *src,
                                      uint64_t n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!p || fd < 0 || !src || p->failed) return false;
    const uint8_t *s = (const uint8_t *)src;
    for (uint64_t o = 0; o < n; o += p->chunk) {
        const uint64_t len = n - o < p->chunk ? n - o : p->chunk;
        const unsigned i = p->next++ % Q4KV_PIPE_NBUF;
        if (!retire(p, i) ||
            hipMemcpyAsync(p->buf[i], s + o, len, hipMemcpyDeviceToHost, q4kv_stream) !=
                hipSuccess ||
            hipEventRecord(p->ev[i], q4kv_stream) != hipSuccess) {
            (void)hipGetLastError();
            p->failed = true;
            return false;
        }
        p->fd[i] = fd;
        p->off[i] = off + o;
        p->len[i] = len;
        p->busy[i] = true;
    }
    return true;
}
