/*
 * q4kv_host.c -- host-side KV-cache layer (C) above the q4kv C ABI.
 *
 * Restates the KV-cache portions of the reference's src/q4_fwd.c: the width
 * switch, cache allocation and addressing, kv_write, the decode append and
 * attention call sites, and the K/V section of the session image.
 */
#define _POSIX_C_SOURCE 200809L
#include "q4kv_host.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <fcntl.h>
#include <unistd.h>

int q4kv_kind_of(const char *e) {
    if (!e) e = getenv("Q4_KV");
    if (e && (!strcmp(e, "f32") || !strcmp(e, "fp32"))) return Q4KV_F32;
    if (e && (!strcmp(e, "f16") || !strcmp(e, "fp16"))) return Q4KV_F16;
    return Q4KV_Q8;
}

uint32_t q4kv_token_bytes(int kind, uint32_t n_kvh, uint32_t hd) {
    const uint32_t kvw = n_kvh * hd;
    if (kind == Q4KV_Q8) return (kvw / 32u) * 34u;
    return kvw * (kind == Q4KV_F16 ? 2u : 4u);
}

uint64_t q4kv_cache_bytes(int kind, uint32_t n_layer, uint32_t n_kvh, uint32_t hd,
                          uint32_t ctx) {
    return 2ull * n_layer * (uint64_t)ctx * q4kv_token_bytes(kind, n_kvh, hd);
}

uint32_t q4kv_tag(int kind) { return kind == Q4KV_Q8 ? 8u : kind == Q4KV_F16 ? 2u : 4u; }

bool q4kv_cache_open(q4kv_cache *c, int kind, uint32_t n_layer, uint32_t n_kvh, uint32_t hd,
                     uint32_t max_kv) {
    if (!c || !n_layer || !n_kvh || !hd || !max_kv || kind < Q4KV_F32 || kind > Q4KV_Q8)
        return false;
    if (kind == Q4KV_Q8 && (n_kvh * hd) % 32u) return false;
    memset(c, 0, sizeof(*c));
    c->kind = kind;
    c->n_layer = n_layer;
    c->n_kvh = n_kvh;
    c->hd = hd;
    c->max_kv = max_kv;
    c->bpt = q4kv_token_bytes(kind, n_kvh, hd);
    const size_t bytes = (size_t)n_layer * max_kv * c->bpt;
    c->d_k = q4_hip_malloc(bytes);
    c->d_v = q4_hip_malloc(bytes);
    if (!c->d_k || !c->d_v) {
        q4kv_cache_close(c);
        fprintf(stderr, "q4: QSA KV %.2f GiB did not fit on the GPU at ctx %u\n",
                2.0 * (double)bytes / (1024.0 * 1024.0 * 1024.0), max_kv);
        return false;
    }
    return true;
}

void q4kv_cache_close(q4kv_cache *c) {
    if (!c) return;
    q4_hip_free(c->d_k);
    q4_hip_free(c->d_v);
    c->d_k = c->d_v = NULL;
    c->n_kv = 0;
}

uint8_t *q4kv_at(const q4kv_cache *c, int is_v, uint32_t layer, uint32_t tok) {
    uint8_t *base = (uint8_t *)(is_v ? c->d_v : c->d_k);
    return base + ((size_t)layer * c->max_kv + tok) * c->bpt;
}

bool q4kv_write(const q4kv_cache *c, void *dst, const float *d_src, uint64_t n) {
    if (c->kind == Q4KV_Q8) return q4_hip_f32_to_q8(dst, d_src, n);
    if (c->kind == Q4KV_F16) return q4_hip_f32_to_f16(dst, d_src, n);
    return q4_hip_copy((float *)dst, d_src, n);
}

bool q4kv_write_chunk(const q4kv_cache *c, uint32_t layer, uint32_t pos0, const float *d_k,
                      const float *d_v, uint32_t n_tok) {
    if (!c || !c->d_k || layer >= c->n_layer || !n_tok) return false;
    if ((uint64_t)pos0 + n_tok > c->max_kv) return false; /* context full */
    const uint64_t n = (uint64_t)n_tok * c->n_kvh * c->hd;
    return q4kv_write(c, q4kv_at(c, 0, layer, pos0), d_k, n) &&
           q4kv_write(c, q4kv_at(c, 1, layer, pos0), d_v, n);
}

bool q4kv_append_d(const q4kv_cache *c, uint32_t layer, const float *d_k, const float *d_v) {
    if (!c || !c->d_k || layer >= c->n_layer) return false;
    return q4_hip_kv_append_d(q4kv_at(c, 0, layer, 0), q4kv_at(c, 1, layer, 0), d_k, d_v,
                              c->n_kvh * c->hd, c->bpt, c->kind);
}

bool q4kv_attend(const q4kv_cache *c, uint32_t layer, const float *d_q, const float *d_gate,
                 float *d_out, uint32_t n_head, uint32_t n_tok, uint32_t pos0,
                 const int32_t *d_sel, uint32_t width, uint64_t sel_tok_stride,
                 uint64_t sel_kvh_stride) {
    if (!c || !c->d_k || layer >= c->n_layer || !n_tok) return false;
    const float scale = 1.0f / sqrtf((float)c->hd);
    const uint8_t *kb = q4kv_at(c, 0, layer, 0), *vb = q4kv_at(c, 1, layer, 0);
    if (!d_sel)
        return q4_hip_qsa_decode_n(d_q, kb, vb, d_gate, d_out, n_head, c->n_kvh, c->hd, n_tok,
                                   pos0, c->max_kv, scale, c->kind);
    return q4_hip_qsa_decode_idx_kv(d_q, kb, vb, d_gate, d_out, d_sel, width, sel_tok_stride,
                                    sel_kvh_stride, n_head, c->n_kvh, c->hd, n_tok, c->max_kv,
                                    scale, c->kind);
}

uint64_t q4kv_image_bytes(const q4kv_cache *c, uint32_t n_kv) {
    return 2ull * c->n_layer * (uint64_t)n_kv * c->bpt;
}

bool q4kv_image_restore(q4kv_cache *c, const uint8_t *host_body, uint32_t n_kv, bool wait) {
    if (!c || !c->d_k || !host_body || n_kv > c->max_kv) return false;
    const uint64_t sec = (uint64_t)n_kv * c->bpt;
    if (sec) {
        for (uint32_t l = 0; l < c->n_layer; l++) {
            const uint8_t *src = host_body + 2ull * l * sec;
            if (!q4_hip_h2d_async(q4kv_at(c, 0, l, 0), src, sec) ||
                !q4_hip_h2d_async(q4kv_at(c, 1, l, 0), src + sec, sec))
                return false;
        }
    }
    c->n_kv = n_kv;
    return wait ? q4_hip_stream_sync() : true;
}

bool q4kv_image_save(const q4kv_cache *c, uint8_t *host_body) {
    if (!c || !c->d_k || !host_body) return false;
    const uint64_t sec = (uint64_t)c->n_kv * c->bpt;
    if (!sec) return true;
    for (uint32_t l = 0; l < c->n_layer; l++) {
        uint8_t *dst = host_body + 2ull * l * sec;
        if (!q4_hip_d2h(dst, q4kv_at(c, 0, l, 0), sec) ||
            !q4_hip_d2h(dst + sec, q4kv_at(c, 1, l, 0), sec))
            return false;
    }
    return true;
}

/* Streamed through the pinned pipe: the device-to-host copy of the next
 * chunk overlaps the file write of the previous one (src/q4_fwd.c:2275-2294
 * stage through one pageable 16 MiB buffer, synchronously). The image is
 * written to path.tmp and renamed into place only when complete. */
#define Q4KV_IO_CHUNK ((size_t)32 << 20)

bool q4kv_image_save_file(const q4kv_cache *c, const char *path) {
    if (!c || !path || strlen(path) > 4096) return false;
    q4kv_img_hdr h = {Q4KV_IMG_MAGIC, Q4KV_IMG_VER, c->n_layer, c->n_kvh, c->hd,
                      c->max_kv,      c->n_kv,      q4kv_tag(c->kind)};
    char tmp[4096 + 8];
    snprintf(tmp, sizeof(tmp), "%s.tmp", path);
    int fd = open(tmp, O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) return false;
    bool ok = pwrite(fd, &h, sizeof(h), 0) == (ssize_t)sizeof(h);
    const uint64_t sec = (uint64_t)c->n_kv * c->bpt;
    if (ok && sec) {
        q4kv_pipe *p = q4kv_pipe_open(Q4KV_IO_CHUNK);
        uint64_t off = sizeof(h);
        ok = p != NULL;
        for (uint32_t l = 0; ok && l < c->n_layer; l++)
            for (int is_v = 0; ok && is_v < 2; is_v++, off += sec)
                ok = q4kv_pipe_dev_to_file(p, fd, off, q4kv_at(c, is_v, l, 0), sec);
        if (p) {
            ok = q4kv_pipe_finish(p) && ok;
            q4kv_pipe_close(p);
        }
    }
    if (close(fd) != 0) ok = false;
    if (!ok || rename(tmp, path) != 0) {
        remove(tmp);
        return false;
    }
    return true;
}

/* Streamed through the pinned pipe: the file read of the next chunk overlaps
 * the DMA of the previous one (src/q4_fwd.c:2393-2470). */
uint32_t q4kv_image_restore_file(q4kv_cache *c, const char *path) {
    if (!c || !c->d_k || !path) return 0;
    int fd = open(path, O_RDONLY);
    if (fd < 0) return 0;
    q4kv_img_hdr h;
    bool ok = pread(fd, &h, sizeof(h), 0) == (ssize_t)sizeof(h) && h.magic == Q4KV_IMG_MAGIC &&
              h.version == Q4KV_IMG_VER && h.n_layer == c->n_layer && h.n_kvh == c->n_kvh &&
              h.hd == c->hd && h.max_kv == c->max_kv && h.pad == q4kv_tag(c->kind) &&
              h.n_kv <= c->max_kv;
    const uint64_t sec = ok ? (uint64_t)h.n_kv * c->bpt : 0;
    if (ok && sec) {
        q4kv_pipe *p = q4kv_pipe_open(Q4KV_IO_CHUNK);
        uint64_t off = sizeof(h);
        ok = p != NULL;
        for (uint32_t l = 0; ok && l < c->n_layer; l++)
            for (int is_v = 0; ok && is_v < 2; is_v++, off += sec)
                ok = q4kv_pipe_file_to_dev(p, fd, off, q4kv_at(c, is_v, l, 0), sec);
        if (p) {
            ok = q4kv_pipe_finish(p) && ok;
            q4kv_pipe_close(p);
        }
    }
    close(fd);
    if (!ok) {
        c->n_kv = 0;
        return 0;
    }
    c->n_kv = h.n_kv;
    return h.n_kv;
}
