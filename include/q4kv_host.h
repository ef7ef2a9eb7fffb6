/*
 * q4kv_host.h -- host-side (C) KV-cache layer above the q4kv.h C ABI.
 *
 * Mirrors the reference's host code for the QSA KV path in src/q4_fwd.c:
 * width selection, bytes per token, cache addressing, the width-dispatched
 * write, the attention call sites and the K/V section of the session image.
 * Everything here is plain C calling the C ABI; device pointers are opaque.
 */
#ifndef Q4KV_HOST_H
#define Q4KV_HOST_H
#include <stdbool.h>
#include <stdint.h>

#include "q4kv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* The QSA KV cache of one session: n_layer QSA layers, each a K and a V
 * buffer of max_kv tokens x bpt bytes, token-major (src/q4_fwd.c:1944-1950,
 * 652-655). */
typedef struct {
    int kind;           /* Q4KV_F32 / Q4KV_F16 / Q4KV_Q8 */
    uint32_t n_layer;   /* QSA layers (n_qsa) */
    uint32_t n_kvh, hd; /* KV heads and head dim */
    uint32_t max_kv;    /* token capacity */
    uint32_t bpt;       /* bytes per token of one K or V buffer */
    uint32_t n_kv;      /* tokens held */
    void *d_k, *d_v;    /* device buffers, n_layer * max_kv * bpt bytes each */
} q4kv_cache;

/* Width from a Q4_KV value ("f32"/"fp32", "f16"/"fp16", else q8_0); NULL
 * reads the Q4_KV environment variable (src/q4_fwd.c:637-642). */
int q4kv_kind_of(const char *q4_kv);
/* Bytes per token of one K or V cache (src/q4_fwd.c:644-650). */
uint32_t q4kv_token_bytes(int kind, uint32_t n_kvh, uint32_t hd);
/* K+V bytes of n_layer QSA layers at ctx tokens (src/q4_place.c:92-106). */
uint64_t q4kv_cache_bytes(int kind, uint32_t n_layer, uint32_t n_kvh, uint32_t hd,
                          uint32_t ctx);
/* Session-image width tag: q8 = 8, f16 = 2, f32 = 4 (src/q4_fwd.c:663-665). */
uint32_t q4kv_tag(int kind);

/* Allocate / free the device caches (src/q4_fwd.c:1940-2010). */
bool q4kv_cache_open(q4kv_cache *c, int kind, uint32_t n_layer, uint32_t n_kvh, uint32_t hd,
                     uint32_t max_kv);
void q4kv_cache_close(q4kv_cache *c);
/* Address of token tok of layer `layer`'s K (is_v = 0) or V cache
 * (src/q4_fwd.c:652-655). */
uint8_t *q4kv_at(const q4kv_cache *c, int is_v, uint32_t layer, uint32_t tok);
/* Width-dispatched write of n fp32 values (src/q4_fwd.c:657-661). */
bool q4kv_write(const q4kv_cache *c, void *dst, const float *d_src, uint64_t n);

/* Write n_tok tokens of K and V ([n_tok][n_kvh*hd] fp32, device) at positions
 * pos0.. of a layer: the prefill chunk write of src/q4_fwd.c:1736-1741. */
bool q4kv_write_chunk(const q4kv_cache *c, uint32_t layer, uint32_t pos0, const float *d_k,
                      const float *d_v, uint32_t n_tok);
/* Graph-safe decode append of one token at the device position
 * (src/q4_fwd.c:889-891). */
bool q4kv_append_d(const q4kv_cache *c, uint32_t layer, const float *d_k, const float *d_v);

/* Attention for n_tok tokens at positions pos0.. of a layer (the QSA call
 * sites of src/q4_fwd.c:722-775): dense causal when d_sel is NULL,
 * otherwise over the selection rows d_sel + t*sel_tok_stride +
 * kh*sel_kvh_stride of `width` entries. d_gate may be NULL only with a
 * selection. */
bool q4kv_attend(const q4kv_cache *c, uint32_t layer, const float *d_q, const float *d_gate,
                 float *d_out, uint32_t n_head, uint32_t n_tok, uint32_t pos0,
                 const int32_t *d_sel, uint32_t width, uint64_t sel_tok_stride,
                 uint64_t sel_kvh_stride);

/* K/V section of the session image (src/q4_fwd.c:2256-2470): a header
 * carrying the width tag, then for each layer the raw K bytes then the raw
 * V bytes of tokens 0..n_kv-1. */
typedef struct {
    uint32_t magic;   /* Q4KV_IMG_MAGIC */
    uint32_t version; /* Q4KV_IMG_VER */
    uint32_t n_layer, n_kvh, hd, max_kv, n_kv;
    uint32_t pad;     /* width tag, must equal q4kv_tag(kind) on restore */
} q4kv_img_hdr;
#define Q4KV_IMG_MAGIC 0x564b3451u /* "Q4KV" */
#define Q4KV_IMG_VER 1u

/* Bytes of the image body for n_kv tokens. */
uint64_t q4kv_image_bytes(const q4kv_cache *c, uint32_t n_kv);
/* Restore n_kv tokens from a host image body (pinned memory gives full link
 * speed) into the device cache layout; asynchronous on the library stream
 * unless `wait`. */
bool q4kv_image_restore(q4kv_cache *c, const uint8_t *host_body, uint32_t n_kv, bool wait);
/* Copy the cache out into a host image body (synchronous). */
bool q4kv_image_save(const q4kv_cache *c, uint8_t *host_body);
/* File variants with the header guard; restore returns the token count on
 * success and 0 on any mismatch (the cache is then left empty). */
bool q4kv_image_save_file(const q4kv_cache *c, const char *path);
uint32_t q4kv_image_restore_file(q4kv_cache *c, const char *path);

#ifdef __cplusplus
}
#endif
#endif
