/*
 * q4kv.h -- C ABI of the MI355X QSA KV-cache library (libq4kv.so).
 *
 * Drop-in for SuzuQu-Engine's KV-cache hot path: every function below keeps
 * the name, signature, argument meaning and error convention of the
 * reference declaration it cites (upstream src/q4.h). All functions return
 * false (or NULL) on bad arguments or a launch error, print "q4 hip: ..." to
 * stderr for launch errors, and never abort. Device work is enqueued on one
 * library stream and is asynchronous unless stated otherwise.
 *
 * Cache layout (unchanged from the reference, src/q4_fwd.c:644-655): one K
 * and one V buffer per QSA layer, token-major [pos][kv_head][head_dim] with
 * bytes-per-token bpt = n_kvh*hd*4 (f32), n_kvh*hd*2 (f16) or
 * n_kvh*(hd/32)*34 (q8_0, blocks of {fp16 scale, 32 x int8}).
 * KV width codes ("kind", "kv_f16"): 0 = f32, 1 = f16, 2 = q8_0.
 */
#ifndef Q4KV_H
#define Q4KV_H
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { Q4KV_F32 = 0, Q4KV_F16 = 1, Q4KV_Q8 = 2 };

/* ---------------- runtime (src/q4.h:708-710, 877-880, 948-949) ---------- */
bool q4_hip_init(void);                       /* src/q4.h:708 */
void q4_hip_shutdown(void);                   /* src/q4.h:709 */
bool q4_hip_ok(void);                         /* src/q4.h:710 */
void *q4_hip_malloc(size_t n);                /* src/q4.h:877 */
void q4_hip_free(void *p);                    /* src/q4.h:878 */
bool q4_hip_h2d(void *d, const void *h, size_t n); /* src/q4.h:879, synchronous */
bool q4_hip_d2h(void *h, const void *d, size_t n); /* src/q4.h:880, synchronous */
void q4_hip_sync(void);                       /* src/q4.h:948 */
void q4_hip_clear(void);                      /* src/q4.h:949 */
bool q4_hip_d2h_async(void *h, const void *d, uint64_t n); /* src/q4.h:787 */
bool q4_hip_h2d_async(void *d, const void *h, uint64_t n); /* src/q4.h:788 */
bool q4_hip_stream_sync(void);                /* src/q4.h:789 */
/* f32 KV width store, n floats device-to-device (src/q4.h:851). Stream
 * ordered, and returns once the copy has landed, as the reference's does
 * (inside a capture it becomes a copy node). */
bool q4_hip_copy(float *d, const float *s, uint64_t n);

/* Graph capture of the compute stream (src/q4.h:782-786). */
int q4_hip_graph_begin(void);
void *q4_hip_graph_end(void);
uint32_t q4_hip_graph_nodes(void *exec);
bool q4_hip_graph_launch(void *exec);
void q4_hip_graph_free(void *exec);

/* Device decode position for graph-captured kernels (src/q4.h:686-688). */
void q4_hip_pos_push(int32_t pos);
int q4_hip_capturing(void);
int q4_hip_pos_dev_ok(void);

/* ---------------- KV writes (a1-a3) ---------------- */
/* fp32 [n] -> q8_0 blocks, n % 32 == 0 (src/q4.h:929). */
bool q4_hip_f32_to_q8(void *dst_q8, const float *src, uint64_t n);
/* fp32 [n] -> fp16 [n], round-to-nearest-even (src/q4.h:928). */
bool q4_hip_f32_to_f16(void *dst_f16, const float *src, uint64_t n);
/* Append one token's K and V (n floats each) at the device position into
 * caches with bpt bytes per token, width `kind` (src/q4.h:694-695).
 * A q8_0 append of whole 256-dim head rows (bpt = n / 256 * 272) is held,
 * not launched: the next one-token decode over the same caches performs it
 * inside its own launch, as do the indexer calls that follow the append in
 * the reference's layer (q4_hip_f32_to_f16_d, q4_hip_qsa_index_score_d: extra
 * workgroups of their launch), and any other q4_hip_* / q4kv_* call launches
 * it first, so every library call sees the appended rows, in stream order.
 * Work the caller enqueues itself on the stream between this call and the
 * next library call does not (it must not read the caches or overwrite k
 * and v there). Q4KV_HOLD_APPEND=0 launches every append at once. */
bool q4_hip_kv_append_d(void *kcache, void *vcache, const float *k, const float *v,
                        uint32_t n, uint32_t bpt, int kind);

/* ---------------- QSA attention (a5-a9) ----------------
 * Shapes, as the reference accepts them: head_dim 1..256 (a multiple of 32
 * for q8_0, whose rows are 32-element blocks), n_head a multiple of n_kvh,
 * any number of query heads per KV head.
 * Value range: any finite query. The MFMA kernels divide each head's q
 * (some of them q * scale / ln 2) by the power of two that brings its
 * largest magnitude into [0.5, 1) before splitting it into fp16 parts, and
 * multiply the head's scores back (exact). The prefill band kernel (q8_0,
 * head_dim 256, prefill-sized indexed calls) dequantises K and V to fp16
 * parts like the reference's prefill tile, so cache values must stay below
 * 65504 in magnitude there. */
/* Dense causal attention: token t of n_tok attends positions
 * 0 .. min(kv_base+t+1, max_kv)-1. q/gate/out are [n_tok][n_head][hd] fp32;
 * out = softmax(q.k*scale) @ v * sigmoid(gate) (src/q4.h:906-909). */
bool q4_hip_qsa_decode_n(const float *d_q, const void *d_kcache, const void *d_vcache,
                         const float *d_gate, float *d_out, uint32_t n_head,
                         uint32_t n_kvh, uint32_t hd, uint32_t n_tok, uint32_t kv_base,
                         uint32_t max_kv, float scale, int kv_f16);
/* Attention over an explicit position list: row t is idx[t*width + j],
 * -1 = padding, shared by all KV heads (src/q4.h:911-915). */
bool q4_hip_qsa_decode_idx(const float *d_q, const void *d_kcache, const void *d_vcache,
                           const float *d_gate, float *d_out, const int32_t *idx,
                           uint32_t width, uint32_t n_head, uint32_t n_kvh, uint32_t hd,
                           uint32_t n_tok, uint32_t max_kv, float scale, int kv_f16);
/* One-token dense decode over n_kv positions (src/q4.h:621-624). */
bool q4_hip_qsa_decode(const float *d_q, const void *d_kcache, const void *d_vcache,
                       const float *d_gate, float *d_out, uint32_t n_head, uint32_t n_kvh,
                       uint32_t hd, uint32_t n_kv, uint32_t max_kv, float scale, int kv_f16);
/* Internal scratch for split decode (src/q4.h:704). The library allocates
 * its split-KV partial buffer in q4_hip_init; this only reports it. */
bool q4_hip_qsa_topk_alloc(void);

/* ---------------- QSA indexer and Q/K preparation ----------------
 * Shapes as the reference: hd (indexer dim) must be 128, n_head <= 4,
 * k_blk <= 512. raw is fp16 [pos][128], pool fp32 [block][128], score fp32
 * [tok][stride], sel int32 [tok][width]. _d variants read the position from
 * the device counter set by q4_hip_pos_push and are graph-capture safe. */
bool q4_hip_qsa_q_prep(const float *d_qg, const float *d_wn, float *d_q, float *d_g,
                       uint32_t n_head, uint32_t hd, uint32_t n_rot, int32_t pos,
                       float base, float eps);                          /* src/q4.h:895-897 */
bool q4_hip_qsa_q_prep_n(const float *d_qg, const float *d_wn, float *d_q, float *d_g,
                         uint32_t n_head, uint32_t hd, uint32_t n_rot, int32_t pos0,
                         float base, float eps, uint32_t n_tok);       /* src/q4.h:898-900 */
bool q4_hip_qsa_q_prep_d(const float *qg, const float *wn, float *q, float *g,
                         uint32_t n_head, uint32_t hd, uint32_t n_rot,
                         float base, float eps);                        /* src/q4.h:689-691 */
bool q4_hip_qsa_k_prep(float *d_k, const float *d_wn, uint32_t n_kvh, uint32_t hd,
                       uint32_t n_rot, int32_t pos, float base, float eps); /* src/q4.h:901-902 */
bool q4_hip_qsa_k_prep_n(float *d_k, const float *d_wn, uint32_t n_kvh, uint32_t hd,
                         uint32_t n_rot, int32_t pos0, float base, float eps,
                         uint32_t n_tok);                               /* src/q4.h:903-905 */
bool q4_hip_qsa_k_prep_d(float *k, const float *wn, uint32_t n_kvh, uint32_t hd,
                         uint32_t n_rot, float base, float eps);        /* src/q4.h:692-693 */
bool q4_hip_f32_to_f16_d(void *dst_base, uint32_t stride_elems, const float *src,
                         uint64_t n);                                   /* src/q4.h:696-697 */
bool q4_hip_qsa_pool(const void *raw_f16, float *pool, const float *wn, uint32_t hd,
                     uint32_t ratio, uint32_t b0, uint32_t b1, uint32_t n_rot,
                     float rope_base, float eps);                       /* src/q4.h:917-920 */
bool q4_hip_qsa_pool_d(const void *raw, float *pool, const float *wn, uint32_t hd,
                       uint32_t ratio, uint32_t n_rot, float rope_base,
                       float eps);                                      /* src/q4.h:698-700 */
bool q4_hip_qsa_score(const float *q, const float *pool, float *score, uint32_t n_tok,
                      uint32_t n_blocks, uint32_t stride, uint32_t n_head, uint32_t hd,
                      uint32_t pos0, uint32_t ratio);                   /* src/q4.h:921-924 */
bool q4_hip_qsa_score_d(const float *q, const float *pool, float *score, uint32_t stride,
                        uint32_t n_head, uint32_t hd, uint32_t ratio);  /* src/q4.h:701-703 */
bool q4_hip_qsa_topk(const float *score, int32_t *sel, uint32_t n_tok, uint32_t n_blocks,
                     uint32_t stride, uint32_t k_blk, uint32_t ratio, uint32_t pos0,
                     uint32_t width);                                   /* src/q4.h:925-927 */
bool q4_hip_qsa_topk_d(const float *score, int32_t *sel, uint32_t stride, uint32_t k_blk,
                       uint32_t ratio, uint32_t width);                 /* src/q4.h:705-706 */

/* ---------------- attention output projection ----------------
 * y[r] = scale * sum_c W[r][c] x[c] with W in q8_0 rows (ncols/32 blocks of
 * 34 bytes). Only ggml type 8 (q8_0) is supported; other types return false. */
bool q4_hip_gemv_dd(uint32_t ggml_type, const uint8_t *d_w, uint64_t nrows, uint64_t ncols,
                    const float *d_x, float *d_y, float scale);         /* src/q4.h:720-721 */

/* ---------------- extensions (no reference counterpart) ----------------
 * Additive entry points; nothing above depends on them. */

/* q4_hip_qsa_decode_idx with a separate position list per KV head: the list
 * of (token t, kv head kh) starts at idx + t*tok_stride + kh*kvh_stride.
 * With tok_stride = width and kvh_stride = 0 it is q4_hip_qsa_decode_idx.
 * d_gate may be NULL (no gate). */
bool q4_hip_qsa_decode_idx_kv(const float *d_q, const void *d_kcache, const void *d_vcache,
                              const float *d_gate, float *d_out, const int32_t *idx,
                              uint32_t width, uint64_t tok_stride, uint64_t kvh_stride,
                              uint32_t n_head, uint32_t n_kvh, uint32_t hd, uint32_t n_tok,
                              uint32_t max_kv, float scale, int kv_f16);

/* One decode item of a batched launch: an independent sequence (or layer)
 * with its own caches, query, output and per-KV-head position lists.
 * All pointers are device pointers; the descriptor array itself lives in
 * device memory (caller-owned, 64 bytes per entry). kcache and vcache must
 * be 16-byte aligned (the batched kernels fetch rows in 16-byte pieces;
 * q4_hip_malloc memory always is): the library cannot read the descriptors
 * on the host to check. */
typedef struct {
    const void *kcache;     /* [max_kv][n_kvh][row] */
    const void *vcache;
    const float *q;         /* [n_head][hd] */
    const float *gate;      /* [n_head][hd] or NULL */
    float *out;             /* [n_head][hd] */
    const int32_t *idx;     /* list of kv head kh at idx + kh*idx_kvh_stride; NULL = dense */
    uint32_t n_sel;         /* list length (indexed) or visible positions (dense) */
    uint32_t idx_kvh_stride;
    uint32_t max_kv;
    uint32_t reserved;
} q4kv_seq_desc;

/* Decode one token for each of n_seq independent items in one launch
 * (batched serving, or several layers' caches with queries already known).
 * max_n bounds the descriptors' n_sel; it sizes the split-KV work division
 * only (a larger n_sel is still processed in full). */
bool q4_hip_qsa_decode_batch(const q4kv_seq_desc *d_descs, uint32_t n_seq,
                             uint32_t n_head, uint32_t n_kvh, uint32_t hd, float scale,
                             int kv_f16, uint32_t max_n);

/* One decode step of one item: append the token's K and V rows at pos, then
 * attend -- q4_hip_kv_append_batch followed by q4_hip_qsa_decode_batch, in
 * one launch when head_dim is 256 with at most 16 query heads per KV head
 * (any width; otherwise an append launch precedes the attention). The
 * attention sees the new row wherever its position list names pos. 96 bytes,
 * device memory. */
typedef struct {
    q4kv_seq_desc seq;      /* caches, query, gate, output, position lists */
    const float *k, *v;     /* the token's rows, [n_kvh][hd] fp32 each */
    uint32_t pos;           /* cache position the rows are written at (< max_kv) */
    uint32_t reserved[3];
} q4kv_step_desc;

bool q4_hip_qsa_step_batch(const q4kv_step_desc *d_descs, uint32_t n_seq, uint32_t n_head,
                           uint32_t n_kvh, uint32_t hd, float scale, int kv_f16,
                           uint32_t max_n);

/* q4_hip_qsa_step_batch without any allocation: no counterpart in the
 * reference. For callers that cannot call hipMalloc (code under hipGraph
 * capture, tight serving loops, harnesses that forbid allocation). The split
 * partials live in a static 16 MiB device array (one per GPU, held until
 * the process ends; q4_hip_init resolves its address), so the call
 * allocates nothing. Same arguments, same split division and results as
 * q4_hip_qsa_step_batch, bit for bit. Returns false, with a message, when
 * the call's partials would exceed 4M floats (n_seq * n_kvh items x splits x
 * n_head/n_kvh x 258). Calls that overlap on one GPU share the array and
 * race: order them on one stream. */
bool q4_hip_qsa_step_batch_noalloc(const q4kv_step_desc *d_descs, uint32_t n_seq,
                                   uint32_t n_head, uint32_t n_kvh, uint32_t hd, float scale,
                                   int kv_f16, uint32_t max_n);

/* A decode step with the query/key preparation fused in (src/q4_fwd.c:806-824:
 * q4_hip_qsa_q_prep + q4_hip_qsa_k_prep + the append + the attention, in
 * one launch plus the merge). step.seq.q points at the raw rows
 * [n_head][q (hd) | gate (hd)]; step.seq.gate receives the gate halves
 * ([n_head][hd], as q_prep's g) and gates the output (NULL: no gate);
 * step.k is the raw K row (read, not modified). 128 bytes. */
typedef struct {
    q4kv_step_desc step;
    const float *wn_q, *wn_k; /* RMSNorm weights [hd]; NULL = 1 */
    uint64_t reserved[2];
} q4kv_prep_step_desc;

/* The same results as q4_hip_qsa_q_prep / q4_hip_qsa_k_prep (at step.pos,
 * with n_rot, rope_base, eps) followed by q4_hip_qsa_step_batch, bit for bit.
 * q8_0 caches with hd 256 and n_head / n_kvh <= 8 only. */
bool q4_hip_qsa_step_prep_batch(const q4kv_prep_step_desc *d_descs, uint32_t n_seq,
                                uint32_t n_head, uint32_t n_kvh, uint32_t hd, float scale,
                                int kv_f16, uint32_t max_n, uint32_t n_rot, float rope_base,
                                float eps);

/* The attention output projection of one item, for q4_hip_qsa_step_out_batch. */
typedef struct {
    const uint8_t *w_o; /* q8_0 attn_output weight [n_embd][n_head*hd / 32 blocks] */
    float *y;           /* [n_embd]: y += y_scale * w_o . out */
} q4kv_out_desc;

/* q4_hip_qsa_step_batch with the merge epilogue fused into the attention
 * output projection (src/q4_fwd.c:922-927: the gated merge, then the q8_0
 * attn_output GEMV): each item's merged, gated output is written to its
 * seq.out and y += y_scale * w_o . out is accumulated with fp32 atomics (the
 * heads' contributions to a row are summed in arrival order, so y matches
 * q4_hip_gemv_dd + add within rounding, not bit for bit). Two launches per
 * call. q8_0 caches with hd 256 and n_head / n_kvh <= 8 only. */
bool q4_hip_qsa_step_out_batch(const q4kv_step_desc *d_descs, const q4kv_out_desc *d_outs,
                               uint32_t n_seq, uint32_t n_head, uint32_t n_kvh, uint32_t hd,
                               float scale, int kv_f16, uint32_t max_n, uint32_t n_embd,
                               float y_scale);

/* One token's K/V rows for one cache, for a batched append. */
typedef struct {
    void *kcache, *vcache; /* cache bases (token 0) */
    const float *k, *v;    /* n fp32 each */
    uint32_t pos;          /* token position to write */
    uint32_t reserved;
} q4kv_append_desc;

/* The decode indexer step in one launch (src/q4_fwd.c:904-916 fused): the
 * effect of q4_hip_f32_to_f16_d(raw_f16, hd, k_new, hd), then
 * q4_hip_qsa_pool_d(raw_f16, pool, wn_k, hd, ratio, n_rot, rope_base, eps),
 * then q4_hip_qsa_k_prep_d on a copy of q with wn_q, then
 * q4_hip_qsa_score_d(that copy, pool, score, stride, n_head, hd, ratio):
 * the same raw row, pool rows and scores. q itself is not modified. */
bool q4_hip_qsa_index_score_d(void *raw_f16, float *pool, const float *wn_k, const float *k_new,
                              const float *q, const float *wn_q, float *score, uint32_t stride,
                              uint32_t n_head, uint32_t hd, uint32_t ratio, uint32_t n_rot,
                              float rope_base, float eps);

/* One item of a batched decode indexer step: an independent sequence (or
 * layer) with its own indexer buffers and position. Device pointers; the
 * descriptor array lives in device memory. 80 bytes. */
typedef struct {
    void *raw;           /* fp16 raw keys [max_kv][hd]; row pos is written */
    float *pool;         /* fp32 pooled blocks [max_kv/ratio][hd] */
    const float *wn_k;   /* k_norm weights [hd] or NULL */
    const float *k_new;  /* the token's raw indexer key, fp32 [hd] */
    const float *q;      /* raw indexer queries, fp32 [n_head][hd] (read, not modified) */
    const float *wn_q;   /* q_norm weights [hd] or NULL */
    float *score;        /* fp32 [max_blocks] scores (written) */
    int32_t *sel;        /* int32 [width] position list (written) */
    uint32_t pos;        /* the token's position */
    uint32_t reserved[3];
} q4kv_index_desc;

/* The decode indexer of n_items independent items in two launches: per item
 * the effect of q4_hip_qsa_index_score_d then q4_hip_qsa_topk_d at the item's
 * own position (the same bytes as those calls; tests/test_gpu_index.py).
 * max_blocks bounds every item's visible blocks (the score grid). */
bool q4_hip_qsa_index_batch(const q4kv_index_desc *d_descs, uint32_t n_items,
                            uint32_t max_blocks, uint32_t n_head, uint32_t hd, uint32_t ratio,
                            uint32_t n_rot, float rope_base, float eps, uint32_t k_blk,
                            uint32_t width);

/* Append into n_desc caches in one launch (the per-layer
 * q4_hip_kv_append_d of a decode step, batched). */
bool q4_hip_kv_append_batch(const q4kv_append_desc *d_descs, uint32_t n_desc, uint32_t n,
                            uint32_t bpt, int kind);

/* Run all library work on the caller's HIP stream (an engine's own compute
 * stream), or on the library's stream again when stream is NULL. */
bool q4kv_use_stream(void *stream);

/* Streamed file <-> device copies through pinned staging buffers of `chunk`
 * bytes (the session image path; src/q4_fwd.c:2275-2294 stage synchronously
 * through one pageable buffer). Reads of the next chunk overlap the DMA of
 * the previous one, and device-to-host copies overlap the file writes. All
 * copies are ordered on the library stream. q4kv_pipe_finish waits for every
 * queued copy and write and reports whether all succeeded; after a failure
 * the pipe refuses further work until finish. */
typedef struct q4kv_pipe q4kv_pipe;
q4kv_pipe *q4kv_pipe_open(size_t chunk);
void q4kv_pipe_close(q4kv_pipe *p);
bool q4kv_pipe_file_to_dev(q4kv_pipe *p, int fd, uint64_t off, void *dst, uint64_t n);
bool q4kv_pipe_dev_to_file(q4kv_pipe *p, int fd, uint64_t off, const void *src, uint64_t n);
bool q4kv_pipe_finish(q4kv_pipe *p);

/* Pinned host buffers for restoring a session KV image (hipHostMalloc). */
void *q4_hip_host_alloc(size_t n);
void q4_hip_host_free(void *p);

/* Event timing on the library stream (benchmark support). */
bool q4kv_timer_begin(int slot);
double q4kv_timer_end_ms(int slot);
int q4kv_device_info(char *name, int name_len, int *n_cu, int *clock_khz);
/* Arm per-launch event timing of the split-KV attention kernel for up to
 * max_launches launches; q4kv_prof_end waits and returns the number timed
 * and their summed duration in ms. */
bool q4kv_prof_begin(int max_launches);
int q4kv_prof_end(double *total_ms);
/* Placement of the split-KV launches: 1 (default) runs the KV heads of each
 * (token, split) on one XCD, 0 uses the plain (split, item) grid, -1 only
 * queries; returns the setting. Results are identical either way (test and
 * measurement support; no counterpart in the reference). */
int q4kv_xcd_group(int on);

#ifdef __cplusplus
}
#endif
#endif
