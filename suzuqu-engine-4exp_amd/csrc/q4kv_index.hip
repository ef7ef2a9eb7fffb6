/*
 * q4kv_index.hip -- the QSA indexer on gfx950: pooled block keys, block
 * scores, exact top-k block selection with expansion to a position list, and
 * the RMSNorm + partial-RoPE preparation of queries and keys.
 *
 * Reference interface: src/q4.h:689-707, 895-927; kernels
 * src/q4_rocm.cu:6229-6343 (prep) and 7366-7960 (indexer).
 *
 * Layouts (as the reference's callers, src/q4_fwd.c:676-770, 895-925):
 *   raw   fp16 [pos][hd]          indexer keys, hd = 128
 *   pool  fp32 [block][hd]        block b pools positions b*ratio .. +ratio-1
 *   q     fp32 [tok][head][hd]    indexer queries, head < 4
 *   score fp32 [tok][stride]      stride = max_blocks
 *   sel   int32 [tok][width]      the attention's position list
 *
 * Design:
 *   pool   one wave per block; lane l owns the RoPE pair (2l, 2l+1), so the
 *          rotation never leaves the lane. The RoPE frequency is computed
 *          once per lane, correctly rounded (pow in double, one rounding).
 *   score  decode: a memory-bound stream over the pool (512 B per block);
 *          eight lanes per block row, each lane holding 16 dims of all four
 *          queries in registers, a 3-step DPP reduction per head.
 *          prefill (>= 4 tokens): bf16 MFMA 16x16x32 with a three-product
 *          hi/lo split (~2^-16 relative per product), A rows (token, head) so
 *          each lane's four accumulators are one token's four heads and the
 *          relu-sum over heads stays in the lane.
 *   topk   one 1024-thread workgroup per token row, keys in VGPRs (64 per
 *          thread). One histogram pass of the distance from the row maximum
 *          (1/16-octave steps of |score|, 32-way replicated LDS counters so
 *          a half-wave's atomics hit distinct banks) isolates a small
 *          candidate set, compacted in index order (LDS atomic-or lane masks
 *          and one block scan); two exact radix passes run over the
 *          threshold bin's candidates only. Rows that do not reduce (heavy ties,
 *          more than 65536 blocks) take four 8-bit radix passes over every
 *          key. One launch replaces the reference's ten on the
 *          device-position path. A device-position row of 16385-65536
 *          blocks is split over 8 workgroups of 8192 keys that hand their
 *          local candidates to the last one to finish; token rows of up to
 *          8192 blocks run on 512 threads (16 keys each), which halves the
 *          waves a prefill slice launches.
 */
#include "q4kv_internal.h"
#include "q4kv.h"

#include <math.h>
#include <stdlib.h>
#include <utility>

namespace {

constexpr uint32_t IDX_HD = 128;

/* Global-memory vector loads/stores (HIP's vector classes do not take an
 * address-space qualified copy, so they go through native vector types). */
typedef float idx_f2 __attribute__((ext_vector_type(2)));
typedef float idx_f4 __attribute__((ext_vector_type(4)));
__device__ inline float4 ld_vec(const float4 *p) {
    const idx_f4 v = *(const GLOBAL idx_f4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ inline float2 ld_vec(const float2 *p) {
    const idx_f2 v = *(const GLOBAL idx_f2 *)p;
    return make_float2(v.x, v.y);
}
__device__ inline void st_vec(float2 *p, float2 v) { *(GLOBAL idx_f2 *)p = (idx_f2){v.x, v.y}; }

/* the shared wave arithmetic of q4kv_internal.h under short names */
__device__ inline float sum8(float v) { return q4kv_sum8(v); }
__device__ inline float wave_sum(float v) { return q4kv_wave_sum(v); }
__device__ inline float rope_freq(float base, uint32_t p, uint32_t np) {
    return q4kv_rope_freq(base, p, np);
}
__device__ inline void rope_rotate(float &x0, float &x1, float pos_f, float freq) {
    q4kv_rope_rotate(x0, x1, pos_f, freq);
}

/* --------------------------------------------------------------- pool ---- */

/* Pool block b into pool[b][0..128): mean of `ratio` fp16 rows, RMSNorm * wn,
 * RoPE at position b*ratio. One wave; lane l owns dims 2l, 2l+1. When last
 * is non-zero it replaces the block's last raw row (fp16 pair bits), the row
 * that is being stored in the same launch. Returns this lane's pooled pair.
 * src/q4_rocm.cu:7366-7401. */
__device__ __attribute__((always_inline)) inline float2 pool_block(const uint32_t *raw2, float *pool, const float *wn,
                                    uint32_t ratio, uint32_t b, uint32_t n_rot, float freq,
                                    float eps, uint32_t lane, bool use_last = false,
                                    uint32_t last = 0) {
    const uint32_t *src = raw2 + (size_t)b * ratio * (IDX_HD / 2) + lane;
    float s0 = 0.f, s1 = 0.f;
    uint32_t j = 0;
    for (; j + 4 <= ratio; j += 4) {
        uint32_t h[4];
#pragma unroll
        for (int i = 0; i < 4; i++) h[i] = ldg(src + (size_t)(j + i) * (IDX_HD / 2));
        if (use_last && j + 4 == ratio) h[3] = last;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            s0 += __half2float(__ushort_as_half((unsigned short)(h[i] & 0xffffu)));
            s1 += __half2float(__ushort_as_half((unsigned short)(h[i] >> 16)));
        }
    }
    for (; j < ratio; j++) {
        uint32_t h = ldg(src + (size_t)j * (IDX_HD / 2));
        if (use_last && j + 1 == ratio) h = last;
        s0 += __half2float(__ushort_as_half((unsigned short)(h & 0xffffu)));
        s1 += __half2float(__ushort_as_half((unsigned short)(h >> 16)));
    }
    float v0 = __fdiv_rn(s0, (float)ratio), v1 = __fdiv_rn(s1, (float)ratio);
    const float ss = wave_sum(v0 * v0 + v1 * v1);
    const float inv = __fdiv_rn(1.f, __fsqrt_rn(__fdiv_rn(ss, (float)IDX_HD) + eps));
    const float w0 = wn ? ldg(wn + 2 * lane) : 1.f, w1 = wn ? ldg(wn + 2 * lane + 1) : 1.f;
    v0 = v0 * inv * w0;
    v1 = v1 * inv * w1;
    if (2 * lane < n_rot) rope_rotate(v0, v1, (float)(b * ratio), freq);
    st_vec((float2 *)(pool + (size_t)b * IDX_HD) + lane, make_float2(v0, v1));
    return make_float2(v0, v1);
}

__global__ __launch_bounds__(256) void qsa_pool_k(const uint32_t *raw2, float *pool,
                                                  const float *wn, uint32_t ratio, uint32_t b0,
                                                  uint32_t b1, uint32_t n_rot, float base,
                                                  float eps) {
    const uint32_t lane = threadIdx.x & 63u;
    const float freq = 2 * lane < n_rot ? rope_freq(base, lane, n_rot / 2) : 0.f;
    const uint32_t nw = gridDim.x * 4u;
    for (uint32_t b = b0 + blockIdx.x * 4u + (threadIdx.x >> 6); b < b1; b += nw)
        pool_block(raw2, pool, wn, ratio, b, n_rot, freq, eps, lane);
}

/* Device-position variant: pools the block that position *pp completes, if
 * any (src/q4_rocm.cu:7893-7930). */
__global__ __launch_bounds__(64) void qsa_pool_dk(const uint32_t *raw2, float *pool,
                                                  const float *wn, uint32_t ratio,
                                                  uint32_t n_rot, float base, float eps,
                                                  const int32_t *pp) {
    const uint32_t pos = (uint32_t)*pp;
    const uint32_t b0 = pos / ratio, b1 = (pos + 1) / ratio;
    if (b1 <= b0) return;
    const uint32_t lane = threadIdx.x;
    const float freq = 2 * lane < n_rot ? rope_freq(base, lane, n_rot / 2) : 0.f;
    pool_block(raw2, pool, wn, ratio, b0, n_rot, freq, eps, lane);
}

/* fp16 store of the raw key at the device position's row
 * (src/q4_rocm.cu:7932-7947) by the first n_wg workgroups; any after them
 * write a held cache append (app). */
__global__ __launch_bounds__(256) void f16_at_k(const float *src, __half *dst0, uint32_t stride,
                                                uint64_t n, const int32_t *pp, uint32_t n_wg,
                                                q4kv_app_args app) {
    if (blockIdx.x >= n_wg) {
        q4kv_app_wg(app, blockIdx.x - n_wg);
        return;
    }
    __half *dst = dst0 + (size_t)(uint32_t)*pp * stride;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = __float2half_rn(ldg(src + i));
}

/* -------------------------------------------------------------- score ---- */

constexpr uint32_t SC_ROWS_WG = 64; /* 4 waves x 2 x 8 rows */

/* The scores of rows rb + [0, 64) (and further grid strides) of one token:
 * eight lanes per row, lane g holding dims {32i + 4g .. +3 : i < 4} of each
 * query in qr. Row b_new, when in range, is taken from nr (this lane's dims
 * of the pooled row this launch produced) instead of the pool. */
/* this lane's dims of its two rows of the 64-row group at rb (rows past
 * n_vis re-read the last visible row) */
__device__ __attribute__((always_inline)) inline void score_load(float4 (&p)[2][4], const float *pool,
                                                                 uint32_t rb, uint32_t n_vis,
                                                                 uint32_t lane, uint32_t wave) {
    const uint32_t g = lane & 7u, rsub = lane >> 3;
    const uint32_t rlast = n_vis ? n_vis - 1 : 0;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint32_t row = rb + wave * 16u + 8u * u + rsub;
        const uint32_t r = row < rlast ? row : rlast;
        const float4 *src = (const float4 *)(pool + (size_t)r * IDX_HD) + g;
#pragma unroll
        for (int i = 0; i < 4; i++) p[u][i] = ld_vec(src + 8 * i);
    }
}

/* Scores of the two rows score_load fetched (row b_new taken from nr). */
__device__ __attribute__((always_inline)) inline void score_store(const float4 (&qr)[4][4], float4 (&p)[2][4],
                                                                  float *srow, uint32_t rb,
                                                                  uint32_t n_blocks, uint32_t n_vis,
                                                                  uint32_t lane, uint32_t wave,
                                                                  float4 nr0, float4 nr1, float4 nr2,
                                                                  float4 nr3, uint32_t b_new) {
    const uint32_t g = lane & 7u, rsub = lane >> 3;
    uint32_t row[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        row[u] = rb + wave * 16u + 8u * u + rsub;
        if (row[u] == b_new) {
            p[u][0] = nr0;
            p[u][1] = nr1;
            p[u][2] = nr2;
            p[u][3] = nr3;
        }
    }
    {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            float s = 0.f;
#pragma unroll
            for (int h = 0; h < 4; h++) {
                float d = 0.f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    d = fmaf(qr[h][i].x, p[u][i].x, d);
                    d = fmaf(qr[h][i].y, p[u][i].y, d);
                    d = fmaf(qr[h][i].z, p[u][i].z, d);
                    d = fmaf(qr[h][i].w, p[u][i].w, d);
                }
                s += fmaxf(sum8(d), 0.f);
            }
            if (g == 0 && row[u] < n_blocks) stg(srow + row[u], row[u] < n_vis ? s : -1.0e30f);
        }
    }
}

__device__ __attribute__((always_inline)) inline void score_rows(const float4 (&qr)[4][4], const float *pool, float *srow,
                                  uint32_t rb, uint32_t n_blocks, uint32_t n_vis,
                                  uint32_t lane, uint32_t wave, float4 nr0, float4 nr1,
                                  float4 nr2, float4 nr3, uint32_t b_new, uint32_t n_wg) {
    for (; rb < n_blocks; rb += n_wg * SC_ROWS_WG) {
        float4 p[2][4];
        score_load(p, pool, rb, n_vis, lane, wave);
        score_store(qr, p, srow, rb, n_blocks, n_vis, lane, wave, nr0, nr1, nr2, nr3, b_new);
    }
}

/* Streaming block scores for few tokens (decode: one token at the device
 * position). Token t = blockIdx.y; rows b < n_vis get sum_h relu(q_h . pool_b),
 * n_vis <= b < n_blocks get -1e30 (src/q4_rocm.cu:7412-7445, 7476-7503).
 * DEV: the device position bounds the rows written to b < n_vis. */
template <bool DEV>
__global__ __launch_bounds__(256) void qsa_score_v_k(const float *q, const float *pool,
                                                     float *score, uint32_t n_blocks,
                                                     uint32_t stride, uint32_t n_head,
                                                     uint32_t pos0, uint32_t ratio,
                                                     const int32_t *pp) {
    const uint32_t t = blockIdx.y;
    const uint32_t pos = (DEV ? (uint32_t)*pp : pos0) + t;
    const uint32_t n_vis = ratio ? (pos + 1) / ratio : 0;
    if (DEV) n_blocks = n_vis;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t g = lane & 7u;
    uint32_t rb = blockIdx.x * SC_ROWS_WG;
    if (rb >= n_blocks) return;

    /* lane g of a row group holds dims {32i + 4g .. +3 : i < 4} of each query */
    float4 qr[4][4];
#pragma unroll
    for (int h = 0; h < 4; h++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            qr[h][i] = (uint32_t)h < n_head
                           ? ld_vec((const float4 *)(q + ((size_t)t * n_head + h) * IDX_HD +
                                                  32 * i + 4 * g))
                           : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    score_rows(qr, pool, score + (size_t)t * stride, rb, n_blocks, n_vis, lane, wave, z, z, z, z,
               0xffffffffu, gridDim.x);
}

/* The decode indexer step in one launch (no reference counterpart; it is
 * q4_hip_f32_to_f16_d + q4_hip_qsa_pool_d + q4_hip_qsa_k_prep_d +
 * q4_hip_qsa_score_d of src/q4_fwd.c:904-916, fused): workgroup 0 stores
 * the new raw key at the device position; every workgroup prepares the
 * indexer queries itself (RMSNorm * wn_q + RoPE at pos, one wave per head,
 * into LDS); the workgroup whose rows hold the block this position
 * completes pools it (with the new key's fp16 row in place of the stored
 * one) and writes it to the pool; then every workgroup scores its 64 rows.
 * q is read, not modified. The first n_wg workgroups do this; any after them
 * write a held cache append (app). */
template <bool BATCH>
__global__ __launch_bounds__(256) void qsa_index_score_dk(uint32_t *raw2, float *pool,
                                                          const float *wn_k, const float *k_new,
                                                          const float *q, const float *wn_q,
                                                          float *score, uint32_t n_head,
                                                          uint32_t ratio, uint32_t n_rot,
                                                          float base, float eps,
                                                          const int32_t *pp,
                                                          const q4kv_index_desc *descs,
                                                          uint32_t n_wg, q4kv_app_args app) {
    if (!BATCH && blockIdx.x >= n_wg) {
        q4kv_app_wg(app, blockIdx.x - n_wg);
        return;
    }
    __shared__ float qs[4][IDX_HD];
    __shared__ float new_row[IDX_HD];
    uint32_t pos;
    if (BATCH) { /* item blockIdx.y of a batch: its own buffers and position */
        const q4kv_index_desc *d = descs + blockIdx.y;
        raw2 = q4kv_gptr<uint32_t>(ldg((const uintptr_t *)&d->raw));
        pool = q4kv_gptr_at(&d->pool);
        wn_k = q4kv_gptr_at(&d->wn_k);
        k_new = q4kv_gptr_at(&d->k_new);
        q = q4kv_gptr_at(&d->q);
        wn_q = q4kv_gptr_at(&d->wn_q);
        score = q4kv_gptr_at(&d->score);
        pos = ldg(&d->pos);
    } else {
        pos = (uint32_t)*pp;
    }
    const uint32_t n_vis = (pos + 1) / ratio;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t rb = blockIdx.x * SC_ROWS_WG;
    /* the small loads first (the new key pair this lane owns, dims 2*lane and
     * 2*lane+1; its query pair; its RMSNorm weights), branch-free, then this
     * workgroup's first 64 rows: the query preparation below waits only for
     * the small ones and overlaps the rows (row b_new, pooled below, is
     * replaced before use); rows past the grid follow in grid strides */
    const float2 kn = ld_vec((const float2 *)k_new + lane);
    float2 x = ld_vec((const float2 *)(q + (wave < n_head ? wave : 0u) * IDX_HD) + lane);
    float2 w = ld_vec((const float2 *)(wn_q ? wn_q : k_new) + lane);
    const bool live = rb < n_vis;
    float4 p[2][4];
    asm volatile("" ::: "memory");
    score_load(p, pool, rb, n_vis, lane, wave); /* no branch: workgroups past n_vis
                                                     * re-read the last row, unused */
    const uint32_t kh = (uint32_t)__half_as_ushort(__float2half_rn(kn.x)) |
                        ((uint32_t)__half_as_ushort(__float2half_rn(kn.y)) << 16);
    if (blockIdx.x == 0 && wave == 0) stg(raw2 + (size_t)pos * (IDX_HD / 2) + lane, kh);
    if (!live) return;
    const float freq = 2 * lane < n_rot ? rope_freq(base, lane, n_rot / 2) : 0.f;
    /* indexer queries: wave h prepares head h (qsa_prep_k's arithmetic) */
    {
        if (wave >= n_head) x = make_float2(0.f, 0.f);
        if (!wn_q) w = make_float2(1.f, 1.f);
        float ss = fmaf(x.x, x.x, 0.f);
        ss = fmaf(x.y, x.y, ss);
        ss = wave_sum(ss);
        const float scale = __fdiv_rn(1.f, __fsqrt_rn(__fdiv_rn(ss, (float)IDX_HD) + eps));
        float y0 = x.x * scale * w.x, y1 = x.y * scale * w.y;
        if (2 * lane < n_rot) rope_rotate(y0, y1, (float)pos, freq);
        if (wave >= n_head) y0 = y1 = 0.f;
        qs[wave][2 * lane] = y0;
        qs[wave][2 * lane + 1] = y1;
    }
    const bool completes = (pos + 1) % ratio == 0;
    const uint32_t b_new = completes ? n_vis - 1 : 0xffffffffu;
    /* the workgroup whose grid-stride row groups hold b_new pools it */
    if (completes && (b_new / SC_ROWS_WG) % n_wg == blockIdx.x && wave == 0) {
        const float2 v = pool_block(raw2, pool, wn_k, ratio, b_new, n_rot, freq, eps, lane,
                                    true, kh);
        new_row[2 * lane] = v.x;
        new_row[2 * lane + 1] = v.y;
    }
    __syncthreads();
    const uint32_t g = lane & 7u;
    float4 qr[4][4], nr[4];
#pragma unroll
    for (int h = 0; h < 4; h++)
#pragma unroll
        for (int i = 0; i < 4; i++) qr[h][i] = *(const float4 *)&qs[h][32 * i + 4 * g];
#pragma unroll
    for (int i = 0; i < 4; i++) nr[i] = *(const float4 *)&new_row[32 * i + 4 * g];
    score_store(qr, p, score, rb, n_vis, n_vis, lane, wave, nr[0], nr[1], nr[2], nr[3], b_new);
    score_rows(qr, pool, score, rb + n_wg * SC_ROWS_WG, n_vis, n_vis, lane, wave, nr[0],
               nr[1], nr[2], nr[3], b_new, n_wg);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

/* fp32 -> (hi, lo) bf16 pairs, both by truncation: hi = x's top 16 bits,
 * lo = the top 16 bits of x - hi (exact in fp32), so x = hi + lo to within
 * 2^-16 |x|. Two values per dword, low half first. */
__device__ inline void split_bf16(const float4 &a, const float4 &b, s16x8 &hi, s16x8 &lo) {
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t u0 = __float_as_uint(v[2 * i]), u1 = __float_as_uint(v[2 * i + 1]);
        const uint32_t h0 = u0 & 0xffff0000u, h1 = u1 & 0xffff0000u;
        const uint32_t l0 = __float_as_uint(v[2 * i] - __uint_as_float(h0));
        const uint32_t l1 = __float_as_uint(v[2 * i + 1] - __uint_as_float(h1));
        h[i] = __builtin_amdgcn_perm(h1, h0, 0x07060302u); /* {h0.hi16, h1.hi16} */
        l[i] = __builtin_amdgcn_perm(l1, l0, 0x07060302u);
    }
    hi = __builtin_bit_cast(s16x8, (uint4){h[0], h[1], h[2], h[3]});
    lo = __builtin_bit_cast(s16x8, (uint4){l[0], l[1], l[2], l[3]});
}

/* Block scores for a chunk of >= 4 tokens on bf16 MFMA 16x16x32 with a
 * three-product split (hi.hi + hi.lo + lo.hi, relative error ~2^-16 per
 * product, fp32 accumulation). A tile = 4 tokens x 4 heads (row 4*token +
 * head), B tile = 16 pool rows; at k-step s lane l supplies dims
 * 32s + 8(l/16) .. +7 of its row (32 contiguous bytes: a row's 128 bytes per
 * step come from its four lanes). The C layout puts one token's four heads in
 * a lane's four accumulators, so the relu-sum over heads stays in the lane.
 * Workgroup tile: 16 tokens x 256 blocks, 64 blocks per wave. */
__global__ __launch_bounds__(256) void qsa_score_mfma_k(const float *q, const float *pool,
                                                        float *score, uint32_t n_tok,
                                                        uint32_t n_blocks, uint32_t stride,
                                                        uint32_t n_head, uint32_t pos0,
                                                        uint32_t ratio) {
    /* the A operands (the workgroup's 16 tokens x 4 heads) are the same for
     * its four waves: wave w loads and splits k-step w once, into LDS */
    __shared__ s16x8 a_hi[4][4][64], a_lo[4][4][64]; /* [k-step][tile][lane] */
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t i16 = lane & 15u, kq = lane >> 4;
    const uint32_t tok0 = blockIdx.y * 16u;
    const uint32_t blk0 = blockIdx.x * 256u + wave * 64u;
    if (blockIdx.x * 256u >= n_blocks) return;

    const float *ap[4];
    bool av[4];
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const uint32_t tok = tok0 + 4u * a + (i16 >> 2), head = i16 & 3u;
        av[a] = tok < n_tok && head < n_head;
        ap[a] = q + ((size_t)(av[a] ? tok : 0) * n_head + (av[a] ? head : 0)) * IDX_HD + 8u * kq;
    }
    const float *bp[4];
#pragma unroll
    for (int b = 0; b < 4; b++) {
        uint32_t blk = blk0 + 16u * b + i16;
        blk = blk < n_blocks ? blk : n_blocks - 1;
        bp[b] = pool + (size_t)blk * IDX_HD + 8u * kq;
    }
    /* every A load is issued (ap points at a real row for any lane) and
     * padding lanes are zeroed by a mask afterwards: a load under the lane's
     * condition would wait for itself. The first k-step's B rows are
     * requested in the same round trip. */
    float4 xa[4][2], yb[2][4][2];
#pragma unroll
    for (int a = 0; a < 4; a++) {
        xa[a][0] = ld_vec((const float4 *)(ap[a] + 32u * wave));
        xa[a][1] = ld_vec((const float4 *)(ap[a] + 32u * wave) + 1);
    }
    auto load_b = [&](uint32_t st, float4 (&y)[4][2]) {
#pragma unroll
        for (int b = 0; b < 4; b++) {
            y[b][0] = ld_vec((const float4 *)(bp[b] + 32u * st));
            y[b][1] = ld_vec((const float4 *)(bp[b] + 32u * st) + 1);
        }
    };
    load_b(0u, yb[0]);
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const uint32_t m = av[a] ? ~0u : 0u;
        float4 x[2];
#pragma unroll
        for (int h = 0; h < 2; h++)
            x[h] = make_float4(__uint_as_float(__float_as_uint(xa[a][h].x) & m),
                               __uint_as_float(__float_as_uint(xa[a][h].y) & m),
                               __uint_as_float(__float_as_uint(xa[a][h].z) & m),
                               __uint_as_float(__float_as_uint(xa[a][h].w) & m));
        split_bf16(x[0], x[1], a_hi[wave][a][lane], a_lo[wave][a][lane]);
    }
    __syncthreads();
    if (blk0 >= n_blocks) return;
    f32x4 acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = (f32x4){0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (uint32_t st = 0; st < 4; st++) {
        s16x8 Ah[4], Al[4], Bh[4], Bl[4];
#pragma unroll
        for (int a = 0; a < 4; a++) {
            Ah[a] = a_hi[st][a][lane];
            Al[a] = a_lo[st][a][lane];
        }
        if (st + 1u < 4u) load_b(st + 1u, yb[(st + 1u) & 1u]);
#pragma unroll
        for (int b = 0; b < 4; b++) split_bf16(yb[st & 1u][b][0], yb[st & 1u][b][1], Bh[b], Bl[b]);
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al[a], Bh[b], acc[a][b], 0, 0, 0);
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah[a], Bl[b], acc[a][b], 0, 0, 0);
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah[a], Bh[b], acc[a][b], 0, 0, 0);
            }
    }
    /* lane holds C[4*kq + r][i16]: token tok0 + 4a + kq, head r, block blk0 + 16b + i16 */
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const uint32_t tok = tok0 + 4u * a + kq;
        if (tok >= n_tok) continue;
        const uint32_t pos = pos0 + tok;
        const uint32_t n_vis = ratio ? (pos + 1) / ratio : 0;
        float *srow = score + (size_t)tok * stride;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t blk = blk0 + 16u * b + i16;
            if (blk >= n_blocks) continue;
            float s = 0.f;
#pragma unroll
            for (int r = 0; r < 4; r++) s += fmaxf(acc[a][b][r], 0.f);
            srow[blk] = blk < n_vis ? s : -1.0e30f;
        }
    }
}

/* --------------------------------------------------------------- topk ---- */

constexpr uint32_t TK_T = 1024;        /* threads per row workgroup */
constexpr uint32_t TK_KPT = 64;        /* register-resident keys per thread (long rows) */
constexpr uint32_t TK_MAXK = 512;      /* largest k_blk */
constexpr uint32_t TK_CAP = 4096;      /* candidate list capacity */
constexpr uint32_t TK_DSHIFT = 19;     /* coarse bins: 1/16 octave of |score| */
constexpr uint32_t TK_DBINS = 512;     /* distance bins from the row maximum */
constexpr uint32_t TK_CBITS = 10;      /* widest digit of the candidate passes */

/* Order-preserving uint32 key (src/q4_rocm.cu:7471-7474). */
__device__ inline uint32_t xkey(float f) {
    const uint32_t u = __float_as_uint(f);
    /* negative: all bits flipped; otherwise the sign bit set */
    return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}

/* HC histogram copies per bin (lane & (HC - 1) picks one: with 32, a
 * half-wave's atomics land on distinct banks); CAP candidate capacity. */
template <uint32_t HC, uint32_t CAP> union TopkHist {
    uint32_t rep[256 * HC];          /* full path: 256 bins x HC copies */
    uint32_t dist[TK_DBINS * HC];    /* distance bins x HC copies */
    uint32_t cand[1u << TK_CBITS];   /* candidate passes */
};
template <uint32_t HC, uint32_t CAP, uint32_t NT> struct TopkSmem {
    TopkHist<HC, CAP> h;
    uint32_t cg[NT], ce[NT];         /* per (key row, wave) counts -> offsets */
    uint64_t wm[NT];                 /* per (key row, wave) candidate lane masks */
    uint32_t ckey[CAP];              /* candidates in index order */
    int32_t cidx[CAP];
    uint32_t bins[TK_DBINS];
    uint32_t wtot[3][16];
    int32_t chosen[TK_MAXK];
    uint32_t st[8];
};

/* Inclusive prefix sum over the 64 lanes (DPP row shifts + row broadcasts). */
__device__ inline uint32_t wave_incl_scan(uint32_t x) {
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false); /* row_shr:1 */
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false); /* row_shr:2 */
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false); /* row_shr:4 */
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false); /* row_shr:8 */
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false); /* row_bcast:15 */
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false); /* row_bcast:31 */
    return x;
}
__device__ inline uint32_t wave_max_u32(uint32_t x) {
    x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false));
    x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false));
    x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false));
    x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false));
    x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false));
    x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
/* Exclusive prefix sum over the NW waves' threads in thread order; *total
 * gets the sum. Uses wtot[0]; ends with a barrier so wtot may be reused. */
template <uint32_t NW = 16>
__device__ inline uint32_t block_excl_scan(uint32_t v, uint32_t *wtot, uint32_t *total) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t inc = wave_incl_scan(v);
    if (lane == 63) wtot[wave] = inc;
    __syncthreads();
    uint32_t pre = 0, tot = 0;
#pragma unroll
    for (uint32_t w = 0; w < NW; w++) {
        const uint32_t x = wtot[w];
        pre += w < wave ? x : 0u;
        tot += x;
    }
    __syncthreads();
    *total = tot;
    return pre + inc - v;
}

/* The same without the trailing barrier: the caller separates two uses of
 * one wtot buffer by another barrier. Returns the exclusive prefix. */
template <uint32_t NW = 16>
__device__ inline uint32_t block_excl_scan_nb(uint32_t v, uint32_t *wtot) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t inc = wave_incl_scan(v);
    if (lane == 63) wtot[wave] = inc;
    __syncthreads();
    uint32_t pre = 0;
#pragma unroll
    for (uint32_t w = 0; w < NW; w++) pre += w < wave ? wtot[w] : 0u;
    return pre + inc - v;
}

/* Write the wave-uniform value n into lane R of v (v_writelane_b32). */
template <uint32_t R> __device__ inline uint32_t set_lane(uint32_t v, uint32_t n) {
    asm("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(n), "i"(R));
    return v;
}
/* f(integral_constant<0>) ... f(integral_constant<N-1>), fully unrolled. */
template <class F, uint32_t... I>
__device__ inline void unroll_seq(F &&f, std::integer_sequence<uint32_t, I...>) {
    (f(std::integral_constant<uint32_t, I>{}), ...);
}
template <uint32_t N, class F> __device__ inline void unroll(F &&f) {
    unroll_seq(f, std::make_integer_sequence<uint32_t, N>{});
}

__device__ inline uint32_t lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

/* One token row: exact top-`need` blocks by (key desc, index asc), emitted
 * above-threshold ascending then threshold ties ascending, expanded to sel.
 * Same list as src/q4_rocm.cu:7736-7846 (and the device-position pipeline
 * :7505-7696). Keys of row element e = c*TK_T*KPT + r*TK_T + tid live in
 * key[r] during chunk c (KPT keys per thread: 16 for rows of up to 16384
 * blocks, 64 for longer ones).
 *
 * Fast path (rows of <= 65536 blocks): one histogram pass of the distance
 * from the row maximum finds the bin holding the need-th key; every key in
 * that bin or nearer is a candidate (typically 1-3 x need). When they fit
 * in TK_CAP, the candidates are compacted in index order into LDS and the
 * exact threshold is found by 12-bit radix passes over them alone.
 * Otherwise (long rows, heavy ties) the full path runs four 8-bit radix
 * passes over all keys and an ordered compaction of all keys. */
/* Where a row comes from: token rows pos0 + t of one score matrix, the
 * device position's single row, or item t of a batch of descriptors. */
enum { TK_ROWS = 0, TK_DEV = 1, TK_BATCH = 2 };

/* Rows of up to 8 keys per thread (8192 blocks) take a smaller instance: 16
 * histogram copies and 2048 candidates, so that two workgroups share a CU
 * (with 8 copies the histogram's bank conflicts cost the prefill indexer
 * 1.2 %). */
template <uint32_t KPT, uint32_t NT = TK_T> struct TopkShape {
    static constexpr bool SMALL = KPT * NT <= 8192u; /* rows of up to 8192 blocks */
    static constexpr uint32_t HC = SMALL ? 16u : 32u;
    static constexpr uint32_t CAP = SMALL ? 2048u : TK_CAP;
    static constexpr int WG_PER_CU = SMALL ? 2 : 1; /* LDS allows two */
};

/* Split selection of one device-position row of up to 65536 keys: workgroup
 * w of G reduces keys w*8192 .. +8191 (TK_T * TKS_KPS) to its local candidates (its keys
 * within the distance bin where its own count reaches need: every key of
 * the row's top need is among them, since such a key has fewer than need
 * greater keys in the row, so in its slice), in index order, plus its
 * distance histogram and maximum. The last workgroup to finish (a ticket
 * taken after an agent-scope release) merges the G histograms, keeps the
 * candidates at or above the row's bin and finishes as the one-workgroup
 * kernel does. One buffer per GPU: launches on one GPU must not overlap
 * (the library issues every launch on its one stream). */
constexpr uint32_t TKS_KPS = 8;       /* keys per thread of a slice: 8192-key slices */
constexpr uint32_t TKS_G = 8;         /* most slices of a row (65536 keys) */
constexpr uint32_t TKS_CAPW = 1024;   /* local candidates per workgroup */
constexpr uint32_t TKS_HC = 8;        /* local histogram copies */
struct TopkSplitScratch {
    uint32_t hist[TKS_G][TK_DBINS];
    uint32_t mx[TKS_G], cnt[TKS_G]; /* cnt 0xffffffff: more than TKS_CAPW */
    uint32_t ticket;
    uint32_t key[TKS_G][TKS_CAPW];
    uint32_t idx[TKS_G][TKS_CAPW];
};
/* agent-scope (sc1) accesses of the split scratch */
__device__ inline void st_agent(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t ld_agent(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int TKS_SC1 = 16; /* buffer-load cache policy: sc1 */
__device__ TopkSplitScratch tks_scratch;

template <int SRC, uint32_t KPT, uint32_t SPLIT = 0, uint32_t NT = TK_T>
__global__ __launch_bounds__(NT, (TopkShape<KPT, NT>::WG_PER_CU)) void qsa_topk_k(const float *score, int32_t *sel,
                                                   uint32_t stride, uint32_t k_blk,
                                                   uint32_t ratio, uint32_t pos0,
                                                   uint32_t width, const int32_t *pp,
                                                   const q4kv_index_desc *descs) {
    constexpr uint32_t HC = TopkShape<KPT, NT>::HC, CAP = TopkShape<KPT, NT>::CAP;
    constexpr uint32_t NW = NT / 64u; /* waves */
    __shared__ TopkSmem<HC, CAP, NT> sm;
    static_assert(!SPLIT || (SRC == TK_DEV && NT == TK_T), "split rows: device-position, 1024 threads");
    static_assert(NT >= 256u && NT <= TK_T && KPT * NW <= NT && CAP % NT == 0u, "row layout");
    /* t: the row (token or batch item); with SPLIT the slice of the one row */
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const uint32_t lane = tid & 63u, wave = tid >> 6;
    const uint32_t rowi = SPLIT ? 0u : t;
    uint32_t pos;
    const float *row;
    int32_t *out;
    if (SRC == TK_BATCH) {
        const q4kv_index_desc *d = descs + rowi;
        pos = ldg(&d->pos);
        row = q4kv_gptr_at(&d->score);
        out = q4kv_gptr_at(&d->sel);
    } else {
        pos = (SRC == TK_DEV ? (uint32_t)*pp : pos0) + rowi;
        row = score + (size_t)rowi * stride;
        out = sel + (size_t)rowi * width;
    }
    const uint32_t n_vis = (pos + 1) / ratio;
    const uint32_t need = n_vis < k_blk ? n_vis : k_blk;
    if (need == n_vis) { /* every complete block fits: the dense prefix */
        if (SPLIT && t != 0) return;
        for (uint32_t w = tid; w < width; w += NT) stg(out + w, w <= pos ? (int32_t)w : -1);
        return;
    }
    constexpr uint32_t TK_CHUNK = NT * KPT;
    const uint32_t nchunk = (n_vis + TK_CHUNK - 1) / TK_CHUNK;
    uint32_t key[KPT];
    /* Elements past n_vis get key 0, the smallest key. Since need <= n_vis
     * they sort below the need-th largest real key (or tie with it only when
     * that key is 0), so the radix passes need no validity test; the
     * compactions check validity where a threshold can be 0. */
    auto load_chunk = [&](uint32_t c) {
        const float *src = row + (size_t)c * TK_CHUNK;
        const uint32_t lim = n_vis - c * TK_CHUNK;
        if (lim >= TK_CHUNK) {
#pragma unroll
            for (uint32_t r = 0; r < KPT; r++) key[r] = xkey(ldg(src + r * NT + tid));
        } else {
            /* a partial chunk through a buffer resource of lim elements:
             * loads past it return 0 with no branch, so all KPT loads are in
             * flight together (a load under a per-element branch waits for
             * itself); those elements then take key 0 */
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)src, (short)0, (int)(lim * 4u), 0x00020000);
#pragma unroll
            for (uint32_t r = 0; r < KPT; r++)
                key[r] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(tid * 4u),
                                                              (int)(r * NT * 4u), 0);
#pragma unroll
            for (uint32_t r = 0; r < KPT; r++) {
                /* xkey with its sign-bit term only where the element is in
                 * the row: past it the word loaded is 0 and its key then 0,
                 * with no select (which would move the load under it) */
                const uint32_t u = key[r];
                const uint32_t in = (r * NT + tid - lim) & 0x80000000u;
                key[r] = u ^ ((uint32_t)((int32_t)u >> 31) | in);
            }
        }
    };
    auto valid = [&](uint32_t c, uint32_t r) { return c * TK_CHUNK + r * NT + tid < n_vis; };

    bool fast = nchunk == 1;
    uint32_t above = 0, ncand = 0, Kc = 0;
    if constexpr (SPLIT != 0) {
        /* ---- this workgroup's slice (SK keys, SPLIT per thread): keys,
         * maximum, distance histogram ---- */
        constexpr uint32_t KS = SPLIT, SK = NT * KS;
        constexpr uint32_t GMAX = TK_CHUNK / SK, P = (NT / 64u) / GMAX; /* waves per slice */
        static_assert(GMAX <= TKS_G && P >= 1u, "slices fit the scratch and the waves");
        constexpr uint32_t LR = TKS_CAPW / P, LK = LR / 64u; /* list entries per wave, per lane */
        const uint32_t G = gridDim.x, base = t * SK;
        const uint32_t lim = n_vis > base ? min(n_vis - base, SK) : 0u;
        TopkSplitScratch &gs = tks_scratch;
        for (uint32_t i = tid; i < TK_DBINS * TKS_HC; i += NT) sm.h.dist[i] = 0;
        uint32_t ks[KS];
        {
            /* loads past the slice's visible keys return 0 (buffer bound),
             * whose key is then 0, as load_chunk's partial chunk */
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(row + base), (short)0, (int)(lim * 4u), 0x00020000);
#pragma unroll
            for (uint32_t r = 0; r < KS; r++)
                ks[r] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(tid * 4u),
                                                             (int)(r * NT * 4u), 0);
#pragma unroll
            for (uint32_t r = 0; r < KS; r++) {
                const uint32_t u = ks[r];
                const uint32_t in = (r * NT + tid - lim) & 0x80000000u;
                ks[r] = u ^ ((uint32_t)((int32_t)u >> 31) | in);
            }
        }
        uint32_t mx = 0;
#pragma unroll
        for (uint32_t r = 0; r < KS; r++) mx = max(mx, ks[r]);
        mx = wave_max_u32(mx);
        if (lane == 0) sm.wtot[1][wave] = mx;
        __syncthreads();
        uint32_t M = 0;
#pragma unroll
        for (uint32_t w = 0; w < NW; w++) M = max(M, sm.wtot[1][w]);
        const uint32_t Mb = M >> TK_DSHIFT;
        uint32_t dist[KS];
#pragma unroll
        for (uint32_t r = 0; r < KS; r++) {
            dist[r] = min(Mb - (ks[r] >> TK_DSHIFT), TK_DBINS - 1u);
            if (r * NT + tid < lim)
                atomicAdd(sm.h.dist + (lane & (TKS_HC - 1u)) + dist[r] * TKS_HC, 1u);
        }
        __syncthreads();
        if (tid < TK_DBINS) { /* fold the copies, in an order rotated by the bin */
            const uint32_t *hp = sm.h.dist + tid * TKS_HC;
            uint32_t v = 0;
#pragma unroll
            for (uint32_t i = 0; i < TKS_HC; i++) v += hp[(i + tid) & (TKS_HC - 1u)];
            sm.bins[tid] = v;
            st_agent(&gs.hist[t][tid], v);
        }
        if (tid == 0) sm.st[0] = TK_DBINS - 1u; /* fewer than need keys: all */
        __syncthreads();
        if (wave == 0) { /* the nearest bin where this slice's count reaches need */
            uint32_t c[8], s = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) { c[i] = sm.bins[8u * lane + i]; s += c[i]; }
            uint32_t acc = wave_incl_scan(s) - s;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (acc < need && acc + c[i] >= need) sm.st[0] = 8u * lane + i;
                acc += c[i];
            }
        }
        __syncthreads();
        /* ---- local candidates in index order: (r, wave) counts by ballot,
         * one wave scan over the 16 KS groups (KS / 4 per lane) ---- */
        const uint32_t Bw = sm.st[0];
        uint64_t cm[KS];
#pragma unroll
        for (uint32_t r = 0; r < KS; r++) {
            cm[r] = __ballot((r * NT + tid < lim) & (dist[r] <= Bw));
            if (lane == 0) sm.cg[r * 16u + wave] = (uint32_t)__popcll(cm[r]);
        }
        __syncthreads();
        if (wave == 0) {
            constexpr uint32_t GL = KS / 4u; /* groups per lane */
            uint32_t v[GL], s = 0;
#pragma unroll
            for (uint32_t i = 0; i < GL; i++) { v[i] = sm.cg[GL * lane + i]; s += v[i]; }
            const uint32_t inc = wave_incl_scan(s);
            uint32_t o = inc - s;
#pragma unroll
            for (uint32_t i = 0; i < GL; i++) { sm.ce[GL * lane + i] = o; o += v[i]; }
            if (lane == 63) sm.st[1] = inc;
        }
        __syncthreads();
        const uint32_t cw = sm.st[1];
        if (cw <= TKS_CAPW) {
#pragma unroll
            for (uint32_t r = 0; r < KS; r++) {
                if ((cm[r] >> lane) & 1u) {
                    const uint32_t i = sm.ce[r * 16u + wave] + lanes_below(cm[r]);
                    st_agent(&gs.key[t][i], ks[r]);
                    st_agent(&gs.idx[t][i], base + r * NT + tid);
                }
            }
        }
        if (tid == 0) {
            st_agent(&gs.mx[t], M);
            st_agent(&gs.cnt[t], cw <= TKS_CAPW ? cw : 0xffffffffu);
        }
        /* ---- the ticket. Everything the merge reads is stored and loaded
         * at agent scope (sc1: coherent across the XCDs' L2s), so the last
         * workgroup needs no L2 invalidate (an acquire fence costs ~1.5 us
         * here): each wave waits for its stores, and after the barrier one
         * release orders them before the ticket ---- */
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            sm.st[3] = __hip_atomic_fetch_add(&gs.ticket, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (sm.st[3] != G - 1u) return;
        if (tid == 0) st_agent(&gs.ticket, 0u);
        /* ---- one round trip for everything the merge reads: the slices'
         * maxima and counts, their histograms (thread: bin hb of slices
         * hw0, hw0 + 2, ...) and their lists (wave w: part w % P of slice
         * w / P, LK entries per lane; entries past a list's count are
         * masked after) ---- */
        uint32_t mxv = 0, cntv = 0;
        if (tid < G) {
            mxv = ld_agent(&gs.mx[tid]);
            cntv = ld_agent(&gs.cnt[tid]);
        }
        const uint32_t hb = tid & (TK_DBINS - 1u), hw0 = tid / TK_DBINS;
        constexpr uint32_t HL = (GMAX + 1u) / 2u;
        uint32_t hv[HL];
#pragma unroll
        for (uint32_t i = 0; i < HL; i++)
            hv[i] = ld_agent(&gs.hist[min(hw0 + 2u * i, G - 1u)][hb]);
        const uint32_t ls = min(wave / P, G - 1u), lp = wave % P;
        uint32_t kk[LK], ii[LK];
        {
            const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
                (void *)&gs.key[ls][lp * LR], (short)0, (int)(LR * 4u), 0x00020000);
            const __amdgpu_buffer_rsrc_t ri = __builtin_amdgcn_make_buffer_rsrc(
                (void *)&gs.idx[ls][lp * LR], (short)0, (int)(LR * 4u), 0x00020000);
#pragma unroll
            for (uint32_t i = 0; i < LK; i++)
                kk[i] = __builtin_amdgcn_raw_buffer_load_b32(rk, (int)(lane * 4u), (int)(i * 256u),
                                                             TKS_SC1);
#pragma unroll
            for (uint32_t i = 0; i < LK; i++)
                ii[i] = __builtin_amdgcn_raw_buffer_load_b32(ri, (int)(lane * 4u), (int)(i * 256u),
                                                             TKS_SC1);
        }
        if (tid < G) {
            sm.cg[tid] = mxv;
            sm.ce[tid] = cntv;
        }
        if (tid < TK_DBINS) sm.bins[tid] = 0;
        for (uint32_t i = tid; i < (1u << TK_CBITS); i += NT) sm.h.cand[i] = 0;
        if (tid == 0) sm.st[0] = TK_DBINS - 1u;
        __syncthreads();
        uint32_t Mg = 0;
        bool ovf = false;
        for (uint32_t w = 0; w < G; w++) {
            Mg = max(Mg, sm.cg[w]);
            ovf |= sm.ce[w] == 0xffffffffu;
        }
        const uint32_t Mgb = Mg >> TK_DSHIFT;
#pragma unroll
        for (uint32_t i = 0; i < HL; i++) {
            const uint32_t w = hw0 + 2u * i;
            if (w < G && hv[i])
                atomicAdd(&sm.bins[min(hb + (Mgb - (sm.cg[w] >> TK_DSHIFT)), TK_DBINS - 1u)], hv[i]);
        }
        __syncthreads();
        if (wave == 0) { /* the nearest bin where the row's count reaches need */
            uint32_t c[8], s = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) { c[i] = sm.bins[8u * lane + i]; s += c[i]; }
            uint32_t acc = wave_incl_scan(s) - s;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (acc < need && acc + c[i] >= need) {
                    sm.st[0] = 8u * lane + i;
                    sm.st[1] = acc;
                }
                acc += c[i];
            }
        }
        __syncthreads();
        const uint32_t B = sm.st[0];
        above = sm.st[1];
        Kc = (Mgb - B) << TK_DSHIFT;
        fast = B < min(Mgb, TK_DBINS - 1u) && !ovf && n_vis <= G * SK;
        if (fast) {
            /* ---- the lists' keys >= Kc; the waves' survivor counts in wave
             * order (slice, then part: index order) give each its offset ---- */
            const uint32_t cnt_w = wave / P < G ? sm.ce[wave / P] : 0u;
            const uint32_t e0 = lp * LR + lane;
            uint32_t n = 0;
#pragma unroll
            for (uint32_t i = 0; i < LK; i++)
                n += (uint32_t)__popcll(__ballot(kk[i] >= Kc && e0 + 64u * i < cnt_w));
            if (lane == 0) sm.wtot[2][wave] = n;
            __syncthreads();
            uint32_t o = 0, tot = 0;
#pragma unroll
            for (uint32_t w = 0; w < 16u; w++) {
                const uint32_t v = sm.wtot[2][w];
                o += w < wave ? v : 0u;
                tot += v;
            }
            fast = tot <= CAP;
            ncand = tot;
            if (fast) {
#pragma unroll
                for (uint32_t i = 0; i < LK; i++) {
                    const bool keep = kk[i] >= Kc && e0 + 64u * i < cnt_w;
                    const uint64_t m = __ballot(keep);
                    if (keep) {
                        const uint32_t p = o + lanes_below(m);
                        sm.ckey[p] = kk[i];
                        sm.cidx[p] = (int32_t)ii[i];
                    }
                    o += (uint32_t)__popcll(m);
                }
            }
            __syncthreads();
        }
    } else if (fast) {
        for (uint32_t i = tid; i < TK_DBINS * HC; i += NT) sm.h.dist[i] = 0;
        sm.wm[tid] = 0;
        load_chunk(0);
        /* ---- row maximum (as the loads land) ---- */
        uint32_t mx = 0;
#pragma unroll
        for (uint32_t r = 0; r < KPT; r++) mx = max(mx, key[r]);
        mx = wave_max_u32(mx);
        if (lane == 0) sm.wtot[1][wave] = mx;
        __syncthreads();
        uint32_t M = 0;
#pragma unroll
        for (uint32_t w = 0; w < NW; w++) M = max(M, sm.wtot[1][w]);
        /* ---- histogram of the distance from the maximum in 1/16-octave
         * steps of |score| (the keys' bits above bit 19), clamped at 511;
         * 32 copies keep a half-wave's atomics on distinct banks ---- */
        const uint32_t Mb = M >> TK_DSHIFT;
        uint32_t *hc = sm.h.dist + (lane & (HC - 1u));
#pragma unroll
        for (uint32_t r = 0; r < KPT; r++)
            atomicAdd(hc + min(Mb - (key[r] >> TK_DSHIFT), TK_DBINS - 1u) * HC, 1u);
        __syncthreads();
        if constexpr (NT == TK_T) {
            /* fold the copies: two threads per bin, each reading its half in
             * an order rotated by the bin, so a wave's reads spread over the
             * banks (in order, lanes 16 dwords apart would meet 16 to a bank) */
            const uint32_t *hp = sm.h.dist + (tid >> 1) * HC + (tid & 1u) * (HC / 2u);
            uint32_t v = 0;
#pragma unroll
            for (uint32_t i = 0; i < HC / 2u; i++) v += hp[(i + (tid >> 1)) & (HC / 2u - 1u)];
            v += __shfl_xor(v, 1);
            if ((tid & 1u) == 0) sm.bins[tid >> 1] = v;
        } else {
            /* TK_DBINS / NT bins per thread, all copies, rotated by the bin */
#pragma unroll
            for (uint32_t b = tid; b < TK_DBINS; b += NT) {
                const uint32_t *hp = sm.h.dist + b * HC;
                uint32_t v = 0;
#pragma unroll
                for (uint32_t i = 0; i < HC; i++) v += hp[(i + b) & (HC - 1u)];
                sm.bins[b] = v;
            }
        }
        __syncthreads();
        if (wave == 0) { /* the nearest bin where the count reaches need */
            uint32_t c[8], s = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) { c[i] = sm.bins[8u * lane + i]; s += c[i]; }
            uint32_t acc = wave_incl_scan(s) - s;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (acc < need && acc + c[i] >= need) {
                    sm.st[0] = 8u * lane + i; /* bin B */
                    sm.st[1] = acc;           /* keys in nearer bins: selected */
                    sm.st[2] = acc + c[i];    /* candidates: bins <= B */
                }
                acc += c[i];
            }
        }
        __syncthreads();
        const uint32_t B = sm.st[0];
        above = sm.st[1];
        ncand = sm.st[2];
        /* the clamped last bin and the padding keys' bin take the full path */
        fast = B < min(Mb, TK_DBINS - 1u) && ncand <= CAP;
        Kc = (Mb - B) << TK_DSHIFT; /* candidates: key >= Kc */
        if (fast) {
            /* ---- ordered compaction of the candidates: each lane's 64-bit
             * row mask, the (row, wave) lane masks by LDS atomic-or, one
             * block scan, then a loop over each lane's few candidates
             * (the full key is fetched again from the row, an L2 hit) ---- */
            uint32_t mlo = 0, mhi = 0;
#pragma unroll
            for (uint32_t r = 0; r < (KPT < 32 ? KPT : 32); r++) mlo |= key[r] >= Kc ? 1u << r : 0u;
#pragma unroll
            for (uint32_t r = 32; r < KPT; r++) mhi |= key[r] >= Kc ? 1u << (r - 32) : 0u;
            const uint64_t mine0 = ((uint64_t)mhi << 32) | mlo;
            for (uint64_t m = mine0; m; m &= m - 1ull)
                atomicOr(&sm.wm[(uint32_t)__builtin_ctzll(m) * NW + wave], 1ull << lane);
            __syncthreads();
            uint32_t tot;
            const uint32_t off = block_excl_scan<NW>((uint32_t)__popcll(sm.wm[tid]), sm.wtot[0], &tot);
            sm.cg[tid] = off;
            for (uint32_t i = tid; i < (1u << TK_CBITS); i += NT) sm.h.cand[i] = 0;
            __syncthreads();
            const uint64_t below = (1ull << lane) - 1ull;
            for (uint64_t m = mine0; m; m &= m - 1ull) {
                const uint32_t r = (uint32_t)__builtin_ctzll(m);
                const uint32_t j = r * NW + wave;
                const uint32_t i = sm.cg[j] + (uint32_t)__popcll(sm.wm[j] & below);
                const uint32_t e = r * NT + tid;
                sm.ckey[i] = xkey(ldg(row + e));
                sm.cidx[i] = (int32_t)e;
            }
            __syncthreads();
        }
    }
    if (fast) {
        /* ---- exact threshold inside bin B: its keys share the bits above
         * bit 19; two radix passes (10 + 9 bits) over those candidates ---- */
        const uint32_t kb = Kc >> TK_DSHIFT;
        uint32_t pre = 0, gt = above;
        for (uint32_t pass = 0; pass < 2; pass++) {
            const uint32_t lo = pass == 0 ? 9u : 0u, wbits = pass == 0 ? 10u : 9u;
            const uint32_t nd = 1u << wbits;
            for (uint32_t i = tid; i < ncand; i += NT) {
                const uint32_t u = sm.ckey[i];
                const uint32_t v = u & ((1u << TK_DSHIFT) - 1u);
                if ((u >> TK_DSHIFT) == kb && (pass == 0 || (v >> 9) == pre))
                    atomicAdd(&sm.h.cand[(v >> lo) & (nd - 1u)], 1u);
            }
            __syncthreads();
            /* thread t owns digits nd-1-DPT*t .. (descending), DPT of them */
            constexpr uint32_t DPT = (1u << TK_CBITS) / NT;
            uint32_t c[DPT], cs = 0;
#pragma unroll
            for (uint32_t j = 0; j < DPT; j++) {
                const int d = (int)nd - 1 - (int)(DPT * tid + j);
                c[j] = d >= 0 ? sm.h.cand[d] : 0u;
                cs += c[j];
            }
            uint32_t acc = block_excl_scan_nb<NW>(cs, sm.wtot[pass]);
            const uint32_t target = need - gt;
#pragma unroll
            for (uint32_t j = 0; j < DPT; j++) {
                if (acc < target && acc + c[j] >= target) {
                    sm.st[4 + 2 * pass] = nd - 1u - (DPT * tid + j);
                    sm.st[5 + 2 * pass] = acc;
                }
                acc += c[j];
            }
            __syncthreads();
#pragma unroll
            for (uint32_t j = 0; j < DPT; j++) {
                const int d = (int)nd - 1 - (int)(DPT * tid + j);
                if (d >= 0) sm.h.cand[d] = 0;
            }
            pre = pass == 0 ? sm.st[4] : (pre << 9) | sm.st[6];
            gt += sm.st[5 + 2 * pass];
            __syncthreads();
        }
        const uint32_t thr = Kc | pre;
        const uint32_t n_gt = gt, rem = need - n_gt;
        /* ---- ordered output over the index-ordered candidates ---- */
        constexpr uint32_t CPT = CAP / NT; /* candidates per thread */
        uint32_t g = 0, e = 0;
        const uint32_t i0 = CPT * tid;
#pragma unroll
        for (uint32_t j = 0; j < CPT; j++) {
            const uint32_t i = i0 + j;
            if (i < ncand) {
                g += sm.ckey[i] > thr;
                e += sm.ckey[i] == thr;
            }
        }
        const uint32_t pk = block_excl_scan_nb<NW>(g | (e << 16), sm.wtot[2]);
        uint32_t og = pk & 0xffffu, oe = pk >> 16;
#pragma unroll
        for (uint32_t j = 0; j < CPT; j++) {
            const uint32_t i = i0 + j;
            if (i < ncand) {
                const uint32_t u = sm.ckey[i];
                if (u > thr) {
                    if (og < TK_MAXK) sm.chosen[og] = sm.cidx[i];
                    og++;
                } else if (u == thr) {
                    if (oe < rem && n_gt + oe < TK_MAXK) sm.chosen[n_gt + oe] = sm.cidx[i];
                    oe++;
                }
            }
        }
        __syncthreads();
    }
    if (!fast) {
        /* ---- full path: four 8-bit radix passes over every key ---- */
        if (SPLIT && nchunk == 1) load_chunk(0);
        if (tid == 0) { sm.st[4] = 0; sm.st[5] = 0; }
        for (uint32_t pass = 0; pass < 4; pass++) {
            for (uint32_t i = tid; i < 256 * HC; i += NT) sm.h.rep[i] = 0;
            __syncthreads();
            const uint32_t sh = 24u - 8u * pass;
            const uint32_t pre = sm.st[4];
            uint32_t *hcopy = sm.h.rep + (lane & (HC - 1u));
            for (uint32_t c = 0; c < nchunk; c++) {
                if (nchunk > 1) load_chunk(c);
#pragma unroll
                for (uint32_t r = 0; r < KPT; r++) {
                    const uint32_t u = key[r];
                    /* digits above this pass must equal the prefix found so
                     * far (pass 0: the empty prefix, (u >> 8) >> 24 == 0) */
                    if (((u >> 8) >> sh) == pre) atomicAdd(hcopy + ((u >> sh) & 255u) * HC, 1u);
                }
            }
            __syncthreads();
            { /* fold the copies: TPB = NT / 256 lanes per bin, HC / TPB copies
               * each, read in an order rotated by the bin (bank spread, as
               * above) */
                constexpr uint32_t TPB = NT / 256u;
                const uint32_t bin = tid / TPB, part = tid % TPB;
                const uint32_t *hp = sm.h.rep + bin * HC + part * (HC / TPB);
                uint32_t v = 0;
#pragma unroll
                for (uint32_t i = 0; i < HC / TPB; i++) v += hp[(i + bin) & (HC / TPB - 1u)];
                if (TPB > 1u) v += __shfl_xor(v, 1);
                if (TPB > 2u) v += __shfl_xor(v, 2);
                if (part == 0) sm.bins[bin] = v;
            }
            __syncthreads();
            if (wave == 0) { /* digit where the count from the top reaches the target */
                uint32_t c[4], s = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) { c[i] = sm.bins[255u - 4u * lane - i]; s += c[i]; }
                uint32_t acc = wave_incl_scan(s) - s;
                const uint32_t above = sm.st[5];
                const uint32_t target = need - above;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (acc < target && acc + c[i] >= target) {
                        sm.st[4] = (pre << 8) | (255u - 4u * lane - (uint32_t)i);
                        sm.st[5] = above + acc;
                    }
                    acc += c[i];
                }
            }
            __syncthreads();
        }
        const uint32_t thr = sm.st[4];
        const uint32_t n_gt = sm.st[5];
        const uint32_t rem = need - n_gt; /* threshold ties still to take */
        /* ordered compaction; element order is (chunk, r, wave, lane) */
        uint32_t carry_g = 0, carry_e = 0;
        for (uint32_t c = 0; c < nchunk; c++) {
            if (nchunk > 1) load_chunk(c);
            uint32_t gv = 0, ev = 0;
            unroll<KPT>([&](auto rc) {
                constexpr uint32_t r = rc;
                const uint32_t ng = (uint32_t)__popcll(__ballot(key[r] > thr));
                const uint32_t ne = (uint32_t)__popcll(
                    __ballot((key[r] == thr) & ((thr != 0u) | valid(c, r))));
                gv = set_lane<r>(gv, ng);
                ev = set_lane<r>(ev, ne);
            });
            sm.cg[lane * NW + wave] = gv;
            sm.ce[lane * NW + wave] = ev;
            __syncthreads();
            uint32_t tg, te;
            const uint32_t og = block_excl_scan<NW>(sm.cg[tid], sm.wtot[0], &tg);
            const uint32_t oe = block_excl_scan<NW>(sm.ce[tid], sm.wtot[1], &te);
            sm.cg[tid] = og;
            sm.ce[tid] = oe;
            __syncthreads();
            const uint32_t gov = sm.cg[lane * NW + wave], eov = sm.ce[lane * NW + wave];
            uint32_t thr2 = thr;
            asm volatile("" : "+v"(thr2)); /* do not carry the first loop's masks */
#pragma unroll
            for (uint32_t r = 0; r < KPT; r++) {
                const bool gt = key[r] > thr2;
                const bool eq = (key[r] == thr2) & ((thr2 != 0u) | valid(c, r));
                const uint64_t bg = __ballot(gt), be = __ballot(eq);
                const uint32_t e = c * TK_CHUNK + r * NT + tid;
                if (bg) {
                    const uint32_t k = carry_g +
                                       (uint32_t)__builtin_amdgcn_readlane((int)gov, (int)r) +
                                       lanes_below(bg);
                    if (gt && k < TK_MAXK) sm.chosen[k] = (int32_t)e;
                }
                if (be) {
                    const uint32_t k = carry_e +
                                       (uint32_t)__builtin_amdgcn_readlane((int)eov, (int)r) +
                                       lanes_below(be);
                    if (eq && k < rem && n_gt + k < TK_MAXK) sm.chosen[n_gt + k] = (int32_t)e;
                }
            }
            carry_g += tg;
            carry_e += te;
            __syncthreads(); /* cg/ce are rewritten by the next chunk */
        }
    }
    /* expansion (src/q4_rocm.cu:7668-7696, 7830-7845) */
    const uint32_t ncs = need * ratio;
    for (uint32_t w = tid; w < width; w += NT) {
        int32_t v;
        if (w < ncs) {
            const uint32_t i = w / ratio, j = w - i * ratio;
            v = (int32_t)((uint32_t)sm.chosen[i] * ratio + j);
        } else {
            const uint32_t tail = n_vis * ratio + (w - ncs);
            v = tail <= pos ? (int32_t)tail : -1;
        }
        stg(out + w, v);
    }
}

/* --------------------------------------------------------------- prep ---- */


/* RMSNorm * wn, then RoPE of pairs p < n_rot/2 at position pos, for one
 * (token, head) row per wave (src/q4_rocm.cu:6229-6289). GATE: the source
 * row is [x | gate] (2*hd floats) and the gate half is copied to g. Lane l
 * owns pairs p = l + 64m. In place when src == dst (k_prep). */
template <bool GATE>
__global__ __launch_bounds__(256) void qsa_prep_k(const float *src, float *dst, float *g,
                                                  const float *wn, uint32_t n_heads,
                                                  uint32_t hd, uint32_t n_rot, int32_t pos0,
                                                  float base, float eps, uint32_t n_rows,
                                                  const int32_t *pp) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t rowi = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (rowi >= n_rows) return;
    const uint32_t t = rowi / n_heads;
    const int32_t pos = (pp ? *pp : pos0) + (int32_t)t;
    const float *in = src + (size_t)rowi * hd * (GATE ? 2u : 1u);
    if (GATE) {
        float *gd = g + (size_t)rowi * hd;
        for (uint32_t p = lane; p < hd / 2; p += 64u)
            st_vec((float2 *)gd + p, ld_vec((const float2 *)(in + hd) + p));
    }
    q4kv_prep_row(in, dst + (size_t)rowi * hd, wn, hd, n_rot, pos, base, eps, lane);
}

bool prep_launch(const float *src, float *dst, float *g, const float *wn, uint32_t n_heads,
                 uint32_t hd, uint32_t n_rot, int32_t pos0, float base, float eps,
                 uint32_t n_tok, const int32_t *pp, const char *what) {
    if (hd == 0 || (hd & 1u) || hd > 128u * Q4KV_PREP_MAXP || n_rot > hd) {
        Q4KV_ERR("%s: unsupported hd %u / n_rot %u", what, hd, n_rot);
        return false;
    }
    if (((uintptr_t)src | (uintptr_t)dst | (uintptr_t)g | (uintptr_t)wn) & 7u) {
        Q4KV_ERR("%s: buffers must be 8-byte aligned", what);
        return false;
    }
    const uint64_t rows = (uint64_t)n_tok * n_heads;
    if (rows > 0xffffffffull / 4u) return false;
    (void)hipGetLastError();
    const uint32_t grid = (uint32_t)((rows + 3u) / 4u);
    if (g)
        qsa_prep_k<true><<<grid, 256, 0, q4kv_stream>>>(src, dst, g, wn, n_heads, hd, n_rot,
                                                         pos0, base, eps, (uint32_t)rows, pp);
    else
        qsa_prep_k<false><<<grid, 256, 0, q4kv_stream>>>(src, dst, nullptr, wn, n_heads, hd,
                                                          n_rot, pos0, base, eps,
                                                          (uint32_t)rows, pp);
    return q4kv_launch_ok(what);
}

} // namespace

/* ------------------------------------------------------------ C ABI ---- */

extern "C" bool q4_hip_qsa_q_prep_n(const float *d_qg, const float *d_wn, float *d_q,
                                    float *d_g, uint32_t n_head, uint32_t hd, uint32_t n_rot,
                                    int32_t pos0, float base, float eps, uint32_t n_tok) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d_qg || !d_q || !d_g || n_head == 0 || n_tok == 0) return false;
    return prep_launch(d_qg, d_q, d_g, d_wn, n_head, hd, n_rot, pos0, base, eps, n_tok,
                       nullptr, "qsa_q_prep");
}
extern "C" bool q4_hip_qsa_q_prep(const float *d_qg, const float *d_wn, float *d_q, float *d_g,
                                  uint32_t n_head, uint32_t hd, uint32_t n_rot, int32_t pos,
                                  float base, float eps) {
    Q4KV_FLUSH_OR_FAIL();
    return q4_hip_qsa_q_prep_n(d_qg, d_wn, d_q, d_g, n_head, hd, n_rot, pos, base, eps, 1);
}
extern "C" bool q4_hip_qsa_q_prep_d(const float *d_qg, const float *d_wn, float *d_q,
                                    float *d_g, uint32_t n_head, uint32_t hd, uint32_t n_rot,
                                    float base, float eps) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !q4kv_pos_d || !d_qg || !d_q || !d_g || n_head == 0) return false;
    return prep_launch(d_qg, d_q, d_g, d_wn, n_head, hd, n_rot, 0, base, eps, 1, q4kv_pos_d,
                       "qsa_q_prep_d");
}
extern "C" bool q4_hip_qsa_k_prep_n(float *d_k, const float *d_wn, uint32_t n_kvh, uint32_t hd,
                                    uint32_t n_rot, int32_t pos0, float base, float eps,
                                    uint32_t n_tok) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d_k || n_kvh == 0 || n_tok == 0) return false;
    return prep_launch(d_k, d_k, nullptr, d_wn, n_kvh, hd, n_rot, pos0, base, eps, n_tok,
                       nullptr, "qsa_k_prep");
}
extern "C" bool q4_hip_qsa_k_prep(float *d_k, const float *d_wn, uint32_t n_kvh, uint32_t hd,
                                  uint32_t n_rot, int32_t pos, float base, float eps) {
    Q4KV_FLUSH_OR_FAIL();
    return q4_hip_qsa_k_prep_n(d_k, d_wn, n_kvh, hd, n_rot, pos, base, eps, 1);
}
extern "C" bool q4_hip_qsa_k_prep_d(float *d_k, const float *d_wn, uint32_t n_kvh, uint32_t hd,
                                    uint32_t n_rot, float base, float eps) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !q4kv_pos_d || !d_k || n_kvh == 0) return false;
    return prep_launch(d_k, d_k, nullptr, d_wn, n_kvh, hd, n_rot, 0, base, eps, 1, q4kv_pos_d,
                       "qsa_k_prep_d");
}

/* The first call after a held q4_hip_kv_append_d in the reference's decode
 * order (src/q4_fwd.c:891-905): this launch carries the held append. */
extern "C" bool q4_hip_f32_to_f16_d(void *dst_base, uint32_t stride_elems, const float *src,
                                    uint64_t n) {
    const uint64_t grid = (n + 255u) / 256u;
    if (!q4kv_ok || !q4kv_pos_d || !dst_base || !src || !n || grid > 0x7fffffffull) {
        Q4KV_FLUSH_OR_FAIL();
        return false;
    }
    q4kv_app_args app{};
    const uint32_t extra = q4kv_take_held(&app);
    (void)hipGetLastError();
    f16_at_k<<<(uint32_t)grid + extra, 256, 0, q4kv_stream>>>(
        src, (__half *)dst_base, stride_elems, n, q4kv_pos_d, (uint32_t)grid, app);
    return q4kv_launch_ok("f32_to_f16_d");
}

extern "C" bool q4_hip_qsa_pool(const void *raw_f16, float *pool, const float *wn, uint32_t hd,
                                uint32_t ratio, uint32_t b0, uint32_t b1, uint32_t n_rot,
                                float rope_base, float eps) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !raw_f16 || !pool || b1 <= b0 || hd != IDX_HD || ratio == 0 || n_rot > hd)
        return false;
    if (((uintptr_t)raw_f16 & 3u) || ((uintptr_t)pool & 7u)) {
        Q4KV_ERR("qsa_pool: raw must be 4-byte and pool 8-byte aligned");
        return false;
    }
    (void)hipGetLastError();
    const uint32_t nwg = (uint32_t)(((uint64_t)(b1 - b0) + 3u) / 4u);
    const uint32_t grid = nwg < 8192u ? nwg : 8192u;
    qsa_pool_k<<<grid, 256, 0, q4kv_stream>>>((const uint32_t *)raw_f16, pool, wn, ratio, b0, b1,
                                              n_rot, rope_base, eps);
    return q4kv_launch_ok("qsa_pool");
}
extern "C" bool q4_hip_qsa_pool_d(const void *raw_f16, float *pool, const float *wn, uint32_t hd,
                                  uint32_t ratio, uint32_t n_rot, float rope_base, float eps) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !q4kv_pos_d || !raw_f16 || !pool || hd != IDX_HD || ratio == 0 ||
        n_rot > hd)
        return false;
    if (((uintptr_t)raw_f16 & 3u) || ((uintptr_t)pool & 7u)) {
        Q4KV_ERR("qsa_pool_d: raw must be 4-byte and pool 8-byte aligned");
        return false;
    }
    (void)hipGetLastError();
    qsa_pool_dk<<<1, 64, 0, q4kv_stream>>>((const uint32_t *)raw_f16, pool, wn, ratio, n_rot,
                                           rope_base, eps, q4kv_pos_d);
    return q4kv_launch_ok("qsa_pool_d");
}

extern "C" bool q4_hip_qsa_score(const float *q, const float *pool, float *score,
                                 uint32_t n_tok, uint32_t n_blocks, uint32_t stride,
                                 uint32_t n_head, uint32_t hd, uint32_t pos0, uint32_t ratio) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !q || !pool || !score || n_tok == 0 || hd != IDX_HD || n_head == 0 ||
        n_head > 4)
        return false;
    if (n_tok > 1 && n_blocks > stride) {
        Q4KV_ERR("qsa_score: n_blocks %u exceeds the row stride %u", n_blocks, stride);
        return false;
    }
    if (((uintptr_t)q & 15u) || ((uintptr_t)pool & 15u)) {
        Q4KV_ERR("qsa_score: q and pool must be 16-byte aligned");
        return false;
    }
    if (n_blocks == 0) return true;
    (void)hipGetLastError();
    if (n_tok < 4) {
        const uint32_t gx = (n_blocks + SC_ROWS_WG - 1) / SC_ROWS_WG;
        qsa_score_v_k<false><<<dim3(gx, n_tok), 256, 0, q4kv_stream>>>(
            q, pool, score, n_blocks, stride, n_head, pos0, ratio, nullptr);
    } else {
        const uint32_t gx = (n_blocks + 255u) / 256u, gy = (n_tok + 15u) / 16u;
        qsa_score_mfma_k<<<dim3(gx, gy), 256, 0, q4kv_stream>>>(q, pool, score, n_tok, n_blocks,
                                                                stride, n_head, pos0, ratio);
    }
    return q4kv_launch_ok("qsa_score");
}
extern "C" bool q4_hip_qsa_score_d(const float *q, const float *pool, float *score,
                                   uint32_t stride, uint32_t n_head, uint32_t hd,
                                   uint32_t ratio) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !q4kv_pos_d || !q || !pool || !score || hd != IDX_HD || n_head == 0 ||
        n_head > 4)
        return false;
    if (((uintptr_t)q & 15u) || ((uintptr_t)pool & 15u)) {
        Q4KV_ERR("qsa_score_d: q and pool must be 16-byte aligned");
        return false;
    }
    if (stride == 0) return true;
    (void)hipGetLastError();
    /* Fixed grid sized by the row capacity (graph-capture safe); workgroups
     * past the device position's visible blocks exit at once. */
    const uint32_t gx = (stride + SC_ROWS_WG - 1) / SC_ROWS_WG;
    qsa_score_v_k<true><<<dim3(gx, 1), 256, 0, q4kv_stream>>>(q, pool, score, stride, stride,
                                                              n_head, 0, ratio, q4kv_pos_d);
    return q4kv_launch_ok("qsa_score_d");
}

/* Q4KV_TOPK_NT=1024 keeps token rows of up to 8192 blocks on 1024-thread
 * workgroups (8 keys per thread) instead of 512 (16 keys per thread). */
static bool topk_rows_512(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4KV_TOPK_NT");
        v = (e && atoi(e) == 1024) ? 0 : 1;
    }
    return v != 0;
}

extern "C" bool q4_hip_qsa_topk(const float *score, int32_t *sel, uint32_t n_tok,
                                uint32_t n_blocks, uint32_t stride, uint32_t k_blk,
                                uint32_t ratio, uint32_t pos0, uint32_t width) {
    Q4KV_FLUSH_OR_FAIL();
    (void)n_blocks; /* rows are bounded by each token's visible blocks */
    if (!q4kv_ok || !score || !sel || n_tok == 0 || k_blk == 0 || k_blk > TK_MAXK ||
        width == 0 || ratio == 0)
        return false;
    (void)hipGetLastError();
    /* the longest row decides the register layout */
    const uint64_t vis_max = ((uint64_t)pos0 + n_tok) / ratio;
    /* rows of up to 8192 blocks (prefill slices): 512 threads per row, so
     * the slice's rows launch half the waves */
    if (vis_max <= 8u * TK_T && topk_rows_512())
        qsa_topk_k<TK_ROWS, 16, 0, 512><<<n_tok, 512, 0, q4kv_stream>>>(
            score, sel, stride, k_blk, ratio, pos0, width, nullptr, nullptr);
    else if (vis_max <= 8u * TK_T)
        qsa_topk_k<TK_ROWS, 8><<<n_tok, TK_T, 0, q4kv_stream>>>(score, sel, stride, k_blk,
                                                                 ratio, pos0, width, nullptr,
                                                                 nullptr);
    else if (vis_max <= 16u * TK_T)
        qsa_topk_k<TK_ROWS, 16><<<n_tok, TK_T, 0, q4kv_stream>>>(score, sel, stride, k_blk,
                                                                  ratio, pos0, width, nullptr,
                                                                  nullptr);
    else
        qsa_topk_k<TK_ROWS, TK_KPT><<<n_tok, TK_T, 0, q4kv_stream>>>(
            score, sel, stride, k_blk, ratio, pos0, width, nullptr, nullptr);
    return q4kv_launch_ok("qsa_topk");
}
/* Q4KV_TOPK_SPLIT=0 keeps a device-position row on one workgroup. */
static bool topk_split_enabled(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4KV_TOPK_SPLIT");
        v = (e && e[0] == '0') ? 0 : 1;
    }
    return v != 0;
}

extern "C" bool q4_hip_qsa_topk_d(const float *score, int32_t *sel, uint32_t stride,
                                  uint32_t k_blk, uint32_t ratio, uint32_t width) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !q4kv_pos_d || !score || !sel || k_blk == 0 || k_blk > TK_MAXK ||
        width == 0 || ratio == 0)
        return false;
    (void)hipGetLastError();
    /* the device position is unknown here: the row capacity (stride blocks)
     * decides the register layout; 0 means unknown. Rows of 16385-65536
     * blocks are split over slices of TK_T * TKS_KPS blocks. */
    if (stride > 16u * TK_T && stride <= TK_T * TK_KPT && topk_split_enabled()) {
        const uint32_t g = (stride + TK_T * TKS_KPS - 1u) / (TK_T * TKS_KPS);
        qsa_topk_k<TK_DEV, TK_KPT, TKS_KPS><<<g, TK_T, 0, q4kv_stream>>>(
            score, sel, stride, k_blk, ratio, 0, width, q4kv_pos_d, nullptr);
    } else if (stride && stride <= 16u * TK_T)
        qsa_topk_k<TK_DEV, 16><<<1, TK_T, 0, q4kv_stream>>>(score, sel, stride, k_blk, ratio,
                                                             0, width, q4kv_pos_d, nullptr);
    else
        qsa_topk_k<TK_DEV, TK_KPT><<<1, TK_T, 0, q4kv_stream>>>(score, sel, stride, k_blk,
                                                                 ratio, 0, width, q4kv_pos_d,
                                                                 nullptr);
    return q4kv_launch_ok("qsa_topk_d");
}

extern "C" bool q4_hip_qsa_index_score_d(void *raw_f16, float *pool, const float *wn_k,
                                         const float *k_new, const float *q, const float *wn_q,
                                         float *score, uint32_t stride, uint32_t n_head,
                                         uint32_t hd, uint32_t ratio, uint32_t n_rot,
                                         float rope_base, float eps) {
    if (!q4kv_ok || !q4kv_pos_d || !raw_f16 || !pool || !k_new || !q || !score ||
        hd != IDX_HD || n_head == 0 || n_head > 4 || ratio == 0 || n_rot > hd) {
        Q4KV_FLUSH_OR_FAIL();
        return false;
    }
    if (((uintptr_t)raw_f16 & 3u) || ((uintptr_t)pool & 15u) || ((uintptr_t)q & 15u) ||
        ((uintptr_t)k_new & 7u) || ((uintptr_t)wn_k & 7u) || ((uintptr_t)wn_q & 7u)) {
        Q4KV_FLUSH_OR_FAIL();
        Q4KV_ERR("qsa_index_score_d: misaligned buffer");
        return false;
    }
    if (stride == 0) return q4kv_flush();
    /* the first call after a held q4_hip_kv_append_d in the fused decode
     * order: this launch carries the held append */
    q4kv_app_args app{};
    const uint32_t extra = q4kv_take_held(&app);
    (void)hipGetLastError();
    const uint32_t gx = (stride + SC_ROWS_WG - 1) / SC_ROWS_WG;
    qsa_index_score_dk<false><<<gx + extra, 256, 0, q4kv_stream>>>(
        (uint32_t *)raw_f16, pool, wn_k, k_new, q, wn_q, score, n_head, ratio, n_rot, rope_base,
        eps, q4kv_pos_d, nullptr, gx, app);
    return q4kv_launch_ok("qsa_index_score_d");
}

extern "C" bool q4_hip_qsa_index_batch(const q4kv_index_desc *d_descs, uint32_t n_items,
                                       uint32_t max_blocks, uint32_t n_head, uint32_t hd,
                                       uint32_t ratio, uint32_t n_rot, float rope_base, float eps,
                                       uint32_t k_blk, uint32_t width) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d_descs || n_items == 0 || n_items > 65535u || max_blocks == 0 ||
        hd != IDX_HD || n_head == 0 || n_head > 4 || ratio == 0 || n_rot > hd || k_blk == 0 ||
        k_blk > TK_MAXK || width == 0)
        return false;
    (void)hipGetLastError();
    const uint32_t gx = (max_blocks + SC_ROWS_WG - 1) / SC_ROWS_WG;
    qsa_index_score_dk<true><<<dim3(gx, n_items), 256, 0, q4kv_stream>>>(
        nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, n_head, ratio, n_rot,
        rope_base, eps, nullptr, d_descs, gx, q4kv_app_args{});
    if (max_blocks <= 16u * TK_T)
        qsa_topk_k<TK_BATCH, 16><<<n_items, TK_T, 0, q4kv_stream>>>(
            nullptr, nullptr, 0, k_blk, ratio, 0, width, nullptr, d_descs);
    else
        qsa_topk_k<TK_BATCH, TK_KPT><<<n_items, TK_T, 0, q4kv_stream>>>(
            nullptr, nullptr, 0, k_blk, ratio, 0, width, nullptr, d_descs);
    return q4kv_launch_ok("qsa_index_batch");
}
