/*
 * qsa_index_oracle.c -- CPU restatement of SuzuQu-Engine's QSA indexer
 * (block pooling, block scoring, exact top-k block selection and expansion)
 * and of the Q/K preparation (RMSNorm + partial RoPE) that feeds it.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (and bench.py's cpu_baseline
 * leg), never by the product library.
 *
 * Numeric contract (the reference's source semantics):
 *  - RoPE frequency freq_p = powf(base, -(p / np)) with the exponent an fp32
 *    quotient, taken correctly rounded (pow in double, rounded once to fp32);
 *    the angle is the fp32 product (float)pos * freq_p, exactly as the
 *    reference kernels form it. cos/sin of that fp32 angle are taken in
 *    double. At pos ~ 2^18 one fp32 ulp of freq moves the angle by ~0.016 rad,
 *    so freq and angle are reproduced bit-exactly rather than approximated.
 *  - Norms and dot products accumulate in double (the golden value the GPU's
 *    fp32 result is compared against within tolerance).
 *  - Selection is integer work on the fp32 score bit patterns and is exact.
 */
#include "q4kv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Order-preserving uint32 key of an fp32 score: larger float -> larger key,
 * +0 above -0, NaNs outside +-inf by sign. src/q4_rocm.cu:7471-7474. */
uint32_t orc_qsa_key(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* fp32 RoPE frequency of pair p out of np pairs, src/q4_rocm.cu:6255, 7391. */
float orc_rope_freq(float base, uint32_t p, uint32_t np) {
    float e = -(float)p / (float)np;
    return (float)pow((double)base, (double)e);
}

/* Rotate pairs (2p, 2p+1), p < n_rot/2, of x by angle pos * freq_p. */
static void rope_pairs(double *x, uint32_t n_rot, float pos_f, float base) {
    uint32_t np = n_rot / 2;
    for (uint32_t p = 0; p < np; p++) {
        float freq = orc_rope_freq(base, p, np);
        float ang = pos_f * freq; /* one fp32 rounding, as the reference */
        double c = cos((double)ang), s = sin((double)ang);
        double x0 = x[2 * p], x1 = x[2 * p + 1];
        x[2 * p] = x0 * c - x1 * s;
        x[2 * p + 1] = x0 * s + x1 * c;
    }
}

/* One head of qsa_q_prep_k / qsa_k_prep_k (src/q4_rocm.cu:6229-6289):
 * dst = RMSNorm(src) * wn, then RoPE of the first n_rot dims at pos. */
int orc_qsa_prep(const float *src, float *dst, const float *wn, uint32_t hd,
                 uint32_t n_rot, int32_t pos, float base, float eps) {
    if (!src || !dst || hd == 0 || hd > 1024 || n_rot > hd) return -1;
    double x[1024], ss = 0;
    for (uint32_t i = 0; i < hd; i++) ss += (double)src[i] * src[i];
    double inv = 1.0 / sqrt(ss / hd + (double)eps);
    for (uint32_t i = 0; i < hd; i++) x[i] = src[i] * inv * (wn ? wn[i] : 1.0);
    rope_pairs(x, n_rot, (float)pos, base);
    for (uint32_t i = 0; i < hd; i++) dst[i] = (float)x[i];
    return 0;
}

/* qsa_pool_k (src/q4_rocm.cu:7366-7401) over blocks [b0, b1): the mean of
 * `ratio` consecutive fp16 raw keys, RMSNorm * wn, RoPE at the block's first
 * position b*ratio. raw is [pos][hd] fp16, pool is [block][hd] fp32. */
int orc_qsa_pool(const uint16_t *raw, float *pool, const float *wn, uint32_t hd,
                 uint32_t ratio, uint32_t b0, uint32_t b1, uint32_t n_rot,
                 float base, float eps) {
    if (!raw || !pool || hd != 128 || ratio == 0 || b1 <= b0 || n_rot > hd) return -1;
    for (uint32_t b = b0; b < b1; b++) {
        double v[128], ss = 0;
        for (uint32_t d = 0; d < hd; d++) {
            double s = 0;
            for (uint32_t j = 0; j < ratio; j++)
                s += orc_f16_to_f32(raw[((uint64_t)b * ratio + j) * hd + d]);
            v[d] = s / ratio;
            ss += v[d] * v[d];
        }
        double inv = 1.0 / sqrt(ss / hd + (double)eps);
        for (uint32_t d = 0; d < hd; d++) v[d] = v[d] * inv * (wn ? wn[d] : 1.0);
        rope_pairs(v, n_rot, (float)(b * ratio), base);
        for (uint32_t d = 0; d < hd; d++) pool[(uint64_t)b * hd + d] = (float)v[d];
    }
    return 0;
}

/* qsa_score_k (src/q4_rocm.cu:7412-7445): for token t at pos0+t, blocks
 * b < n_vis = (pos+1)/ratio score sum_h max(q[t,h] . pool[b], 0); blocks
 * n_vis <= b < n_blocks get -1e30. q is [n_tok][n_head][hd]. */
int orc_qsa_score(const float *q, const float *pool, float *score, uint32_t n_tok,
                  uint32_t n_blocks, uint32_t stride, uint32_t n_head, uint32_t hd,
                  uint32_t pos0, uint32_t ratio) {
    if (!q || !pool || !score || hd != 128 || n_head == 0 || n_head > 4) return -1;
    for (uint32_t t = 0; t < n_tok; t++) {
        uint32_t pos = pos0 + t;
        uint32_t n_vis = ratio ? (pos + 1) / ratio : 0;
        for (uint32_t b = 0; b < n_blocks; b++) {
            double s = -1.0e30;
            if (b < n_vis) {
                s = 0;
                const float *kb = pool + (uint64_t)b * hd;
                for (uint32_t h = 0; h < n_head; h++) {
                    const float *qq = q + ((uint64_t)t * n_head + h) * hd;
                    double dot = 0;
                    for (uint32_t i = 0; i < hd; i++) dot += (double)qq[i] * kb[i];
                    s += dot > 0 ? dot : 0;
                }
            }
            score[(uint64_t)t * stride + b] = (float)s;
        }
    }
    return 0;
}

/* Exact top-`need` of keys[0..n) under (key desc, index asc), the reference's
 * radix threshold search (src/q4_rocm.cu:7760-7790): four passes over the
 * 8-bit digits of the key, most significant first, each pass keeping the
 * digit whose cumulative count from the top reaches the remaining target.
 * Returns the threshold key; *n_gt receives the count strictly above it. */
static uint32_t radix_threshold(const uint32_t *keys, uint32_t n, uint32_t need,
                                uint32_t *n_gt) {
    uint32_t prefix = 0, above = 0;
    for (int p = 0; p < 4; p++) {
        uint32_t hist[256] = {0};
        uint32_t sh = 24 - 8 * p;
        for (uint32_t b = 0; b < n; b++)
            if (p == 0 || (keys[b] >> (sh + 8)) == prefix) hist[(keys[b] >> sh) & 255]++;
        uint32_t target = need - above, acc = 0, dg = 0;
        for (int i = 255; i >= 0; i--) {
            if (acc + hist[i] >= target) { dg = (uint32_t)i; break; }
            acc += hist[i];
        }
        above += acc;
        prefix = (prefix << 8) | dg;
    }
    *n_gt = above;
    return prefix;
}

/* qsa_topk_k + qsa_write_sel (src/q4_rocm.cu:7722-7846), one row per token.
 * n_vis <= k_blk: the dense causal prefix sel[w] = w <= pos ? w : -1.
 * Otherwise the chosen blocks are those with key above the threshold in
 * ascending block order, then threshold ties in ascending order until `need`
 * = k_blk; entry w < need*ratio expands chosen[w/ratio]*ratio + w%ratio, then
 * the causal tail n_vis*ratio .. pos, then -1. */
int orc_qsa_topk(const float *score, int32_t *sel, uint32_t n_tok, uint32_t stride,
                 uint32_t k_blk, uint32_t ratio, uint32_t pos0, uint32_t width) {
    if (!score || !sel || k_blk == 0 || k_blk > 512 || width == 0 || ratio == 0) return -1;
    for (uint32_t t = 0; t < n_tok; t++) {
        uint32_t pos = pos0 + t;
        uint32_t n_vis = (pos + 1) / ratio;
        uint32_t need = n_vis < k_blk ? n_vis : k_blk;
        int32_t *row = sel + (uint64_t)t * width;
        if (need == n_vis) {
            for (uint32_t w = 0; w < width; w++) row[w] = w <= pos ? (int32_t)w : -1;
            continue;
        }
        uint32_t *keys = malloc((size_t)n_vis * 4);
        if (!keys) return -1;
        for (uint32_t b = 0; b < n_vis; b++)
            keys[b] = orc_qsa_key(score[(uint64_t)t * stride + b]);
        uint32_t n_gt, thr = radix_threshold(keys, n_vis, need, &n_gt);
        int32_t chosen[512];
        uint32_t nc = 0;
        for (uint32_t b = 0; b < n_vis; b++)
            if (keys[b] > thr) chosen[nc++] = (int32_t)b;
        for (uint32_t b = 0; b < n_vis && nc < need; b++)
            if (keys[b] == thr) chosen[nc++] = (int32_t)b;
        free(keys);
        uint32_t ncs = nc * ratio;
        for (uint32_t w = 0; w < width; w++) {
            if (w < ncs) {
                row[w] = (int32_t)((uint32_t)chosen[w / ratio] * ratio + w % ratio);
            } else {
                uint32_t tail = n_vis * ratio + (w - ncs);
                row[w] = tail <= pos ? (int32_t)tail : -1;
            }
        }
        (void)n_gt;
    }
    return 0;
}
