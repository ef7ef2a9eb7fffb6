/*
 * q4kv_oracle.c -- CPU restatement of SuzuQu-Engine's QSA KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, never by the product library.
 *
 * Built with -O2 -fno-fast-math -ffp-contract=off so that every float
 * operation is a single IEEE-754 binary32 operation in round-to-nearest-even
 * (the source semantics of the reference kernels, see orc_quant_q8_0).
 */
#include "q4kv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* IEEE binary32 -> binary16, round-to-nearest-even, with subnormals,
 * overflow to infinity and quiet NaNs. This is what HIP's __float2half does
 * for the reference's scale store (src/q4_rocm.cu:7230, 7208-7211). The
 * reference has no host-side encoder (the src C files only decode), so this is
 * written from the IEEE-754 definition. */
uint16_t orc_f16_from_f32(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) /* NaN: keep the top payload bits, force quiet */
        return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) /* >= 65520 rounds to +-inf (ties-to-even) */
        return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) { /* below 2^-14: binary16 subnormal or zero */
        if (a <= 0x33000000u) return sign; /* <= 2^-25 rounds to 0 */
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t s = 126u - e; /* value / 2^-24 == m >> s */
        uint32_t r = m >> s;
        uint32_t rem = m & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t e = (a >> 23) - 112u;
    uint32_t mant = a & 0x7fffffu;
    uint32_t r = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

/* binary16 -> binary32, restating src/q4_quant.c:21-46 (q4_f16_to_f32). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t s = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        if (m == 0) {
            u = s;
        } else { /* subnormal: normalise */
            int sh = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                sh++;
            }
            m &= 0x3ffu;
            u = s | ((uint32_t)(113 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        u = s | 0x7f800000u | (m << 13);
    } else {
        u = s | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* q8_0 quantiser, restating f32_to_q8_k (src/q4_rocm.cu:7221-7238) and the
 * q8 branch of kv_append_k (src/q4_rocm.cu:7972-7990) under IEEE source
 * semantics: amax = max |x| (fmaxf/fabsf), d = amax / 127 (division), id =
 * d > 0 ? 1/d : 0 (division), the block's scale is fp16_rne(d), and
 * q = clamp(rint(x * id), -127, 127). Inputs must be finite. */
int orc_quant_q8_0(const float *x, uint64_t n, uint8_t *out) {
    if (!x || !out || n % 32u) return -1;
    for (uint64_t b = 0; b < n / 32u; b++) {
        const float *xb = x + b * 32u;
        uint8_t *o = out + b * 34u;
        float amax = 0.f;
        for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(xb[i]));
        float d = amax / 127.f;
        float id = d > 0.f ? 1.f / d : 0.f;
        uint16_t h = orc_f16_from_f32(d);
        memcpy(o, &h, 2);
        for (int i = 0; i < 32; i++) {
            int q = (int)rintf(xb[i] * id);
            if (q > 127) q = 127;
            if (q < -127) q = -127;
            o[2 + i] = (uint8_t)(int8_t)q;
        }
    }
    return 0;
}

/* fp16 KV width: per-element RNE, src/q4_rocm.cu:7208-7211. */
void orc_quant_f16(const float *x, uint64_t n, uint16_t *out) {
    for (uint64_t i = 0; i < n; i++) out[i] = orc_f16_from_f32(x[i]);
}

/* q8_0 dequantisation, restating dequant_q8_0 (src/q4_quant.c:123-133):
 * x = (float)q * f16(scale). */
void orc_dequant_q8_0(const uint8_t *src, uint64_t n, float *dst) {
    for (uint64_t b = 0; b < n / 32u; b++) {
        uint16_t dh;
        memcpy(&dh, src + b * 34u, 2);
        float d = orc_f16_to_f32(dh);
        const int8_t *qs = (const int8_t *)(src + b * 34u + 2u);
        for (int j = 0; j < 32; j++) dst[b * 32u + j] = (float)qs[j] * d;
    }
}

/* src/q4_fwd.c:644-650 (kv_token_bytes). */
uint32_t orc_kv_token_bytes(int kind, uint32_t n_kvh, uint32_t hd) {
    uint32_t kvw = n_kvh * hd;
    if (kind == ORC_KV_Q8) return (kvw / 32u) * 34u;
    return kvw * (kind == ORC_KV_F16 ? 2u : 4u);
}

/* src/q4_fwd.c:663-665 (kv_tag). */
uint32_t orc_kv_tag(int kind) {
    return kind == ORC_KV_Q8 ? 8u : kind == ORC_KV_F16 ? 2u : 4u;
}

/* src/q4_rocm.cu:7962-8000 (kv_append_k): write K and V at pos * bpt. */
int orc_kv_append(uint8_t *kc, uint8_t *vc, const float *k, const float *v,
                  uint32_t n, uint32_t bpt, int kind, uint32_t pos) {
    uint8_t *dk = kc + (size_t)pos * bpt, *dv = vc + (size_t)pos * bpt;
    if (kind == ORC_KV_Q8) {
        if (n % 32u) return -1;
        orc_quant_q8_0(k, n, dk);
        orc_quant_q8_0(v, n, dv);
    } else if (kind == ORC_KV_F16) {
        orc_quant_f16(k, n, (uint16_t *)dk);
        orc_quant_f16(v, n, (uint16_t *)dv);
    } else {
        memcpy(dk, k, (size_t)n * 4u);
        memcpy(dv, v, (size_t)n * 4u);
    }
    return 0;
}

/* Element d of the (position p, kv head kh) row of a cache laid out
 * [pos][kvh][hd] with the given width (src/q4_fwd.c:652-655 for the token
 * stride, src/q4_rocm.cu:6816-6824 / 6834-6842 for the in-row layout). */
static void load_row(const void *cache, int kind, uint32_t n_kvh, uint32_t hd,
                     int32_t p, uint32_t kh, float *row) {
    size_t r = (size_t)p * n_kvh + kh;
    if (kind == ORC_KV_Q8) {
        orc_dequant_q8_0((const uint8_t *)cache + r * (hd / 32u) * 34u, hd, row);
    } else if (kind == ORC_KV_F16) {
        const uint16_t *e = (const uint16_t *)cache + r * hd;
        for (uint32_t d = 0; d < hd; d++) row[d] = orc_f16_to_f32(e[d]);
    } else {
        memcpy(row, (const float *)cache + r * hd, hd * 4u);
    }
}

/* One (token, head) of gated attention in double precision. The softmax is
 * the textbook one: max-subtracted exp, normalised by the sum; positions
 * < 0 (padding, src/q4_rocm.cu:6816, 6861) and >= max_kv are skipped; an
 * empty list yields 0 (the `sum > 0 ? 1/sum : 0` guard of
 * src/q4_rocm.cu:7001 and src/q4_fwd.c:391). */
static void attn_one_dbl(const float *qh, const void *kc, const void *vc,
                         int kind, const float *gh, float *oh, uint32_t n_kvh,
                         uint32_t hd, uint32_t kh, const int32_t *list,
                         uint32_t n_list, int32_t dense_n, uint32_t max_kv,
                         float scale, double *sc, float *row, double *acc) {
    uint32_t n = list ? n_list : (uint32_t)dense_n;
    double m = -INFINITY;
    for (uint32_t j = 0; j < n; j++) {
        int32_t p = list ? list[j] : (int32_t)j;
        if (p < 0 || (uint32_t)p >= max_kv) {
            sc[j] = -INFINITY;
            continue;
        }
        load_row(kc, kind, n_kvh, hd, p, kh, row);
        double dot = 0.0;
        for (uint32_t d = 0; d < hd; d++) dot += (double)qh[d] * (double)row[d];
        sc[j] = dot * (double)scale;
        if (sc[j] > m) m = sc[j];
    }
    for (uint32_t d = 0; d < hd; d++) acc[d] = 0.0;
    double sum = 0.0;
    if (m > -INFINITY) {
        for (uint32_t j = 0; j < n; j++) {
            if (sc[j] == -INFINITY) continue;
            int32_t p = list ? list[j] : (int32_t)j;
            double w = exp(sc[j] - m);
            sum += w;
            load_row(vc, kind, n_kvh, hd, p, kh, row);
            for (uint32_t d = 0; d < hd; d++) acc[d] += w * (double)row[d];
        }
    }
    double inv = sum > 0.0 ? 1.0 / sum : 0.0;
    for (uint32_t d = 0; d < hd; d++) {
        double g = gh ? 1.0 / (1.0 + exp(-(double)gh[d])) : 1.0;
        oh[d] = (float)(acc[d] * inv * g);
    }
}

/* The same in fp32, in the loop shape of the reference's CPU attention
 * qsa_one (src/q4_fwd.c:358-398): fp32 dot, expf, 1/sum, sigmoid gate. */
static void attn_one_f32(const float *qh, const void *kc, const void *vc,
                         int kind, const float *gh, float *oh, uint32_t n_kvh,
                         uint32_t hd, uint32_t kh, const int32_t *list,
                         uint32_t n_list, int32_t dense_n, uint32_t max_kv,
                         float scale, float *sc, float *row) {
    uint32_t n = list ? n_list : (uint32_t)dense_n;
    float m = -INFINITY;
    for (uint32_t j = 0; j < n; j++) {
        int32_t p = list ? list[j] : (int32_t)j;
        if (p < 0 || (uint32_t)p >= max_kv) {
            sc[j] = -INFINITY;
            continue;
        }
        load_row(kc, kind, n_kvh, hd, p, kh, row);
        float dot = 0.f;
        for (uint32_t d = 0; d < hd; d++) dot += qh[d] * row[d];
        sc[j] = dot * scale;
        if (sc[j] > m) m = sc[j];
    }
    float sum = 0.f;
    for (uint32_t j = 0; j < n; j++) {
        sc[j] = sc[j] == -INFINITY ? 0.f : expf(sc[j] - m);
        sum += sc[j];
    }
    float inv = sum > 0.f ? 1.f / sum : 0.f;
    memset(oh, 0, hd * sizeof(float));
    for (uint32_t j = 0; j < n; j++) {
        if (sc[j] == 0.f) continue;
        int32_t p = list ? list[j] : (int32_t)j;
        float w = sc[j] * inv;
        load_row(vc, kind, n_kvh, hd, p, kh, row);
        for (uint32_t d = 0; d < hd; d++) oh[d] += w * row[d];
    }
    if (gh)
        for (uint32_t d = 0; d < hd; d++) oh[d] *= 1.0f / (1.0f + expf(-gh[d]));
}

int orc_attn(const float *q, const void *kcache, const void *vcache, int kind,
             const float *gate, float *out, uint32_t n_head, uint32_t n_kvh,
             uint32_t hd, uint32_t n_tok, const int32_t *idx, uint32_t width,
             uint64_t tok_stride, uint64_t kvh_stride, uint32_t kv_base,
             uint32_t max_kv, float scale, int dbl, int nthreads) {
    if (!q || !kcache || !vcache || !out || !n_head || !n_kvh || !hd ||
        n_head % n_kvh)
        return -1;
    if (kind == ORC_KV_Q8 && hd % 32u) return -1;
    const uint32_t gqa = n_head / n_kvh;
    const uint32_t nmax = idx ? width : (kv_base + n_tok < max_kv ? kv_base + n_tok : max_kv);
    const int64_t total = (int64_t)n_tok * n_head;
    int err = 0;
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel num_threads(nthreads)
#endif
    {
        double *scd = malloc((size_t)(nmax ? nmax : 1) * sizeof(double));
        float *scf = malloc((size_t)(nmax ? nmax : 1) * sizeof(float));
        float *row = malloc((size_t)hd * sizeof(float));
        double *acc = malloc((size_t)hd * sizeof(double));
        if (!scd || !scf || !row || !acc) {
            err = -1;
        } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
            for (int64_t th = 0; th < total; th++) {
                uint32_t t = (uint32_t)(th / n_head), h = (uint32_t)(th % n_head);
                uint32_t kh = h / gqa;
                const float *qh = q + ((size_t)t * n_head + h) * hd;
                const float *gh = gate ? gate + ((size_t)t * n_head + h) * hd : NULL;
                float *oh = out + ((size_t)t * n_head + h) * hd;
                const int32_t *list = idx ? idx + t * tok_stride + kh * kvh_stride : NULL;
                uint32_t nkv = kv_base + t + 1u;
                if (nkv > max_kv) nkv = max_kv;
                if (dbl)
                    attn_one_dbl(qh, kcache, vcache, kind, gh, oh, n_kvh, hd, kh,
                                 list, width, (int32_t)nkv, max_kv, scale, scd, row, acc);
                else
                    attn_one_f32(qh, kcache, vcache, kind, gh, oh, n_kvh, hd, kh,
                                 list, width, (int32_t)nkv, max_kv, scale, scf, row);
            }
        }
        free(scd);
        free(scf);
        free(row);
        free(acc);
    }
    return err;
}

/* q8_0 GEMV: y[r] = scale * sum_b d_b * sum_i q_bi * x[32b + i] over the
 * ncols/32 blocks of row r (34 bytes each: fp16 d, 32 int8), accumulated in
 * double. src/q4_rocm.cu:1262-1285 (wgv_q8_0_k), q8_0 layout
 * src/q4_quant.c:123-133. */
int orc_gemv_q8_0(const uint8_t *w, uint64_t nrows, uint64_t ncols, const float *x, float *y,
                  float scale) {
    if (!w || !x || !y || ncols % 32) return -1;
    const uint64_t nb = ncols / 32;
    for (uint64_t r = 0; r < nrows; r++) {
        const uint8_t *row = w + r * nb * 34;
        double acc = 0;
        for (uint64_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + b * 34;
            const double d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            double s = 0;
            for (int i = 0; i < 32; i++) s += (double)(int8_t)blk[2 + i] * x[b * 32 + i];
            acc += d * s;
        }
        y[r] = (float)(acc * scale);
    }
    return 0;
}
