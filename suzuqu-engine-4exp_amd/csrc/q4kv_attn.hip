/*
 * q4kv_attn.hip -- QSA attention over a q8_0 / f16 / f32 KV cache on gfx950.
 *
 * Semantics (the reference's gqa_dec_split_k + gqa_dec_comb_k and
 * gqa_prefill_k, src/q4_rocm.cu:6762-7205): for every (token, query head),
 *   out = sum_p softmax_p(scale * q.k_p) v_p * sigmoid(gate)
 * over a position list (explicit, -1 = padding, or the dense causal prefix),
 * with the query heads of one KV head sharing that head's cache rows (GQA).
 * Empty lists give 0.
 *
 * Design (MI355X-native, not a translation of the wave32 reference):
 *  - One workgroup (4 x wave64) owns one (item, split): an item is one
 *    (token or sequence, KV head) pair, a split a contiguous run of 64-position
 *    chunks of its list. Every chunk's K and V rows are fetched with 16-byte
 *    loads (17 per 272-byte q8_0 row), all issued before any is consumed, and
 *    staged raw in LDS.
 *  - Q.K^T and P.V run on MFMA (v_mfma_f32_16x16x32_f16). The 16 MFMA rows
 *    hold the 8 GQA query heads twice: rows 0-7 the fp16 "hi" part of q (or
 *    of the softmax weight), rows 8-15 the fp16 residual "lo" = x - hi. The
 *    int8 cache values are exact in fp16, so hi+lo makes the contraction
 *    accurate to ~2^-22 relative with fp32 accumulation, at no extra MFMA
 *    cost. q8_0 scales are applied per 32-element block in fp32 (QK) or
 *    folded into the weights before the fp16 split (PV).
 *  - int8 -> fp16 is exact and branch-free: v_perm_b32 places each byte
 *    (xor 0x80) under the exponent 0x64 (1024 + u), one packed subtract of
 *    1152 leaves the signed value.
 *  - Online softmax in base 2 per chunk; the split partials (m, l, acc[hd])
 *    are merged by a second kernel that also applies the gate. A single
 *    split (prefill, or short lists) finalises in place.
 */
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <math.h>

#include "q4kv_internal.h"

extern "C" {
#include "q4kv.h"
}

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

enum { MODE_DENSE = 0, MODE_INDEXED = 1, MODE_BATCH = 2 };

struct AttnArgs {
    const uint8_t *kc, *vc;
    const float *q, *gate;
    float *out;
    const int32_t *idx;
    uint64_t tok_stride, kvh_stride;
    const q4kv_seq_desc *seqs;
    float *part;
    uint32_t width, kv_base, max_kv;
    uint32_t n_head, n_kvh, hd;
    uint32_t S, cps, item0;
    float scale_log2;
};

struct Item {
    const uint8_t *kc, *vc;
    const float *q, *gate;
    float *out;
    const int32_t *list;
    uint32_t n, max_kv;
};

template <int MODE>
__device__ static inline Item resolve_item(const AttnArgs &a, uint32_t item) {
    const uint32_t kh = item % a.n_kvh, t = item / a.n_kvh;
    const uint32_t gqa = a.n_head / a.n_kvh;
    const size_t hoff = (size_t)kh * gqa * a.hd;
    Item it;
    if (MODE == MODE_BATCH) {
        const q4kv_seq_desc *d = a.seqs + t;
        it.kc = (const uint8_t *)d->kcache;
        it.vc = (const uint8_t *)d->vcache;
        it.q = d->q + hoff;
        it.gate = d->gate ? d->gate + hoff : nullptr;
        it.out = d->out + hoff;
        it.max_kv = d->max_kv;
        it.list = d->idx ? d->idx + (size_t)kh * d->idx_kvh_stride : nullptr;
        it.n = d->idx ? d->n_sel : (d->n_sel < d->max_kv ? d->n_sel : d->max_kv);
    } else {
        const size_t qo = (size_t)t * a.n_head * a.hd + hoff;
        it.kc = a.kc;
        it.vc = a.vc;
        it.q = a.q + qo;
        it.gate = a.gate ? a.gate + qo : nullptr;
        it.out = a.out + qo;
        it.max_kv = a.max_kv;
        if (MODE == MODE_INDEXED) {
            it.list = a.idx + t * a.tok_stride + kh * a.kvh_stride;
            it.n = a.width;
        } else {
            const uint32_t nkv = a.kv_base + t + 1u;
            it.list = nullptr;
            it.n = nkv < a.max_kv ? nkv : a.max_kv;
        }
    }
    return it;
}

/* Value of the lane 32 apart (v_permlane32_swap; lanes < 32 receive the upper
 * half's operand in the second result, lanes >= 32 the lower half's in the
 * first). */
__device__ static inline float xor32(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                              false);
    return __uint_as_float((threadIdx.x & 32u) ? r[0] : r[1]);
}

__device__ static inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ static inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

/* Four signed bytes -> four exact fp16 (1024 + (b ^ 0x80) - 1152). */
__device__ static inline void i8x4_to_h4(uint32_t w, uint32_t &lo, uint32_t &hi) {
    w ^= 0x80808080u;
    lo = __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u);
}
__device__ static inline h8_t h8_minus_1152(u4_t r) {
    h8_t h = __builtin_bit_cast(h8_t, r);
    return h - (h8_t)((_Float16)1152.0f);
}

/* Dimension (within a 32-block) held by element i of k-group j of the MFMA
 * operand for q8_0 block b. Odd blocks are 4-byte aligned inside the 68-byte
 * block pair and map naturally; even blocks start 2 bytes into a dword, so
 * group 3 takes the two leading and two trailing bytes as one dword. */
__device__ static inline uint32_t q8_kdim(uint32_t b, uint32_t j, uint32_t i) {
    if (b & 1u) return 8u * j + i;
    if (j < 3u) return 2u + 8u * j + i;
    return i < 4u ? 26u + i : (i < 6u ? i - 4u : 24u + i);
}

/* K operand (8 int8 of block b for k-group j) from a raw q8_0 row in LDS. */
__device__ static inline h8_t load_k_q8(const uint8_t *row, uint32_t b, uint32_t j) {
    const uint32_t *pw = (const uint32_t *)(row + 68u * (b >> 1));
    uint32_t w0, w1;
    if (b & 1u) {
        w0 = pw[9u + 2u * j];
        w1 = pw[10u + 2u * j];
    } else {
        const uint32_t i0 = j < 3u ? 1u + 2u * j : 7u;
        w0 = pw[i0];
        w1 = pw[i0 + 1u];
        const uint32_t lead = pw[0];
        if (j == 3u) w1 = __builtin_amdgcn_perm(w1, lead, 0x05040302u);
    }
    uint32_t r0, r1, r2, r3;
    i8x4_to_h4(w0, r0, r1);
    i8x4_to_h4(w1, r2, r3);
    return h8_minus_1152((u4_t){r0, r1, r2, r3});
}

__device__ static inline float ld_f16(const uint8_t *p) {
    return __half2float(__ushort_as_half(*(const uint16_t *)p));
}

/* x -> fp16 hi part (rows < 8) or fp16 residual (rows >= 8). */
__device__ static inline _Float16 split_hl(float x, bool lo) {
    _Float16 h = (_Float16)x;
    return lo ? (_Float16)(x - (float)h) : h;
}

template <int KIND> struct KCfg;
template <> struct KCfg<Q4KV_Q8> { static constexpr uint32_t CP = 64, RMAX = 272; };
template <> struct KCfg<Q4KV_F16> { static constexpr uint32_t CP = 64, RMAX = 512; };
template <> struct KCfg<Q4KV_F32> { static constexpr uint32_t CP = 32, RMAX = 1024; };

template <int KIND, int MODE, int HG>
__global__ __launch_bounds__(256) void qsa_attn_k(AttnArgs a) {
    constexpr uint32_t CP = KCfg<KIND>::CP;
    constexpr uint32_t RMAX = KCfg<KIND>::RMAX;
    constexpr uint32_t NH = HG * 8u; /* query-head slots */
    constexpr uint32_t NLD = (CP * RMAX / 16u + 255u) / 256u;
    __shared__ __attribute__((aligned(16))) uint8_t kraw[CP * RMAX];
    __shared__ __attribute__((aligned(16))) uint8_t vraw[CP * RMAX];
    __shared__ __attribute__((aligned(16))) float sc[NH * CP];
    __shared__ __attribute__((aligned(16))) float vsc[KIND == Q4KV_Q8 ? 8u * CP : 4u];
    __shared__ int32_t s_pos[CP];
    __shared__ float s_m[NH], s_l[NH], s_al[NH];

    const uint32_t s = blockIdx.x, item = a.item0 + blockIdx.y;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t hd = a.hd, NB = hd / 32u, gqa = a.n_head / a.n_kvh;
    const uint32_t kh = item % a.n_kvh;
    const Item it = resolve_item<MODE>(a, item);
    const uint32_t rowb =
        KIND == Q4KV_Q8 ? NB * 34u : hd * (KIND == Q4KV_F16 ? 2u : 4u);
    const uint32_t RS = (rowb + 15u) & ~15u;
    const bool al16 =
        (rowb & 15u) == 0 && ((((uintptr_t)it.kc) | ((uintptr_t)it.vc)) & 15u) == 0;
    const uint32_t n_chunks = (it.n + CP - 1u) / CP;
    const uint32_t c0 = s * a.cps;
    const uint32_t c1 = (s + 1u == a.S) ? n_chunks : min(c0 + a.cps, n_chunks);

    const uint32_t mrow = lane & 15u; /* MFMA A row / B,C column */
    const uint32_t jg = lane >> 4;    /* MFMA k-group */
    const bool lo_row = mrow >= 8u;

    /* Q operands, hi/lo split across the row halves. */
    h8_t qa[HG][8];
#pragma unroll
    for (uint32_t hg = 0; hg < HG; hg++) {
        const uint32_t g = hg * 8u + (mrow & 7u);
#pragma unroll
        for (uint32_t b = 0; b < 8u; b++) {
#pragma unroll
            for (uint32_t i = 0; i < 8u; i++) {
                float x = 0.f;
                if (b < NB && g < gqa) {
                    const uint32_t d = KIND == Q4KV_Q8 ? q8_kdim(b, jg, i) : 8u * jg + i;
                    x = it.q[(size_t)g * hd + 32u * b + d];
                }
                qa[hg][b][i] = split_hl(x, lo_row);
            }
        }
    }
    if (tid < NH) {
        s_m[tid] = -INFINITY;
        s_l[tid] = 0.f;
        s_al[tid] = 1.f;
    }
    f4_t acc[HG][4];
#pragma unroll
    for (uint32_t hg = 0; hg < HG; hg++)
#pragma unroll
        for (uint32_t t = 0; t < 4u; t++) acc[hg][t] = (f4_t){0.f, 0.f, 0.f, 0.f};
    __syncthreads();

    for (uint32_t c = c0; c < c1; c++) {
        const uint32_t base = c * CP;
        if (tid < CP) {
            const uint32_t j = base + tid;
            int32_t p = -1;
            if (j < it.n) {
                p = it.list ? it.list[j] : (int32_t)j;
                if (p < 0 || (uint32_t)p >= it.max_kv) p = -1;
            }
            s_pos[tid] = p;
        }
        __syncthreads();
        /* ---- stage raw K/V rows; invalid positions read row 0 (masked) ---- */
        if (al16) {
            const uint32_t nch = rowb / 16u, total = CP * nch;
            uint4 kr[NLD], vr[NLD];
#pragma unroll
            for (uint32_t u = 0; u < NLD; u++) {
                const uint32_t e = tid + u * 256u;
                if (e < total) {
                    const uint32_t r = e / nch, q = e - r * nch;
                    int32_t p = s_pos[r];
                    p = p < 0 ? 0 : p;
                    const size_t off = ((size_t)p * a.n_kvh + kh) * rowb + q * 16u;
                    kr[u] = *(const uint4 *)(it.kc + off);
                    vr[u] = *(const uint4 *)(it.vc + off);
                }
            }
#pragma unroll
            for (uint32_t u = 0; u < NLD; u++) {
                const uint32_t e = tid + u * 256u;
                if (e < total) {
                    const uint32_t r = e / nch, q = e - r * nch;
                    *(uint4 *)(kraw + r * RS + q * 16u) = kr[u];
                    *(uint4 *)(vraw + r * RS + q * 16u) = vr[u];
                }
            }
        } else {
            const uint32_t nh = rowb / 2u, total = CP * nh;
            for (uint32_t e = tid; e < total; e += 256u) {
                const uint32_t r = e / nh, q = e - r * nh;
                int32_t p = s_pos[r];
                p = p < 0 ? 0 : p;
                const size_t off = ((size_t)p * a.n_kvh + kh) * rowb + q * 2u;
                *(uint16_t *)(kraw + r * RS + q * 2u) = *(const uint16_t *)(it.kc + off);
                *(uint16_t *)(vraw + r * RS + q * 2u) = *(const uint16_t *)(it.vc + off);
            }
        }
        __syncthreads();
        if (KIND == Q4KV_Q8) {
            for (uint32_t e = tid; e < NB * CP; e += 256u) {
                const uint32_t b = e / CP, r = e - b * CP;
                vsc[b * CP + r] = s_pos[r] < 0 ? 0.f : ld_f16(vraw + r * RS + 34u * b);
            }
        }
        /* ---- scores: wave w owns positions 16w .. 16w+15 ---- */
        if (wave * 16u < CP) {
            const uint32_t r = wave * 16u + mrow;
            const uint8_t *krow = kraw + r * RS;
            f4_t S[HG];
#pragma unroll
            for (uint32_t hg = 0; hg < HG; hg++) S[hg] = (f4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t b = 0; b < 8u; b++) {
                if (b >= NB) break;
                if (KIND == Q4KV_Q8) {
                    const h8_t kb = load_k_q8(krow, b, jg);
                    const float ks = ld_f16(krow + 34u * b);
#pragma unroll
                    for (uint32_t hg = 0; hg < HG; hg++) {
                        f4_t C = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            qa[hg][b], kb, (f4_t){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        S[hg] += ks * C;
                    }
                } else if (KIND == Q4KV_F16) {
                    const h8_t kb = *(const h8_t *)(krow + 64u * b + 16u * jg);
#pragma unroll
                    for (uint32_t hg = 0; hg < HG; hg++)
                        S[hg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[hg][b], kb, S[hg],
                                                                       0, 0, 0);
                } else {
                    const float *kf = (const float *)(krow + 128u * b + 32u * jg);
                    h8_t kh8, kl8;
#pragma unroll
                    for (uint32_t i = 0; i < 8u; i++) {
                        kh8[i] = split_hl(kf[i], false);
                        kl8[i] = split_hl(kf[i], true);
                    }
#pragma unroll
                    for (uint32_t hg = 0; hg < HG; hg++) {
                        S[hg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[hg][b], kh8, S[hg],
                                                                       0, 0, 0);
                        S[hg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[hg][b], kl8, S[hg],
                                                                       0, 0, 0);
                    }
                }
            }
            const bool valid = s_pos[r] >= 0;
#pragma unroll
            for (uint32_t hg = 0; hg < HG; hg++) {
#pragma unroll
                for (uint32_t i = 0; i < 4u; i++) {
                    const float tot = S[hg][i] + xor32(S[hg][i]);
                    const uint32_t head = hg * 8u + 4u * jg + i;
                    if (lane < 32u && head < gqa)
                        sc[head * CP + r] = valid ? tot * a.scale_log2 : -INFINITY;
                }
            }
        }
        __syncthreads();
        /* ---- online softmax statistics, one wave per head ---- */
        for (uint32_t g = wave; g < gqa; g += 4u) {
            const float v = lane < CP ? sc[g * CP + lane] : -INFINITY;
            const float cm = wave_max(v);
            const float mo = s_m[g];
            const float mn = fmaxf(mo, cm);
            const float al = mo == -INFINITY ? 0.f : exp2f(mo - mn);
            const float w = v == -INFINITY ? 0.f : exp2f(v - mn);
            if (lane < CP) sc[g * CP + lane] = w;
            const float ls = wave_sum(w);
            if (lane == 0) {
                s_m[g] = mn;
                s_l[g] = s_l[g] * al + ls;
                s_al[g] = al;
            }
        }
        __syncthreads();
        /* ---- P.V: wave w owns head dims 64w .. 64w+63 ---- */
#pragma unroll
        for (uint32_t hg = 0; hg < HG; hg++)
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                const float al = s_al[hg * 8u + ((4u * jg + i) & 7u)];
#pragma unroll
                for (uint32_t t = 0; t < 4u; t++) acc[hg][t][i] *= al;
            }
#pragma unroll
        for (uint32_t kc = 0; kc < CP / 32u; kc++) {
            const uint32_t p0 = 32u * kc + 8u * jg;
            if (KIND == Q4KV_Q8) {
#pragma unroll
                for (uint32_t u = 0; u < 2u; u++) {
                    const uint32_t bb = 2u * wave + u;
                    if (bb >= NB) break;
                    /* B: dims 32bb + 2n (tile 0) and 32bb + 2n + 1 (tile 1). */
                    const uint8_t *vb = vraw + p0 * RS + 34u * bb + 2u + 2u * mrow;
                    u4_t r0, r1;
#pragma unroll
                    for (uint32_t k = 0; k < 4u; k++) {
                        uint32_t x = (uint32_t)*(const uint16_t *)(vb + (2u * k) * RS) |
                                     ((uint32_t)*(const uint16_t *)(vb + (2u * k + 1u) * RS)
                                      << 16);
                        x ^= 0x80808080u;
                        r0[k] = __builtin_amdgcn_perm(0x64646464u, x, 0x04020400u);
                        r1[k] = __builtin_amdgcn_perm(0x64646464u, x, 0x04030401u);
                    }
                    const h8_t B0 = h8_minus_1152(r0), B1 = h8_minus_1152(r1);
                    const float *sp = vsc + bb * CP + p0;
#pragma unroll
                    for (uint32_t hg = 0; hg < HG; hg++) {
                        const uint32_t head = hg * 8u + (mrow & 7u);
                        const float *wp = sc + head * CP + p0;
                        h8_t A;
#pragma unroll
                        for (uint32_t i = 0; i < 8u; i++)
                            A[i] = split_hl(head < gqa ? wp[i] * sp[i] : 0.f, lo_row);
                        acc[hg][2u * u] =
                            __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B0, acc[hg][2u * u], 0, 0, 0);
                        acc[hg][2u * u + 1u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            A, B1, acc[hg][2u * u + 1u], 0, 0, 0);
                    }
                }
            } else {
                h8_t A[HG];
#pragma unroll
                for (uint32_t hg = 0; hg < HG; hg++) {
                    const uint32_t head = hg * 8u + (mrow & 7u);
                    const float *wp = sc + head * CP + p0;
#pragma unroll
                    for (uint32_t i = 0; i < 8u; i++)
                        A[hg][i] = split_hl(head < gqa ? wp[i] : 0.f, lo_row);
                }
#pragma unroll
                for (uint32_t t = 0; t < 4u; t++) {
                    const uint32_t dim = 64u * wave + 16u * t + mrow;
                    if (64u * wave + 16u * t >= hd) break;
                    if (KIND == Q4KV_F16) {
                        const uint8_t *vb = vraw + p0 * RS + 2u * dim;
                        u4_t r;
#pragma unroll
                        for (uint32_t k = 0; k < 4u; k++)
                            r[k] = (uint32_t)*(const uint16_t *)(vb + (2u * k) * RS) |
                                   ((uint32_t)*(const uint16_t *)(vb + (2u * k + 1u) * RS) << 16);
                        const h8_t B = __builtin_bit_cast(h8_t, r);
#pragma unroll
                        for (uint32_t hg = 0; hg < HG; hg++)
                            acc[hg][t] =
                                __builtin_amdgcn_mfma_f32_16x16x32_f16(A[hg], B, acc[hg][t], 0, 0, 0);
                    } else {
                        const uint8_t *vb = vraw + p0 * RS + 4u * dim;
                        h8_t Bh, Bl;
#pragma unroll
                        for (uint32_t i = 0; i < 8u; i++) {
                            const float x = *(const float *)(vb + i * RS);
                            Bh[i] = split_hl(x, false);
                            Bl[i] = split_hl(x, true);
                        }
#pragma unroll
                        for (uint32_t hg = 0; hg < HG; hg++) {
                            acc[hg][t] =
                                __builtin_amdgcn_mfma_f32_16x16x32_f16(A[hg], Bh, acc[hg][t], 0, 0, 0);
                            acc[hg][t] =
                                __builtin_amdgcn_mfma_f32_16x16x32_f16(A[hg], Bl, acc[hg][t], 0, 0, 0);
                        }
                    }
                }
            }
        }
        __syncthreads();
    }

    /* ---- epilogue: fold lo rows into hi rows, then finalise or spill ---- */
    const bool fin = a.S == 1u;
    const size_t pstride = (size_t)hd + 2u;
    float *pbase = fin ? nullptr : a.part + ((size_t)item * a.S + s) * gqa * pstride;
#pragma unroll
    for (uint32_t hg = 0; hg < HG; hg++) {
#pragma unroll
        for (uint32_t t = 0; t < 4u; t++) {
            uint32_t dim;
            bool dvalid;
            if (KIND == Q4KV_Q8) {
                const uint32_t bb = 2u * wave + (t >> 1);
                dim = 32u * bb + 2u * mrow + (t & 1u);
                dvalid = bb < NB;
            } else {
                dim = 64u * wave + 16u * t + mrow;
                dvalid = 64u * wave + 16u * t < hd;
            }
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                const float tot = acc[hg][t][i] + xor32(acc[hg][t][i]);
                const uint32_t head = hg * 8u + 4u * jg + i;
                if (lane < 32u && dvalid && head < gqa) {
                    if (fin) {
                        const float l = s_l[head];
                        float r = l > 0.f ? tot / l : 0.f;
                        if (it.gate) r *= 1.f / (1.f + expf(-it.gate[(size_t)head * hd + dim]));
                        it.out[(size_t)head * hd + dim] = r;
                    } else {
                        pbase[head * pstride + 2u + dim] = tot;
                    }
                }
            }
        }
    }
    if (!fin && tid < gqa) {
        pbase[tid * pstride] = s_m[tid];
        pbase[tid * pstride + 1u] = s_l[tid];
    }
}

/* Merge the S split partials of one (item, head): weights 2^(m_s - M) over
 * splits with l_s > 0, then the sigmoid gate (src/q4_rocm.cu:6968-7013). */
template <int MODE>
__global__ __launch_bounds__(256) void qsa_comb_k(AttnArgs a) {
    const uint32_t g = blockIdx.x, item = a.item0 + blockIdx.y, d = threadIdx.x;
    const uint32_t gqa = a.n_head / a.n_kvh, hd = a.hd;
    const Item it = resolve_item<MODE>(a, item);
    const size_t pstride = (size_t)hd + 2u;
    const float *pb = a.part + ((size_t)item * a.S * gqa + g) * pstride;
    const size_t sstride = (size_t)gqa * pstride;
    float M = -INFINITY;
    for (uint32_t s = 0; s < a.S; s++) {
        const float m = pb[s * sstride], l = pb[s * sstride + 1u];
        if (l > 0.f) M = fmaxf(M, m);
    }
    float L = 0.f, acc = 0.f;
    for (uint32_t s = 0; s < a.S; s++) {
        const float l = pb[s * sstride + 1u];
        if (l > 0.f) {
            const float w = exp2f(pb[s * sstride] - M);
            L += w * l;
            if (d < hd) acc += w * pb[s * sstride + 2u + d];
        }
    }
    if (d < hd) {
        float r = L > 0.f ? acc / L : 0.f;
        if (it.gate) r *= 1.f / (1.f + expf(-it.gate[(size_t)g * hd + d]));
        it.out[(size_t)g * hd + d] = r;
    }
}

/* ------------------------------------------------------------------------ */

#define Q4KV_TARGET_WG 2048u /* aim for >= 8 workgroups per CU */
#define Q4KV_MAX_GRID_Y 65535u

template <int KIND, int MODE>
static bool launch_kind(AttnArgs a, uint32_t n_items, uint32_t max_n, uint32_t gqa) {
    constexpr uint32_t CP = KCfg<KIND>::CP;
    const uint32_t n_chunks = (max_n + CP - 1u) / CP;
    uint32_t S = (Q4KV_TARGET_WG + n_items - 1u) / n_items;
    if (S > n_chunks) S = n_chunks;
    if (S < 1u) S = 1u;
    const size_t per = (size_t)gqa * (a.hd + 2u);
    while (S > 1u && (size_t)n_items * S * per > q4kv_part_cap) S--;
    if (!q4kv_part) S = 1u;
    const uint32_t cps = n_chunks ? (n_chunks + S - 1u) / S : 1u;
    if (n_chunks) S = (n_chunks + cps - 1u) / cps;
    if (S < 1u) S = 1u;
    a.S = S;
    a.cps = cps;
    a.part = q4kv_part;
    for (uint32_t i0 = 0; i0 < n_items; i0 += Q4KV_MAX_GRID_Y) {
        const uint32_t ni = n_items - i0 < Q4KV_MAX_GRID_Y ? n_items - i0 : Q4KV_MAX_GRID_Y;
        a.item0 = i0;
        dim3 grid(S, ni);
        if (gqa <= 8u)
            qsa_attn_k<KIND, MODE, 1><<<grid, 256, 0, q4kv_stream>>>(a);
        else
            qsa_attn_k<KIND, MODE, 2><<<grid, 256, 0, q4kv_stream>>>(a);
        if (S > 1u) qsa_comb_k<MODE><<<dim3(gqa, ni), 256, 0, q4kv_stream>>>(a);
    }
    return q4kv_launch_ok("qsa attention");
}

template <int MODE>
static bool launch_attn(int kind, const AttnArgs &a, uint32_t n_items, uint32_t max_n) {
    const uint32_t gqa = a.n_head / a.n_kvh;
    switch (kind) {
    case Q4KV_Q8: return launch_kind<Q4KV_Q8, MODE>(a, n_items, max_n, gqa);
    case Q4KV_F16: return launch_kind<Q4KV_F16, MODE>(a, n_items, max_n, gqa);
    case Q4KV_F32: return launch_kind<Q4KV_F32, MODE>(a, n_items, max_n, gqa);
    default: return false;
    }
}

/* Shapes this kernel family supports: head_dim a multiple of 32 up to 256,
 * n_head a multiple of n_kvh with at most 16 query heads per KV head. */
static bool shape_ok(uint32_t n_head, uint32_t n_kvh, uint32_t hd, int kind) {
    if (!n_head || !n_kvh || !hd || hd > 256u || (hd % 32u) || (n_head % n_kvh)) return false;
    if (n_head / n_kvh > 16u) return false;
    return kind >= Q4KV_F32 && kind <= Q4KV_Q8;
}

static AttnArgs base_args(const float *q, const void *kc, const void *vc, const float *gate,
                          float *out, uint32_t n_head, uint32_t n_kvh, uint32_t hd,
                          uint32_t max_kv, float scale) {
    AttnArgs a = {};
    a.kc = (const uint8_t *)kc;
    a.vc = (const uint8_t *)vc;
    a.q = q;
    a.gate = gate;
    a.out = out;
    a.n_head = n_head;
    a.n_kvh = n_kvh;
    a.hd = hd;
    a.max_kv = max_kv;
    a.scale_log2 = scale * 1.4426950408889634f;
    return a;
}

extern "C" bool q4_hip_qsa_decode_n(const float *d_q, const void *d_kcache,
                                    const void *d_vcache, const float *d_gate, float *d_out,
                                    uint32_t n_head, uint32_t n_kvh, uint32_t hd,
                                    uint32_t n_tok, uint32_t kv_base, uint32_t max_kv,
                                    float scale, int kv_f16) {
    if (!q4kv_ok || !d_q || !d_kcache || !d_vcache || !d_gate || !d_out) return false;
    if (n_tok == 0 || !shape_ok(n_head, n_kvh, hd, kv_f16)) return false;
    (void)hipGetLastError();
    AttnArgs a = base_args(d_q, d_kcache, d_vcache, d_gate, d_out, n_head, n_kvh, hd, max_kv,
                           scale);
    a.kv_base = kv_base;
    const uint64_t last = (uint64_t)kv_base + n_tok;
    const uint32_t max_n = last < max_kv ? (uint32_t)last : max_kv;
    return launch_attn<MODE_DENSE>(kv_f16, a, n_tok * n_kvh, max_n);
}

extern "C" bool q4_hip_qsa_decode_idx_kv(const float *d_q, const void *d_kcache,
                                         const void *d_vcache, const float *d_gate,
                                         float *d_out, const int32_t *idx, uint32_t width,
                                         uint64_t tok_stride, uint64_t kvh_stride,
                                         uint32_t n_head, uint32_t n_kvh, uint32_t hd,
                                         uint32_t n_tok, uint32_t max_kv, float scale,
                                         int kv_f16) {
    if (!q4kv_ok || !d_q || !d_kcache || !d_vcache || !d_out || !idx) return false;
    if (n_tok == 0 || width == 0 || !shape_ok(n_head, n_kvh, hd, kv_f16)) return false;
    (void)hipGetLastError();
    AttnArgs a = base_args(d_q, d_kcache, d_vcache, d_gate, d_out, n_head, n_kvh, hd, max_kv,
                           scale);
    a.idx = idx;
    a.width = width;
    a.tok_stride = tok_stride;
    a.kvh_stride = kvh_stride;
    return launch_attn<MODE_INDEXED>(kv_f16, a, n_tok * n_kvh, width);
}

extern "C" bool q4_hip_qsa_decode_idx(const float *d_q, const void *d_kcache,
                                      const void *d_vcache, const float *d_gate, float *d_out,
                                      const int32_t *idx, uint32_t width, uint32_t n_head,
                                      uint32_t n_kvh, uint32_t hd, uint32_t n_tok,
                                      uint32_t max_kv, float scale, int kv_f16) {
    if (!d_gate) return false; /* the reference requires a gate here */
    return q4_hip_qsa_decode_idx_kv(d_q, d_kcache, d_vcache, d_gate, d_out, idx, width, width,
                                    0, n_head, n_kvh, hd, n_tok, max_kv, scale, kv_f16);
}

extern "C" bool q4_hip_qsa_decode(const float *d_q, const void *d_kcache, const void *d_vcache,
                                  const float *d_gate, float *d_out, uint32_t n_head,
                                  uint32_t n_kvh, uint32_t hd, uint32_t n_kv, uint32_t max_kv,
                                  float scale, int kv_f16) {
    if (n_kv == 0) return false;
    return q4_hip_qsa_decode_n(d_q, d_kcache, d_vcache, d_gate, d_out, n_head, n_kvh, hd, 1,
                               n_kv - 1, max_kv, scale, kv_f16);
}

extern "C" bool q4_hip_qsa_decode_batch(const q4kv_seq_desc *d_descs, uint32_t n_seq,
                                        uint32_t n_head, uint32_t n_kvh, uint32_t hd,
                                        float scale, int kv_f16, uint32_t max_n) {
    if (!q4kv_ok || !d_descs || !n_seq || !max_n || !shape_ok(n_head, n_kvh, hd, kv_f16))
        return false;
    (void)hipGetLastError();
    AttnArgs a = base_args(nullptr, nullptr, nullptr, nullptr, nullptr, n_head, n_kvh, hd, 0,
                           scale);
    a.seqs = d_descs;
    return launch_attn<MODE_BATCH>(kv_f16, a, n_seq * n_kvh, max_n);
}

extern "C" bool q4_hip_qsa_topk_alloc(void) { return q4kv_ok && q4kv_part != nullptr; }
