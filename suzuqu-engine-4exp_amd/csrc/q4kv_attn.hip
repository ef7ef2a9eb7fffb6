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
 *    1152 leaves the signed value. The q8_0 fast kernel skips the subtract and
 *    removes the bias on the MFMA pipe instead (accumulator input q x -1152
 *    for Q.K, one more MFMA with a -1152 operand for P.V).
 *  - Online softmax in base 2 per chunk; the split partials (m, l, acc[hd])
 *    are merged by a second kernel that also applies the gate. A single
 *    split (prefill, or short lists) finalises in place.
 */
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <math.h>
#include <stdlib.h>

#include "q4kv_internal.h"

extern "C" {
#include "q4kv.h"
}

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

/* MODE_STEP: MODE_BATCH over q4kv_step_desc entries, with the token's K/V
 * append done by the same launch (fast q8_0 kernel only). */
/* MODE_PSTEP: MODE_STEP over q4kv_prep_step_desc entries, with the query
 * and key preparation (RMSNorm + RoPE) done in the kernel. */
enum { MODE_DENSE = 0, MODE_INDEXED = 1, MODE_BATCH = 2, MODE_STEP = 3, MODE_PSTEP = 4 };
#define IS_STEP(M) ((M) == MODE_STEP || (M) == MODE_PSTEP)
#define IS_BATCH(M) ((M) == MODE_BATCH || IS_STEP(M))

struct AttnArgs {
    const uint8_t *kc, *vc;
    const float *q, *gate;
    float *out;
    const int32_t *idx;
    uint64_t tok_stride, kvh_stride;
    const q4kv_seq_desc *seqs;
    uint32_t desc_stride; /* bytes between descriptors (64, or 96 for steps) */
    float *part;
    uint32_t width, kv_base, max_kv;
    uint32_t n_head, n_kvh, hd;
    uint32_t S, cps, item0;
    float scale_log2;
    /* MODE_PSTEP */
    uint32_t n_rot;
    float rope_base, eps;
    /* prefill band (MODE_INDEXED): per item, the list entries before its
     * band (the slab kernel's list length) and the band's (m, l) per head;
     * the band's unnormalised output rows are in out */
    int32_t *band_nb;
    float *band_ml;
    /* XCD grouping (xcd_slot; 1D grid when xgrp > 0): xgrp (token, split)
     * groups, each run by its n_kvh KV heads' workgroups on one XCD */
    uint32_t xgrp;
    /* the held append of one token's K/V rows ([n_kvh][hd] fp32 each) at
     * the device position *app_pos (qsa_q8d256_k with APP) */
    const float *app_k, *app_v;
    const int32_t *app_pos;
};

struct Item {
    const uint8_t *kc, *vc;
    const float *q, *gate;
    float *out;
    const int32_t *list;
    uint32_t n, max_kv;
    /* index-load source and mask: (list, ~0) for a list, (any readable word,
     * 0) for a dense item, so that loads and selects need no branch */
    const int32_t *lsrc;
    uint32_t lmask;
    /* MODE_STEP: this KV head's new K/V rows and their position */
    const float *knew, *vnew;
    uint32_t pos_new;
    /* MODE_PSTEP: RMSNorm weights; q rows are [q | gate] (head stride 2*hd) */
    const float *wnq, *wnk;
};

template <int MODE>
__device__ static inline Item resolve_item(const AttnArgs &a, uint32_t item) {
    const uint32_t kh = item % a.n_kvh, t = item / a.n_kvh;
    const uint32_t gqa = a.n_head / a.n_kvh;
    const size_t hoff = (size_t)kh * gqa * a.hd;
    Item it;
    it.knew = it.vnew = nullptr;
    it.wnq = it.wnk = nullptr;
    it.pos_new = ~0u;
    if (IS_BATCH(MODE)) {
        /* every descriptor word this mode reads, in one batch of scalar loads
         * issued together (field-by-field loads behind the pointer tests
         * cost extra dependent round trips before the first index load) */
        constexpr uint32_t NW = MODE == MODE_PSTEP ? 28u : IS_STEP(MODE) ? 21u : 15u;
        const uint32_t *dw =
            (const uint32_t *)((const uint8_t *)a.seqs + (size_t)t * a.desc_stride);
        uint32_t w[NW];
#pragma unroll
        for (uint32_t i = 0; i < NW; i++) w[i] = ldg(dw + i);
        /* consume every word here so none of the loads sinks to its use */
#pragma unroll
        for (uint32_t i = 0; i < NW; i++) asm volatile("" ::"s"(w[i]));
        auto word = [&](uint32_t byte_off) {
            return (uintptr_t)w[byte_off / 4u] | ((uintptr_t)w[byte_off / 4u + 1u] << 32);
        };
        /* descriptor pointers as global-address-space pointers: accesses
         * through them need no flat instructions */
        static_assert(offsetof(q4kv_seq_desc, kcache) == 0 && offsetof(q4kv_seq_desc, vcache) == 8 &&
                          offsetof(q4kv_seq_desc, q) == 16 && offsetof(q4kv_seq_desc, gate) == 24 &&
                          offsetof(q4kv_seq_desc, out) == 32 && offsetof(q4kv_seq_desc, idx) == 40 &&
                          offsetof(q4kv_seq_desc, n_sel) == 48 &&
                          offsetof(q4kv_seq_desc, idx_kvh_stride) == 52 &&
                          offsetof(q4kv_seq_desc, max_kv) == 56,
                      "q4kv_seq_desc layout");
        static_assert(offsetof(q4kv_step_desc, k) == 64 && offsetof(q4kv_step_desc, v) == 72 &&
                          offsetof(q4kv_step_desc, pos) == 80,
                      "q4kv_step_desc layout");
        static_assert(offsetof(q4kv_prep_step_desc, wn_q) == 96 &&
                          offsetof(q4kv_prep_step_desc, wn_k) == 104,
                      "q4kv_prep_step_desc layout");
        const float *gate = q4kv_gptr<const float>(word(24));
        const int32_t *idx = q4kv_gptr<const int32_t>(word(40));
        const uint32_t n_sel = w[12];
        it.kc = q4kv_gptr<const uint8_t>(word(0));
        it.vc = q4kv_gptr<const uint8_t>(word(8));
        it.q = q4kv_gptr<const float>(word(16)) + hoff * (MODE == MODE_PSTEP ? 2u : 1u);
        it.gate = gate ? gate + hoff : nullptr;
        it.out = q4kv_gptr<float>(word(32)) + hoff;
        it.max_kv = w[14];
        it.list = idx ? idx + (size_t)kh * w[13] : nullptr;
        it.n = idx ? n_sel : (n_sel < it.max_kv ? n_sel : it.max_kv);
        it.lsrc = idx ? it.list : (const int32_t *)a.seqs;
        it.lmask = idx ? ~0u : 0u;
        if (IS_STEP(MODE)) {
            it.knew = q4kv_gptr<const float>(word(64)) + (size_t)kh * a.hd;
            it.vnew = q4kv_gptr<const float>(word(72)) + (size_t)kh * a.hd;
            it.pos_new = w[20];
        }
        if (MODE == MODE_PSTEP) {
            it.wnq = q4kv_gptr<const float>(word(96));
            it.wnk = q4kv_gptr<const float>(word(104));
        }
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
            it.lsrc = it.list;
            it.lmask = ~0u;
        } else {
            const uint32_t nkv = a.kv_base + t + 1u;
            it.list = nullptr;
            it.n = nkv < a.max_kv ? nkv : a.max_kv;
            it.lsrc = nullptr;
            it.lmask = 0u;
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
/* v + (value of the lane 32 apart): the swap leaves each lane's own value in
 * one result and its partner's in the other, so their sum needs no select. */
__device__ static inline float pair32_sum(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                              false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
/* max(a, b) for non-NaN operands in one v_med3_f32 (fmaxf adds NaN-quieting
 * canonicalisations of both operands). */
__device__ static inline float fmax2(float a, float b) {
    return __builtin_amdgcn_fmed3f(a, b, INFINITY);
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

/* x -> fp16 hi part (nsel = 0) or fp16 residual x - hi (nsel = -1) without a
 * select: one conversion and one mixed-precision FMA (v_fma_mix). */
__device__ static inline _Float16 split_sel(float x, float nsel) {
    const _Float16 h = (_Float16)x;
    return (_Float16)__builtin_fmaf(nsel, (float)h, x);
}

/* x -> fp16 hi part (rows < 8) or fp16 residual (rows >= 8). */
__device__ static inline _Float16 split_hl(float x, bool lo) {
    _Float16 h = (_Float16)x;
    return lo ? (_Float16)(x - (float)h) : h;
}

#ifdef Q4KV_TRACE
/* Debug-only phase timestamps (100 MHz wall clock) of thread 0 of every
 * workgroup: [block][slot]. Not compiled into the product library. */
__device__ uint64_t q4kv_trace_buf[4096 * 16];
#define TRACE(slot)                                                                \
    do {                                                                           \
        if (threadIdx.x == 0)                                                      \
            q4kv_trace_buf[((blockIdx.y * gridDim.x + blockIdx.x) & 4095u) * 16u + (slot)] = \
                wall_clock64();                                                    \
    } while (0)
/* per wave: [wave][slot] for the first 4096 waves of the launch (later
 * waves are not recorded, so no slot mixes two waves) */
#define TRACEW(slot)                                                                   \
    do {                                                                               \
        const uint32_t tw_ = (blockIdx.y * gridDim.x + blockIdx.x) * (blockDim.x >> 6) + \
                             (threadIdx.x >> 6);                                       \
        if ((threadIdx.x & 63u) == 0 && tw_ < 4096u)                                   \
            q4kv_trace_buf[tw_ * 16u + (slot)] = wall_clock64();                       \
    } while (0)
/* the prefill band kernel's own per-wave stamps (it runs before the slab
 * kernel of the same call, which would overwrite q4kv_trace_buf) */
__device__ uint64_t q4kv_trace_band[4096 * 16];
#define TRACEB(slot)                                                                   \
    do {                                                                               \
        const uint32_t tw_ = (blockIdx.y * gridDim.x + blockIdx.x) * (blockDim.x >> 6) + \
                             (threadIdx.x >> 6);                                       \
        if ((threadIdx.x & 63u) == 0 && tw_ < 4096u)                                   \
            q4kv_trace_band[tw_ * 16u + (slot)] = wall_clock64();                      \
    } while (0)
#else
#define TRACE(slot) do { } while (0)
#define TRACEW(slot) do { } while (0)
#define TRACEB(slot) do { } while (0)
#endif

template <int KIND> struct KCfg;
template <> struct KCfg<Q4KV_Q8> { static constexpr uint32_t CP = 64, RMAX = 272; };
template <> struct KCfg<Q4KV_F16> { static constexpr uint32_t CP = 64, RMAX = 512; };
template <> struct KCfg<Q4KV_F32> { static constexpr uint32_t CP = 32, RMAX = 1024; };

typedef float fv2 __attribute__((ext_vector_type(2)));

/* Position of list entry j of an item, or -1 (padding, beyond the list, or
 * outside the cache). */
__device__ static inline int32_t item_pos(const Item &it, uint32_t j) {
    if (j >= it.n) return -1;
    int32_t p = it.list ? ldg(it.list + j) : (int32_t)j;
    return (p < 0 || (uint32_t)p >= it.max_kv) ? -1 : p;
}

/* Positions of list entries j[0..N), in two steps so that the index loads
 * (issued back to back, one memory round trip) are only waited for where
 * the positions are used: pos_issue loads the raw entries, pos_finish
 * maps them to positions (-1 for padding / out of range). Requires n > 0. */
template <int N, int MODE>
__device__ static inline void pos_issue(const Item &it, const uint32_t (&j)[N],
                                        int32_t (&raw)[N]) {
    if (MODE == MODE_DENSE) {
#pragma unroll
        for (int u = 0; u < N; u++) raw[u] = (int32_t)j[u];
    } else {
        /* no branch on the list pointer (a branch would force a wait at its
         * merge): dense batch items load a harmless word and keep j */
        const uint32_t m = MODE == MODE_INDEXED ? ~0u : it.lmask;
#pragma unroll
        for (int u = 0; u < N; u++) {
            const uint32_t jj = (j[u] < it.n ? j[u] : it.n - 1u) & m;
            raw[u] = *(const GLOBAL int32_t *)(it.lsrc + jj);
        }
    }
}
template <int N, int MODE>
__device__ static inline void pos_finish(const Item &it, const uint32_t (&j)[N],
                                         const int32_t (&raw)[N], int32_t (&p)[N]) {
    const uint32_t m = MODE == MODE_INDEXED ? ~0u : (IS_BATCH(MODE) ? it.lmask : 0u);
#pragma unroll
    for (int u = 0; u < N; u++) {
        const int32_t r = (int32_t)(((uint32_t)raw[u] & m) | (j[u] & ~m));
        p[u] = (j[u] < it.n && r >= 0 && (uint32_t)r < it.max_kv) ? r : -1;
    }
}

/* 16 bytes global -> LDS without passing through VGPRs (gfx950
 * global_load_lds_dwordx4). Every active lane of the wave writes its 16 bytes
 * at lds_wave_base + 16*lane. */
__device__ static inline void dma16(const void *src, void *lds_wave_base) {
    __builtin_amdgcn_global_load_lds((const GLOBAL void *)src, (LOCAL void *)lds_wave_base, 16,
                                     0, 0);
}

/* 16 bytes global -> LDS like dma16, issued from inline assembly so that the
 * compiler does not add its own wait for the DMA before every LDS read of
 * the staging buffers (it cannot tell the two buffers apart); the kernels
 * that use it wait for their DMAs themselves, with explicit vmcnt counts.
 * m0 is a reserved register, so its clobber is not honoured (the compiler
 * warns): the kernels that use this issue every DMA through it and hold
 * nothing of their own in m0 (checked in their gfx950 assembly: every m0
 * write there is this s_mov_b32). */
__device__ static inline void dma16_manual(const void *src, void *lds_wave_base) {
    const uint32_t m0 =
        __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(LOCAL void *)lds_wave_base);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(m0), "v"((const GLOBAL void *)src)
                 : "memory", "m0");
}
/* Reductions over the 16 lanes of a DPP row (one MFMA column group). */
template <int CTRL> __device__ static inline float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
__device__ static inline float row16_max(float v) {
    v = fmax2(v, dppf<0xB1>(v));  /* quad_perm [1,0,3,2] */
    v = fmax2(v, dppf<0x4E>(v));  /* quad_perm [2,3,0,1] */
    v = fmax2(v, dppf<0x141>(v)); /* row_half_mirror */
    return fmax2(v, dppf<0x140>(v)); /* row_mirror */
}
/* Maxima of four values over their DPP rows, one v_max_f32_dpp per step. The
 * compiler folds fmed3(a, b, +inf) back into maxnum and then canonicalises
 * both operands of every max (three instructions a step), so the steps are
 * written out: the four chains interleave, which gives each DPP read the two
 * wait states it needs after the previous write of its source; the s_nop
 * covers the first step. Operands are scores or -inf, never NaN. */
__device__ static inline void row16_max4(float (&v)[4]) {
#define Q4KV_DPPMAX4(CTL)                                                                      \
    "v_max_f32_dpp %0, %0, %0 " CTL " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"            \
    "v_max_f32_dpp %1, %1, %1 " CTL " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"            \
    "v_max_f32_dpp %2, %2, %2 " CTL " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"            \
    "v_max_f32_dpp %3, %3, %3 " CTL " row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
    asm("s_nop 1\n\t" Q4KV_DPPMAX4("quad_perm:[1,0,3,2]") Q4KV_DPPMAX4("quad_perm:[2,3,0,1]")
            Q4KV_DPPMAX4("row_half_mirror") Q4KV_DPPMAX4("row_mirror")
        : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]));
#undef Q4KV_DPPMAX4
}
/* max(a, b, c) in one v_max3_f32, without the canonicalisations (non-NaN
 * operands). */
__device__ static inline float fmax3v(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ static inline float row16_sum(float v) {
    v += dppf<0xB1>(v);
    v += dppf<0x4E>(v);
    v += dppf<0x141>(v);
    return v + dppf<0x140>(v);
}

/* Sum and maximum over the 64 lanes of a wave (every lane gets the result). */
__device__ static inline float wave_sum64(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ static inline float wave_max64(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

/* Partial row layout: [m, l, 256 columns in MFMA output order]. */
#define PSTRIDE 258u

/* Head dimension held by output column col (MFMA order) of a wave's tiles:
 * q8_0 tiles pair even/odd dims of one 32-block (the two bytes a 16-bit LDS
 * read returns), f16/f32 tiles are 16 consecutive dims. */
template <int KIND> __device__ static inline uint32_t col_dim(uint32_t col) {
    if (KIND != Q4KV_Q8) return col;
    const uint32_t w = col >> 6, t = (col >> 4) & 3u, n = col & 15u;
    return 32u * (2u * w + (t >> 1)) + 2u * n + (t & 1u);
}

/* The (split, item) of this workgroup. With a.xgrp > 0 the grid is 1D and
 * groups the n_kvh KV heads of each (token, split) on one XCD: workgroup L
 * runs on XCD L mod 8 (MI355X dispatches workgroups round-robin over its 8
 * XCDs), and group P = 8 (r / n_kvh) + L mod 8 with r = L / 8 takes
 * workgroups L of one residue mod 8. A position's head rows are adjacent, so
 * the lines they share are fetched once into that XCD's L2. Placement only:
 * results do not depend on it. Returns false for the padding of the last
 * group row. */
__device__ static inline bool xcd_slot(const AttnArgs &a, uint32_t &s, uint32_t &item) {
    if (!a.xgrp) {
        s = blockIdx.x;
        item = a.item0 + blockIdx.y;
        return true;
    }
    const uint32_t L = blockIdx.x, r = L >> 3, kh = r % a.n_kvh;
    const uint32_t P = (r / a.n_kvh) * 8u + (L & 7u);
    const uint32_t t = P / a.S;
    s = P - t * a.S;
    item = a.item0 + t * a.n_kvh + kh;
    return P < a.xgrp;
}

template <int KIND, int MODE, int HG>
__global__ __launch_bounds__(256) void qsa_attn_k(AttnArgs a) {
    constexpr uint32_t CP = KCfg<KIND>::CP;
    constexpr uint32_t RMAX = KCfg<KIND>::RMAX;
    constexpr uint32_t NH = HG * 8u;     /* query-head slots */
    constexpr uint32_t NQW = CP / 16u;   /* waves computing scores */
    constexpr uint32_t NLD = (CP * RMAX / 16u + 255u) / 256u;
    __shared__ __attribute__((aligned(16))) uint8_t kraw[CP * RMAX];
    __shared__ __attribute__((aligned(16))) uint8_t vraw[CP * RMAX];
    __shared__ __attribute__((aligned(16))) float sc[NH * CP];
    __shared__ __attribute__((aligned(16))) float vsc[KIND == Q4KV_Q8 ? 8u * CP : 4u];
    __shared__ int32_t s_pos[CP];
    __shared__ float s_cmax[NQW][NH], s_psum[NQW][NH];
    /* per head: scale_log2 x 2^e, e the power of two its q was divided by */
    __shared__ float s_qm[NH];

    TRACE(0);
    uint32_t s, item;
    if (!xcd_slot(a, s, item)) return; /* padding of the last group row */
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t hd = a.hd, NB = hd / 32u, gqa = a.n_head / a.n_kvh;
    const uint32_t kh = item % a.n_kvh;
    const Item it = resolve_item<MODE>(a, item);
    const uint32_t rowb =
        KIND == Q4KV_Q8 ? NB * 34u : hd * (KIND == Q4KV_F16 ? 2u : 4u);
    /* LDS row stride: rows packed back to back when 16-byte granular (the
     * DMA writes contiguous 16-byte chunks), padded otherwise. */
    const uint32_t RS = (rowb + 15u) & ~15u;
    const bool al16 =
        (rowb & 15u) == 0 && ((((uintptr_t)it.kc) | ((uintptr_t)it.vc)) & 15u) == 0;
    const uint32_t n_chunks = (it.n + CP - 1u) / CP;
    const uint32_t c0 = s * a.cps;
    const uint32_t c1 = (s + 1u == a.S) ? n_chunks : min(c0 + a.cps, n_chunks);
    const uint32_t nch = rowb / 16u, total = CP * nch;

    const uint32_t mrow = lane & 15u; /* MFMA A row / B,C column */
    const uint32_t jg = lane >> 4;    /* MFMA k-group; C rows 4jg..4jg+3 */
    const bool lo_row = mrow >= 8u;

    /* ---- positions of the first chunk: all index loads in flight at once ---- */
    /* pidx[0..NLD) = rows this lane DMAs, pidx[NLD] = s_pos entry tid */
    int32_t pidx[NLD + 1];
    uint32_t jrow[NLD + 1];
#pragma unroll
    for (uint32_t u = 0; u < NLD; u++) {
        const uint32_t e = (wave + 4u * u) * 64u + lane;
        jrow[u] = e < total ? e / nch : 0u;
    }
    jrow[NLD] = tid < CP ? tid : 0u;
    uint32_t jcur[NLD + 1];
    int32_t raw[NLD + 1];
#pragma unroll
    for (uint32_t u = 0; u <= NLD; u++) {
        jcur[u] = c0 * CP + jrow[u];
        raw[u] = -1;
    }
    if (c0 < c1) pos_issue<NLD + 1, MODE>(it, jcur, raw);

    /* ---- Q operands straight from global (8-byte loads), hi/lo split
     * across the row halves; overlaps the index round trip ---- */
    h8_t qa[HG][8];
    /* raw fp32 pairs (all loads in flight together), split in the first
     * chunk once the row DMAs are issued */
    fv2 qv[HG][8][4];
    {
        const float *qh[HG];
#pragma unroll
        for (uint32_t hg = 0; hg < HG; hg++) {
            const uint32_t g = hg * 8u + (mrow & 7u);
            qh[hg] = it.q + (size_t)(g < gqa ? g : 0u) * hd;
        }
        if ((((uintptr_t)it.q) & 7u) == 0) {
#pragma unroll
            for (uint32_t hg = 0; hg < HG; hg++)
#pragma unroll
                for (uint32_t b = 0; b < 8u; b++)
#pragma unroll
                    for (uint32_t k = 0; k < 4u; k++) {
                        const uint32_t d =
                            KIND == Q4KV_Q8 ? q8_kdim(b, jg, 2u * k) : 8u * jg + 2u * k;
                        /* blocks beyond hd re-read block 0 and are zeroed below */
                        qv[hg][b][k] = ldg((const fv2 *)(qh[hg] + 32u * (b < NB ? b : 0u) + d));
                    }
        } else {
#pragma unroll
            for (uint32_t hg = 0; hg < HG; hg++)
#pragma unroll
                for (uint32_t b = 0; b < 8u; b++)
#pragma unroll
                    for (uint32_t k = 0; k < 4u; k++) {
                        const uint32_t d =
                            KIND == Q4KV_Q8 ? q8_kdim(b, jg, 2u * k) : 8u * jg + 2u * k;
                        const float *pq = qh[hg] + 32u * (b < NB ? b : 0u) + d;
                        qv[hg][b][k][0] = ldg(pq);
                        qv[hg][b][k][1] = ldg(pq + 1);
                    }
        }
    }

    /* running max (base 2) and sum of the heads of this lane's C rows */
    float m_run[HG][4], l_run[HG][4];
    f4_t acc[HG][4];
#pragma unroll
    for (uint32_t hg = 0; hg < HG; hg++)
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            m_run[hg][i] = -INFINITY;
            l_run[hg][i] = 0.f;
            acc[hg][i] = (f4_t){0.f, 0.f, 0.f, 0.f};
        }
    TRACE(1);

    for (uint32_t c = c0; c < c1; c++) {
        const uint32_t base = c * CP;
        pos_finish<NLD + 1, MODE>(it, jcur, raw, pidx);
        if (tid < CP) s_pos[tid] = pidx[NLD];
        /* ---- K/V rows of this chunk -> LDS; invalid positions read row 0
         * (their scores are masked) ---- */
        if (al16) {
#pragma unroll
            for (uint32_t u = 0; u < NLD; u++) {
                const uint32_t e0 = (wave + 4u * u) * 64u, e = e0 + lane;
                if (e < total) {
                    const uint32_t r = e / nch, q = e - r * nch;
                    const int32_t p = pidx[u] < 0 ? 0 : pidx[u];
                    const size_t off = ((size_t)p * a.n_kvh + kh) * rowb + q * 16u;
                    dma16(it.kc + off, kraw + e0 * 16u);
                    dma16(it.vc + off, vraw + e0 * 16u);
                }
            }
        } else {
            const uint32_t nh = rowb / 2u;
            for (uint32_t e = tid; e < CP * nh; e += 256u) {
                const uint32_t r = e / nh, q = e - r * nh;
                int32_t p = item_pos(it, base + r);
                p = p < 0 ? 0 : p;
                const size_t off = ((size_t)p * a.n_kvh + kh) * rowb + q * 2u;
                *(uint16_t *)(kraw + r * RS + q * 2u) = ldg((const uint16_t *)(it.kc + off));
                *(uint16_t *)(vraw + r * RS + q * 2u) = ldg((const uint16_t *)(it.vc + off));
            }
        }
        if (c == c0) {
#pragma unroll
            for (uint32_t hg = 0; hg < HG; hg++) {
                const uint32_t g = hg * 8u + (mrow & 7u);
                /* q divided by the power of two 2^e that brings the head's
                 * largest |q| into [0.5, 1) (exact): its fp16 parts never
                 * overflow; the scores are multiplied by scale_log2 x 2^e.
                 * The head's lanes: rows g, g + 8, k-groups 0-3. */
                float am = 0.f;
#pragma unroll
                for (uint32_t b = 0; b < NB; b++)
#pragma unroll
                    for (uint32_t k = 0; k < 4u; k++)
                        am = fmaxf(am, fmaxf(fabsf(qv[hg][b][k][0]), fabsf(qv[hg][b][k][1])));
                am = fmaxf(am, __shfl_xor(am, 8));
                am = fmaxf(am, __shfl_xor(am, 16));
                am = fmaxf(am, __shfl_xor(am, 32));
                const int e = (am > 0.f && am <= 3.4e38f) ? __builtin_amdgcn_frexp_expf(am) : 0;
                const float qf = __builtin_ldexpf(1.f, -e);
                if (jg == 0u && mrow < 8u) s_qm[g] = __builtin_ldexpf(a.scale_log2, e);
#pragma unroll
                for (uint32_t b = 0; b < 8u; b++) {
                    const float qscale = (g < gqa && b < NB) ? qf : 0.f;
#pragma unroll
                    for (uint32_t k = 0; k < 4u; k++) {
                        qa[hg][b][2u * k] = split_hl(qv[hg][b][k][0] * qscale, lo_row);
                        qa[hg][b][2u * k + 1u] = split_hl(qv[hg][b][k][1] * qscale, lo_row);
                    }
                }
            }
        }
        TRACE(2);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        TRACE(3);
        /* ---- prefetch the next chunk's positions (lands during compute) ---- */
        if (c + 1u < c1) {
#pragma unroll
            for (uint32_t u = 0; u <= NLD; u++) jcur[u] = base + CP + jrow[u];
            pos_issue<NLD + 1, MODE>(it, jcur, raw);
        }
        if (KIND == Q4KV_Q8) {
            for (uint32_t e = tid; e < NB * CP; e += 256u) {
                const uint32_t b = e / CP, r = e - b * CP;
                vsc[b * CP + r] = s_pos[r] < 0 ? 0.f : ld_f16(vraw + r * RS + 34u * b);
            }
        }
        /* ---- scores for positions 16w .. 16w+15, chunk max per head ---- */
        f4_t T[HG];
        const uint32_t r = wave * 16u + mrow;
        if (wave < NQW) {
            const uint8_t *krow = kraw + r * RS;
            f4_t S[HG];
#pragma unroll
            for (uint32_t hg = 0; hg < HG; hg++) S[hg] = (f4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t b = 0; b < 8u; b++) {
                if (b < NB) {
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
                            S[hg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[hg][b], kb,
                                                                           S[hg], 0, 0, 0);
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
                            S[hg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[hg][b], kh8,
                                                                           S[hg], 0, 0, 0);
                            S[hg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[hg][b], kl8,
                                                                           S[hg], 0, 0, 0);
                        }
                    }
                }
            }
            const bool valid = s_pos[r] >= 0;
#pragma unroll
            for (uint32_t hg = 0; hg < HG; hg++) {
#pragma unroll
                for (uint32_t i = 0; i < 4u; i++) {
                    const float tot = S[hg][i] + xor32(S[hg][i]);
                    T[hg][i] = valid ? tot * s_qm[hg * 8u + ((4u * jg + i) & 7u)] : -INFINITY;
                    const float cm = row16_max(T[hg][i]);
                    if (mrow == 0 && jg < 2u) s_cmax[wave][hg * 8u + 4u * jg + i] = cm;
                }
            }
        }
        TRACE(4);
        __syncthreads();
        TRACE(5);
        /* ---- new running max for this lane's heads; weights of this chunk ---- */
        float alpha[HG][4];
#pragma unroll
        for (uint32_t hg = 0; hg < HG; hg++)
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                const uint32_t h = hg * 8u + ((4u * jg + i) & 7u);
                float cm = s_cmax[0][h];
#pragma unroll
                for (uint32_t w = 1; w < NQW; w++) cm = fmaxf(cm, s_cmax[w][h]);
                const float mn = fmaxf(m_run[hg][i], cm);
                alpha[hg][i] = m_run[hg][i] == -INFINITY ? 0.f : exp2f(m_run[hg][i] - mn);
                m_run[hg][i] = mn;
            }
        if (wave < NQW) {
#pragma unroll
            for (uint32_t hg = 0; hg < HG; hg++)
#pragma unroll
                for (uint32_t i = 0; i < 4u; i++) {
                    const float w = T[hg][i] == -INFINITY ? 0.f : exp2f(T[hg][i] - m_run[hg][i]);
                    const uint32_t h = hg * 8u + 4u * jg + i;
                    if (lane < 32u) sc[h * CP + r] = w;
                    const float ps = row16_sum(w);
                    if (mrow == 0 && jg < 2u) s_psum[wave][h] = ps;
                }
        }
        TRACE(6);
        __syncthreads();
        TRACE(7);
        /* ---- running sums; P.V with wave w owning head dims 64w .. 64w+63 ---- */
#pragma unroll
        for (uint32_t hg = 0; hg < HG; hg++)
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                const uint32_t h = hg * 8u + ((4u * jg + i) & 7u);
                float ps = 0.f;
#pragma unroll
                for (uint32_t w = 0; w < NQW; w++) ps += s_psum[w][h];
                l_run[hg][i] = l_run[hg][i] * alpha[hg][i] + ps;
#pragma unroll
                for (uint32_t t = 0; t < 4u; t++) acc[hg][t][i] *= alpha[hg][i];
            }
#pragma unroll
        for (uint32_t kc = 0; kc < CP / 32u; kc++) {
            const uint32_t p0 = 32u * kc + 8u * jg;
            if (KIND == Q4KV_Q8) {
#pragma unroll
                for (uint32_t u = 0; u < 2u; u++) {
                    const uint32_t bb = 2u * wave + u;
                    if (bb < NB) {
                        /* B: dims 32bb + 2n (tile 0) and 32bb + 2n + 1 (tile 1). */
                        const uint8_t *vb = vraw + p0 * RS + 34u * bb + 2u + 2u * mrow;
                        u4_t r0, r1;
#pragma unroll
                        for (uint32_t k = 0; k < 4u; k++) {
                            uint32_t x =
                                (uint32_t)*(const uint16_t *)(vb + (2u * k) * RS) |
                                ((uint32_t)*(const uint16_t *)(vb + (2u * k + 1u) * RS) << 16);
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
                            acc[hg][2u * u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                A, B0, acc[hg][2u * u], 0, 0, 0);
                            acc[hg][2u * u + 1u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                A, B1, acc[hg][2u * u + 1u], 0, 0, 0);
                        }
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
                    if (64u * wave + 16u * t < hd) {
                        if (KIND == Q4KV_F16) {
                            const uint8_t *vb = vraw + p0 * RS + 2u * dim;
                            u4_t rr;
#pragma unroll
                            for (uint32_t k = 0; k < 4u; k++)
                                rr[k] = (uint32_t)*(const uint16_t *)(vb + (2u * k) * RS) |
                                        ((uint32_t)*(const uint16_t *)(vb + (2u * k + 1u) * RS)
                                         << 16);
                            const h8_t B = __builtin_bit_cast(h8_t, rr);
#pragma unroll
                            for (uint32_t hg = 0; hg < HG; hg++)
                                acc[hg][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    A[hg], B, acc[hg][t], 0, 0, 0);
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
                                acc[hg][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    A[hg], Bh, acc[hg][t], 0, 0, 0);
                                acc[hg][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    A[hg], Bl, acc[hg][t], 0, 0, 0);
                            }
                        }
                    }
                }
            }
        }
        TRACE(8);
        __syncthreads();
        TRACE(9);
    }

    /* ---- epilogue: fold lo rows into hi rows, then finalise or spill ---- */
    const bool fin = a.S == 1u;
    float *pbase = fin ? nullptr : a.part + ((size_t)item * a.S + s) * gqa * PSTRIDE;
#pragma unroll
    for (uint32_t hg = 0; hg < HG; hg++) {
#pragma unroll
        for (uint32_t t = 0; t < 4u; t++) {
            const uint32_t col = (wave * 4u + t) * 16u + mrow;
            const uint32_t dim = col_dim<KIND>(col);
            const bool dvalid = dim < hd;
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                const float tot = acc[hg][t][i] + xor32(acc[hg][t][i]);
                const uint32_t head = hg * 8u + 4u * jg + i;
                if (lane < 32u && dvalid && head < gqa) {
                    if (fin) {
                        const float l = l_run[hg][i];
                        float rv = l > 0.f ? tot / l : 0.f;
                        if (it.gate)
                            rv *= 1.f / (1.f + expf(-ldg(it.gate + (size_t)head * hd + dim)));
                        stg(it.out + (size_t)head * hd + dim, rv);
                    } else {
                        stg(pbase + head * PSTRIDE + 2u + col, tot);
                    }
                }
            }
        }
        if (!fin && wave == 0 && mrow == 0 && jg < 2u) {
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                const uint32_t head = hg * 8u + 4u * jg + i;
                if (head < gqa) {
                    stg(pbase + head * PSTRIDE, m_run[hg][i]);
                    stg(pbase + head * PSTRIDE + 1u, l_run[hg][i]);
                }
            }
        }
    }
    TRACE(10);
}

/* MFMA output column (fast kernel tile order) holding head dimension d. */
__device__ static inline uint32_t q8_col_of_dim(uint32_t d) {
    const uint32_t bb = d >> 5, w = bb >> 1;
    const uint32_t t = 2u * (bb & 1u) + (d & 1u), n = (d & 31u) >> 1;
    return (w * 4u + t) * 16u + n;
}

/* Fast path for the production shape: q8_0 cache, head_dim 256 (272-byte
 * rows, 17 x 16 B), at most 8 query heads per KV head. Same algorithm as
 * qsa_attn_k with every shape constant compile-time, the weight hi/lo split
 * done with mixed-precision FMAs, and the partial / output rows staged
 * through LDS for 16-byte stores. */
/* MFMA A operands of the Q.K product from the fp32 Q rows in LDS (1040-byte
 * stride, q8_kdim order): rows 0-7 fp16(q), rows 8-15 the residual
 * (nsel = -1); rows past gqa are zero. qbias[b] = qa[b] x (-1152) is the
 * accumulator input that removes the +1152 bias of the K operands. */
/* Each head's q is first scaled by the power of two 2^-e that brings its
 * largest |q| into [0.5, 1) (exact), so the fp16 parts never overflow and
 * keep their relative precision at any magnitude of q; the score of head g
 * is then multiplied by scale_log2 * 2^e, which build_qa stores in qm[g]
 * (lanes of k-group 0). */
__device__ static inline void build_qa(const float *qraw, uint32_t g, uint32_t gqa, uint32_t jg,
                                       float nsel, h8_t (&qa)[8], f4_t (&qbias)[8],
                                       float scale_log2, float *qm) {
    const float *qr = qraw + (g < gqa ? g : 0u) * 260u;
    fv2 v[32];
    float amax = 0.f;
#pragma unroll
    for (uint32_t b = 0; b < 8u; b++)
#pragma unroll
        for (uint32_t kk = 0; kk < 4u; kk++) {
            v[4u * b + kk] = *(const fv2 *)(qr + 32u * b + q8_kdim(b, jg, 2u * kk));
            amax = fmaxf(amax, fmaxf(fabsf(v[4u * b + kk][0]), fabsf(v[4u * b + kk][1])));
        }
    /* the eight lanes of head g: rows g and g + 8, k-groups 0-3 */
    amax = fmaxf(amax, __shfl_xor(amax, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const int e = (amax > 0.f && amax <= 3.4e38f) ? __builtin_amdgcn_frexp_expf(amax) : 0;
    const float qs = g < gqa ? __builtin_ldexpf(1.f, -e) : 0.f;
    if (jg == 0u && (threadIdx.x & 15u) < 8u) qm[g] = __builtin_ldexpf(scale_log2, e);
#pragma unroll
    for (uint32_t b = 0; b < 8u; b++)
#pragma unroll
        for (uint32_t kk = 0; kk < 4u; kk++) {
            qa[b][2u * kk] = split_sel(v[4u * b + kk][0] * qs, nsel);
            qa[b][2u * kk + 1u] = split_sel(v[4u * b + kk][1] * qs, nsel);
        }
    const h8_t neg = (h8_t)((_Float16)-1152.0f);
#pragma unroll
    for (uint32_t b = 0; b < 8u; b++)
        qbias[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[b], neg, (f4_t){0.f, 0.f, 0.f, 0.f}, 0, 0,
                                                          0);
}

/* DB: two row buffers, chunk c + 1's rows DMA'd while chunk c is computed
 * (for workgroups with many chunks: prefill); the Q rows are staged in the
 * second buffer, which the first chunk does not use. */
/* APP: the launch also performs a held append of one token's K/V rows at
 * the device position (the splits that list that position take its
 * quantised bytes in LDS; split 0 of token 0 writes them to the caches). */
template <int MODE, bool DB, bool APP = false>
__global__ __launch_bounds__(256, 2) void qsa_q8d256_k(AttnArgs a) {
    constexpr uint32_t CP = 64, ROWB = 272, NCH = 17, NLD = 5;
    /* row buffers: [K rows | V rows] each */
    __shared__ __attribute__((aligned(16))) uint8_t rowbuf[DB ? 2 : 1][2 * CP * ROWB];
    /* DB: weights [head][pos] and V scales [block][pos], combined per P.V
     * tile. Single buffer: the P.V A operands themselves, fp16 hi | lo of
     * weight x V scale, [block][hi, lo][head][pos] with 72-entry rows (16-byte
     * pad: the 16 rows a wave's operand reads touch start 4 banks apart) */
    constexpr uint32_t AROW = 72;
    __shared__ __attribute__((aligned(16))) float sw[DB ? 8 * CP : 1];
    __shared__ __attribute__((aligned(16))) float vsc[DB ? 8 * CP : 1];
    __shared__ __attribute__((aligned(16))) _Float16 aop[DB ? 1 : 8 * 2 * 8 * AROW];
    /* raw fp32 Q rows, 1040-byte stride (4 pad floats) against bank conflicts */
    __shared__ __attribute__((aligned(16))) float qraw_s[DB ? 1 : 8 * 260];
    float *const qraw = DB ? (float *)rowbuf[DB ? 1 : 0] : qraw_s;
    __shared__ int32_t s_pos[DB ? 2 : 1][CP];
    __shared__ float s_cmax[4][8], s_psum[4][8], s_ml[2][8];
    /* per-head score multipliers (scale_log2 x 2^e of the q pre-scaling) */
    __shared__ float s_qm[8];
    __shared__ uint32_t s_subst[2];
    __shared__ __attribute__((aligned(16))) float kst[MODE == MODE_PSTEP ? 256 : 1];

    TRACE(0);
    constexpr bool STEPL = IS_STEP(MODE) || APP; /* a token's rows are appended */
    uint32_t s, item;
    if (!xcd_slot(a, s, item)) return; /* padding of the last group row */
    /* the wave index in a scalar register: the LDS addresses derived from it
     * are then uniform without a readfirstlane per row DMA */
    const uint32_t tid = threadIdx.x, lane = tid & 63u,
                   wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    /* query heads h0 .. h0 + gqa - 1 of the KV head: blockIdx.z is the group
     * of 8 (9-16 heads per KV head run as two groups over the same rows) */
    const uint32_t gqa_all = a.n_head / a.n_kvh, h0 = 8u * blockIdx.z;
    const uint32_t gqa = gqa_all - h0 < 8u ? gqa_all - h0 : 8u;
    const uint32_t kh = item % a.n_kvh;
    Item it = resolve_item<MODE>(a, item);
    if (h0) {
        it.q += (size_t)h0 * (MODE == MODE_PSTEP ? 512u : 256u);
        it.out += (size_t)h0 * 256u;
        if (it.gate) it.gate += (size_t)h0 * 256u;
    }
    if (APP) {
        it.knew = a.app_k + (size_t)kh * 256u;
        it.vnew = a.app_v + (size_t)kh * 256u;
        it.pos_new = (uint32_t)ldg(a.app_pos);
    }
    const bool al16 = ((((uintptr_t)it.kc) | ((uintptr_t)it.vc)) & 15u) == 0;
    const uint32_t n_chunks = (it.n + CP - 1u) / CP;
    const uint32_t c0 = s * a.cps;
    const uint32_t c1 = (s + 1u == a.S) ? n_chunks : min(c0 + a.cps, n_chunks);
    const uint32_t mrow = lane & 15u, jg = lane >> 4;
    const bool lo_row = mrow >= 8u;
    const size_t rstride = (size_t)a.n_kvh * ROWB; /* bytes per token */
    const uint32_t rstride32 = a.n_kvh * ROWB;     /* < 2^32: one 32 x 32 -> 64-bit mad per row */
    /* even q8_0 blocks: byte offset of this lane's first dword in the block
     * pair, and the perm selector of its second (identity except group 3) */
    const uint32_t k_eoff = jg < 3u ? 4u + 8u * jg : 28u;
    const float nsel = lo_row ? -1.f : 0.f;
    const uint32_t k_esel = jg == 3u ? 0x05040302u : 0x07060504u;
    const uint8_t *kbase = it.kc + (size_t)kh * ROWB, *vbase = it.vc + (size_t)kh * ROWB;

    /* MODE_STEP: threads 0-63 hold four fp32 of the token's K row, 64-127 of
     * its V row (block (tid >> 3) & 7, part tid & 7); split 0 writes the
     * quantised rows to the caches, and any split whose chunk lists the
     * position uses the same bytes in LDS instead of the fetched row */
    float nx[4] = {0.f, 0.f, 0.f, 0.f};
    const bool step_lane = STEPL && tid < 128u;
    if (step_lane) {
        const float *src = (tid < 64u ? it.knew : it.vnew) + 32u * ((tid >> 3) & 7u) + 4u * (tid & 7u);
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) nx[i] = ldg(src + i);
    }

    if (MODE == MODE_PSTEP && wave == 0) {
        /* wave 0 holds the K row (lane l: dims 4l .. 4l+3): RMSNorm + RoPE
         * at the token's position, through LDS in the shared prep layout */
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) kst[4u * lane + i] = nx[i];
        q4kv_prep_row(kst, kst, it.wnk, 256u, a.n_rot, (int32_t)it.pos_new, a.rope_base, a.eps,
                      lane);
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) nx[i] = kst[4u * lane + i];
    }

    /* rows this lane DMAs (u < 4 always valid, u = 4 only in wave 0) and the
     * s_pos entry of thread tid */
    uint32_t jcur[NLD + 1];
    int32_t raw[NLD + 1], pidx[NLD + 1];
#pragma unroll
    for (uint32_t u = 0; u < NLD; u++) jcur[u] = c0 * CP + ((wave + 4u * u) * 64u + lane) / NCH;
    jcur[NLD] = c0 * CP + (tid & (CP - 1u));
#pragma unroll
    for (uint32_t u = 0; u <= NLD; u++) raw[u] = -1;

    /* Q: one 1 KiB DMA per head row (coalesced). Without the prep (every mode
     * but MODE_PSTEP) and with 16-byte aligned rows, each wave DMAs every row
     * itself (the waves write identical bytes), ahead of the index loads: the
     * wait for those covers its own DMAs, so the wave builds its operands
     * while the first chunk's rows are in flight, with no barrier. Otherwise
     * the waves share the rows and build after the first chunk's barrier. */
    const uint32_t g = mrow & 7u;
    constexpr uint32_t QHS = MODE == MODE_PSTEP ? 512u : 256u; /* q head stride */
    const bool q_own = MODE != MODE_PSTEP && (((uintptr_t)it.q) & 15u) == 0;
    if (q_own) {
        for (uint32_t h = 0; h < gqa; h++)
            dma16(it.q + (size_t)h * QHS + 4u * lane, qraw + h * 260u);
    } else if ((((uintptr_t)it.q) & 15u) == 0) {
        for (uint32_t h = wave; h < gqa; h += 4u)
            dma16(it.q + (size_t)h * QHS + 4u * lane, qraw + h * 260u);
    } else {
        for (uint32_t e = tid; e < gqa * 256u; e += 256u)
            qraw[(e >> 8) * 260u + (e & 255u)] = ldg(it.q + (e >> 8) * QHS + (e & 255u));
    }
    /* the index loads stay behind the Q DMAs, so the wait for them covers
     * those too */
    asm volatile("" ::: "memory");
    if (c0 < c1) pos_issue<NLD + 1, MODE>(it, jcur, raw);
    if (MODE == MODE_PSTEP && s == 0u && it.gate) {
        /* the gate halves of the [q | gate] rows go to the gate buffer the
         * merge reads */
        for (uint32_t e = tid; e < gqa * 64u; e += 256u) {
            const uint32_t h = e >> 6, d = (e & 63u) * 4u;
            *(float4 *)((float *)it.gate + (size_t)h * 256u + d) =
                *(const float4 *)(it.q + (size_t)h * 512u + 256u + d);
        }
    }
    h8_t qa[8];
    /* K operands stay biased by +1152 (the exponent trick's 1024 + 128);
     * qbias[b] = qa[b] x (-1152) is the MFMA accumulator input that removes
     * the bias, computed once per workgroup */
    f4_t qbias[8];
    TRACE(1);
    float m_run[4], l_run[4];
    f4_t acc[4];
#pragma unroll
    for (uint32_t i = 0; i < 4u; i++) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.f;
        acc[i] = (f4_t){0.f, 0.f, 0.f, 0.f};
    }

    /* positions of chunk c (from the index loads in flight) into s_pos[bs],
     * and its K and V rows into buffer bs */
    auto issue_rows = [&](uint32_t c, uint32_t bs) {
        pos_finish<NLD + 1, MODE>(it, jcur, raw, pidx);
        if (tid < CP) s_pos[bs][tid] = pidx[NLD];
        uint8_t *kr = rowbuf[bs], *vr = rowbuf[bs] + CP * ROWB;
        if (al16) {
#pragma unroll
            for (uint32_t u = 0; u < NLD; u++) {
                const uint32_t e0 = (wave + 4u * u) * 64u, e = e0 + lane;
                if (u < 4u || wave == 0) {
                    const uint32_t r = e / NCH, q = e - r * NCH;
                    const uint64_t off = (uint64_t)(uint32_t)(pidx[u] < 0 ? 0 : pidx[u]) * rstride32 + q * 16u;
                    (void)r;
                    dma16(kbase + off, kr + e0 * 16u);
                    dma16(vbase + off, vr + e0 * 16u);
                }
            }
        } else {
            for (uint32_t e = tid; e < CP * (ROWB / 2u); e += 256u) {
                const uint32_t r = e / (ROWB / 2u), q = e - r * (ROWB / 2u);
                const int32_t p = item_pos(it, c * CP + r);
                const size_t off = (size_t)(p < 0 ? 0 : p) * rstride + q * 2u;
                *(uint16_t *)(kr + r * ROWB + q * 2u) = ldg((const uint16_t *)(kbase + off));
                *(uint16_t *)(vr + r * ROWB + q * 2u) = ldg((const uint16_t *)(vbase + off));
            }
        }
    };
    if (DB && c0 < c1) {
        /* the first chunk's rows, then the second chunk's indices */
        if (q_own && MODE == MODE_DENSE) {
            __builtin_amdgcn_s_waitcnt(0);
            build_qa(qraw, g, gqa, jg, nsel, qa, qbias, a.scale_log2, s_qm);
        }
        issue_rows(c0, 0u);
        if (q_own && MODE != MODE_DENSE) build_qa(qraw, g, gqa, jg, nsel, qa, qbias, a.scale_log2, s_qm);
        if (c0 + 1u < c1) {
#pragma unroll
            for (uint32_t u = 0; u <= NLD; u++) jcur[u] += CP;
            pos_issue<NLD + 1, MODE>(it, jcur, raw);
        }
    }

    for (uint32_t c = c0; c < c1; c++) {
        const uint32_t bs = DB ? (c - c0) & 1u : 0u;
        if (!DB) {
            /* one buffer: this chunk's rows now */
            issue_rows(c, 0u);
            if (q_own && c == c0) {
                /* dense items load no indices: wait for the Q DMAs explicitly */
                if (MODE == MODE_DENSE) __builtin_amdgcn_s_waitcnt(0);
                build_qa(qraw, g, gqa, jg, nsel, qa, qbias, a.scale_log2, s_qm);
            }
        }
        uint8_t *const kraw = rowbuf[bs], *const vraw = rowbuf[bs] + CP * ROWB;
        const int32_t *const spos = s_pos[bs];
        TRACE(2);
        /* this chunk's rows (with DB, also the next chunk's indices) have landed */
        __builtin_amdgcn_s_waitcnt(0);
        if (STEPL) {
            /* rows at the appended position take the new token's bytes:
             * wave 0 (thread r owns row r) ballots the matching rows, the
             * mask goes through LDS with the barrier, and the 128 step lanes
             * store their precomputed bytes into just those rows */
            if (wave == 0) {
                const bool mine = pidx[NLD] >= 0 && (uint32_t)pidx[NLD] == it.pos_new;
                const uint64_t mm = __ballot(mine);
                if (lane == 0) {
                    s_subst[0] = (uint32_t)mm;
                    s_subst[1] = (uint32_t)(mm >> 32);
                }
            }
            __syncthreads();
            uint64_t mm = (uint64_t)s_subst[0] | ((uint64_t)s_subst[1] << 32);
            if (mm) {
                if (step_lane) {
                    int nq[4];
                    const float nd = q8_lane_quant(nx[0], nx[1], nx[2], nx[3], nq);
                    uint8_t *base = (tid < 64u ? kraw : vraw) + 34u * ((tid >> 3) & 7u);
                    for (; mm; mm &= mm - 1u)
                        q8_lane_store(base + (uint32_t)__builtin_ctzll(mm) * ROWB, tid & 7u, nd,
                                      nq);
                }
                __syncthreads();
            }
        } else {
            __syncthreads();
        }
        TRACE(3);
        if (!q_own && c == c0) {
            if (MODE == MODE_PSTEP) {
                /* query heads wave, wave + 4: RMSNorm + RoPE in place */
                for (uint32_t h = wave; h < gqa; h += 4u)
                    q4kv_prep_row(qraw + h * 260u, qraw + h * 260u, it.wnq, 256u, a.n_rot,
                                  (int32_t)it.pos_new, a.rope_base, a.eps, lane);
                __syncthreads();
            }
            build_qa(qraw, g, gqa, jg, nsel, qa, qbias, a.scale_log2, s_qm);
            if (DB) __syncthreads(); /* buffer 1 (the Q rows) is refilled below */
        }
        if (c + 1u < c1) {
            if (DB) {
                issue_rows(c + 1u, bs ^ 1u);
                if (c + 2u < c1) {
#pragma unroll
                    for (uint32_t u = 0; u <= NLD; u++) jcur[u] += CP;
                    pos_issue<NLD + 1, MODE>(it, jcur, raw);
                }
            } else {
#pragma unroll
                for (uint32_t u = 0; u <= NLD; u++) jcur[u] += CP;
                pos_issue<NLD + 1, MODE>(it, jcur, raw);
            }
        }
        /* V block scales, 0 for masked positions */
        if (DB) {
#pragma unroll
            for (uint32_t k = 0; k < 2u; k++) {
                const uint32_t e = tid + 256u * k, b = e >> 6, r = e & 63u;
                const float x = ld_f16(vraw + r * ROWB + 34u * b);
                vsc[e] = spos[r] < 0 ? 0.f : x;
            }
        }
        /* ---- scores: wave w, positions 16w .. 16w+15 ---- */
        const uint32_t r = wave * 16u + mrow;
        const uint8_t *krow = kraw + r * ROWB;
        f4_t S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t b = 0; b < 8u; b++) {
            /* k-group jg of block b: odd blocks are dword aligned; even ones
             * take their group-3 tail from the pair's leading dword */
            const uint8_t *pb = krow + 68u * (b >> 1);
            uint32_t w0, w1;
            if (b & 1u) {
                w0 = *(const uint32_t *)(pb + 36u + 8u * jg);
                w1 = *(const uint32_t *)(pb + 40u + 8u * jg);
            } else {
                w0 = *(const uint32_t *)(pb + k_eoff);
                w1 = __builtin_amdgcn_perm(*(const uint32_t *)(pb + k_eoff + 4u),
                                           *(const uint32_t *)pb, k_esel);
            }
            uint32_t r0, r1, r2, r3;
            i8x4_to_h4(w0, r0, r1);
            i8x4_to_h4(w1, r2, r3);
            const h8_t kb = __builtin_bit_cast(h8_t, (u4_t){r0, r1, r2, r3}); /* 1152 + k */
            const float ks = ld_f16(krow + 34u * b);
            const f4_t C = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[b], kb, qbias[b], 0, 0, 0);
            S += ks * C;
        }
        TRACE(4);
        const bool valid = spos[r] >= 0;
        float T[4], cm[4];
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            const float t = pair32_sum(S[i]) * s_qm[(4u * jg + i) & 7u];
            T[i] = valid ? t : -INFINITY;
            cm[i] = T[i];
        }
        row16_max4(cm);
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++)
            if (mrow == 0 && jg < 2u) s_cmax[wave][4u * jg + i] = cm[i];
        TRACE(5);
        __syncthreads();
        TRACE(6);
        float alpha[4], wv[4];
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            const uint32_t h = (4u * jg + i) & 7u;
            const float mn = fmax3v(fmax3v(s_cmax[0][h], s_cmax[1][h], s_cmax[2][h]),
                                    s_cmax[3][h], m_run[i]);
            /* exp2(-inf) = 0 handles masked scores and the first chunk; a
             * still-empty max is shifted to 0 so that -inf - -inf is avoided */
            const float ms = mn == -INFINITY ? 0.f : mn;
            alpha[i] = __builtin_amdgcn_exp2f(m_run[i] - ms);
            m_run[i] = mn;
            const float w = __builtin_amdgcn_exp2f(T[i] - ms);
            if (DB && lane < 32u) sw[(4u * jg + i) * CP + r] = w;
            wv[i] = w;
            const float ps = row16_sum(w);
            if (mrow == 0 && jg < 2u) s_psum[wave][4u * jg + i] = ps;
        }
        if (!DB) {
            /* the P.V A operands of position r, heads 4 (jg & 1) .. + 3 (lanes
             * l and l + 32 hold the same weights): lanes < 32 blocks 0-3,
             * lanes >= 32 blocks 4-7; each product once, split hi / lo */
            const bool rv = spos[r] >= 0;
            const uint32_t b0 = 4u * (lane >> 5), h0 = 4u * (jg & 1u);
            float vsr[4];
#pragma unroll
            for (uint32_t k = 0; k < 4u; k++) vsr[k] = ld_f16(vraw + r * ROWB + 34u * (b0 + k));
#pragma unroll
            for (uint32_t k = 0; k < 4u; k++) {
                const uint32_t b = b0 + k;
                const float vs = rv ? vsr[k] : 0.f;
#pragma unroll
                for (uint32_t i = 0; i < 4u; i++) {
                    const float x = wv[i] * vs;
                    const _Float16 hi = (_Float16)x;
                    _Float16 *d = aop + ((b * 2u) * 8u + h0 + i) * AROW + r;
                    d[0] = hi;
                    d[8u * AROW] = (_Float16)(x - (float)hi);
                }
            }
        }
        TRACE(7);
        __syncthreads();
        TRACE(8);
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            const uint32_t h = (4u * jg + i) & 7u;
            l_run[i] = l_run[i] * alpha[i] + (s_psum[0][h] + s_psum[1][h]) +
                       (s_psum[2][h] + s_psum[3][h]);
#pragma unroll
            for (uint32_t t = 0; t < 4u; t++) acc[t][i] *= alpha[i];
        }
        /* ---- P.V: wave w, dims 64w .. 64w+63 (blocks 2w, 2w+1) ---- */
#pragma unroll
        for (uint32_t kc = 0; kc < 2u; kc++) {
            const uint32_t p0 = 32u * kc + 8u * jg;
            const float *wp = sw + g * CP + p0;
#pragma unroll
            for (uint32_t u = 0; u < 2u; u++) {
                const uint32_t bb = 2u * wave + u;
                const uint8_t *vb = vraw + p0 * ROWB + 34u * bb + 2u + 2u * mrow;
                u4_t r0, r1;
#pragma unroll
                for (uint32_t k = 0; k < 4u; k++) {
                    uint32_t x = (uint32_t)*(const uint16_t *)(vb + (2u * k) * ROWB) |
                                 ((uint32_t)*(const uint16_t *)(vb + (2u * k + 1u) * ROWB) << 16);
                    x ^= 0x80808080u;
                    r0[k] = __builtin_amdgcn_perm(0x64646464u, x, 0x04020400u);
                    r1[k] = __builtin_amdgcn_perm(0x64646464u, x, 0x04030401u);
                }
                h8_t A;
                if (DB) {
                    const float *sp = vsc + bb * CP + p0;
#pragma unroll
                    for (uint32_t i = 0; i < 8u; i++) A[i] = split_sel(wp[i] * sp[i], nsel);
                } else {
                    A = *(const h8_t *)(aop + ((bb * 2u + (lo_row ? 1u : 0u)) * 8u + g) * AROW + p0);
                }
                /* biased V (1152 + v): the bias leaves with A x (-1152), on the
                 * otherwise idle MFMA pipe */
                const h8_t neg = (h8_t)((_Float16)-1152.0f);
                acc[2u * u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, neg, acc[2u * u], 0, 0, 0);
                acc[2u * u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    A, __builtin_bit_cast(h8_t, r0), acc[2u * u], 0, 0, 0);
                acc[2u * u + 1u] =
                    __builtin_amdgcn_mfma_f32_16x16x32_f16(A, neg, acc[2u * u + 1u], 0, 0, 0);
                acc[2u * u + 1u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    A, __builtin_bit_cast(h8_t, r1), acc[2u * u + 1u], 0, 0, 0);
            }
        }
        TRACE(9);
        __syncthreads();
        TRACE(10);
    }

    /* ---- epilogue: hi+lo rows -> LDS [head][col], then 16-byte stores ---- */
    float *so = (float *)rowbuf[0]; /* 8 x 256 floats, free after the last chunk */
    if (c0 >= c1) __syncthreads();
#pragma unroll
    for (uint32_t t = 0; t < 4u; t++)
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            const float tot = acc[t][i] + xor32(acc[t][i]);
            if (lane < 32u) so[(4u * jg + i) * 256u + (wave * 4u + t) * 16u + mrow] = tot;
        }
    if (wave == 0 && mrow == 0 && jg < 2u) {
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            s_ml[0][4u * jg + i] = m_run[i];
            s_ml[1][4u * jg + i] = l_run[i];
        }
    }
    __syncthreads();
    TRACE(11);
    if (a.S == 1u) {
        /* thread -> (head, 8 consecutive dims) */
#pragma unroll
        for (uint32_t k = 0; k < 2u; k++) {
            const uint32_t e = tid + 256u * k, h = e >> 6, d0 = (e & 63u) * 4u;
            if (h < gqa) {
                const float l = s_ml[1][h];
                const float inv = l > 0.f ? 1.f / l : 0.f;
                f4_t o;
#pragma unroll
                for (uint32_t j = 0; j < 4u; j++) {
                    const uint32_t d = d0 + j;
                    float rv = so[h * 256u + q8_col_of_dim(d)] * inv;
                    if (it.gate) {
                        /* MODE_PSTEP: the gate half of the source row (the
                         * copy above is for the merge kernel) */
                        const float gv = MODE == MODE_PSTEP ? ldg(it.q + (size_t)h * 512u + 256u + d)
                                                            : ldg(it.gate + (size_t)h * 256u + d);
                        rv *= 1.f / (1.f + expf(-gv));
                    }
                    o[j] = rv;
                }
                stg((f4_t *)(it.out + (size_t)h * 256u + d0), o);
            }
        }
    } else {
        float *pbase = a.part + (((size_t)item * a.S + s) * gqa_all + h0) * PSTRIDE;
#pragma unroll
        for (uint32_t k = 0; k < 2u; k++) {
            const uint32_t e = tid + 256u * k, h = e >> 6, c4 = (e & 63u) * 4u;
            if (h < gqa) {
                const float *src = so + h * 256u + c4;
                float *dst = pbase + h * PSTRIDE + 2u + c4;
                /* PSTRIDE rows start 8-byte aligned: two 8-byte stores */
                stg((fv2 *)dst, (fv2){src[0], src[1]});
                stg((fv2 *)(dst + 2), (fv2){src[2], src[3]});
            }
        }
        if (tid < gqa) {
            stg((fv2 *)(pbase + tid * PSTRIDE), (fv2){s_ml[0][tid], s_ml[1][tid]});
        }
    }
    /* MODE_STEP: split 0 writes the quantised rows last, so no wait inside
     * the kernel covers these stores (the chunks that list the position
     * took the same bytes in LDS) */
    const bool writer = s == 0u && h0 == 0u && (!APP || item < a.n_kvh);
    if (STEPL && writer && (APP || it.pos_new < it.max_kv) && step_lane) {
        int nq[4];
        const float nd = q8_lane_quant(nx[0], nx[1], nx[2], nx[3], nq);
        uint8_t *row = (uint8_t *)(tid < 64u ? kbase : vbase) + (size_t)it.pos_new * rstride;
        q8_lane_store(row + 34u * ((tid >> 3) & 7u), tid & 7u, nd, nq);
    }
    TRACE(12);
}

/* ------------------------------------------------------------------------
 * Slab kernel: the q8_0 / head_dim 256 decode path for up to 16 query heads
 * per KV head. One wave owns a slab of 32 list entries and computes it end to
 * end (Q.K, softmax, P.V) with no workgroup barrier; the workgroup's waves
 * merge their (m, l, acc) once at the end. Every wave issues its slab's
 * index load and K/V row DMAs first, so all of a workgroup's rows are in
 * flight together; the workgroup builds the Q operands in LDS meanwhile.
 *
 * Per wave, in S^T = K.Q^T form (MFMA v_mfma_f32_16x16x32_f16):
 *  - A = K rows (16 positions x 32 dims of one q8_0 block, int8 -> fp16 via
 *    the exponent trick: 1152 + k), B = Q^T for 16 columns: columns 0-7 the
 *    fp16 part (truncated) of 8 query heads' q, pre-scaled to log2 units,
 *    columns 8-15 the fp16 residual, so a score is column c plus column c + 8.
 *  - The K operands lose the +1152 bias in four packed fp16 subtracts (exact:
 *    k is an integer), so the per-block products sum at the size of q.k for
 *    any |q|; the per-position q8_0 scales: S = sum_b ks[p][b] C_b, started
 *    at -inf for list entries that are padding.
 *  - A lane's C rows (4 positions of each 16-position tile) are exactly the
 *    8 K slots its P.V B operand needs, so the softmax weights never leave
 *    the lane: P.V runs as O^T = V^T.P^T with B = the weights times the V
 *    block scale, split hi (columns 0-7) / lo (8-15), and A = V^T gathered
 *    with 16-bit LDS reads (two adjacent dims feed an even-dim and an odd-dim
 *    tile). The V bias leaves through one MFMA with a -1152 operand per tile.
 * ------------------------------------------------------------------------ */
constexpr uint32_t SLAB = 32;
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

/* K operand of block b, k-group jg from a raw q8_0 row in LDS, biased
 * (1152 + k), in q8_kdim order. */
__device__ static inline h8_t k_operand_biased(const uint8_t *row, uint32_t b, uint32_t jg,
                                               uint32_t k_eoff, uint32_t k_esel) {
    const uint8_t *pb = row + 68u * (b >> 1);
    uint32_t w0, w1;
    if (b & 1u) {
        w0 = *(const uint32_t *)(pb + 36u + 8u * jg);
        w1 = *(const uint32_t *)(pb + 40u + 8u * jg);
    } else {
        w0 = *(const uint32_t *)(pb + k_eoff);
        w1 = __builtin_amdgcn_perm(*(const uint32_t *)(pb + k_eoff + 4u), *(const uint32_t *)pb,
                                   k_esel);
    }
    uint32_t r0, r1, r2, r3;
    i8x4_to_h4(w0, r0, r1);
    i8x4_to_h4(w1, r2, r3);
    return __builtin_bit_cast(h8_t, (u4_t){r0, r1, r2, r3});
}

/* Reductions across the four 16-lane rows (v_permlane16_swap: the lane 16
 * apart within each half; v_permlane32_swap: the lane 32 apart). */
__device__ static inline float sum16(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ static inline float max16(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ static inline float max32(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
/* v + (value of lane c + 8 mod 16 in the same DPP row): hi + lo columns */
__device__ static inline float add_ror8(float v) {
    return v + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
}
/* fp16 halves of a packed word as fp32 (folded into v_fma_mix operands) */
__device__ static inline float h2lo(uint32_t w) { return (float)__builtin_bit_cast(h2_t, w)[0]; }
__device__ static inline float h2hi(uint32_t w) { return (float)__builtin_bit_cast(h2_t, w)[1]; }
/* x, y -> two fp16 by truncation, packed (v_cvt_pkrtz_f16_f32) */
__device__ static inline uint32_t pkrtz(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x, y));
}
/* fp16 hi part of (x, y) (nsel = 0) or the fp16 residual x - hi (nsel = -1),
 * packed; hi by truncation, so hi + lo carries ~21 bits. */
__device__ static inline uint32_t split_pk(float x, float y, float nsel) {
    const uint32_t h = pkrtz(x, y);
    return pkrtz(__builtin_fmaf(nsel, h2lo(h), x), __builtin_fmaf(nsel, h2hi(h), y));
}
/* an fp16 in LDS as fp32 (folded into v_fma_mix operands) */
__device__ static inline float ld_h(const uint8_t *p) {
    return (float)__builtin_bit_cast(_Float16, *(const uint16_t *)p);
}

/* APP: the launch also performs a held append of one token's K/V rows at
 * the device position (as the step modes do with a descriptor's rows). */
/* PIPE (one head group, two or more passes per wave: prefill, batched
 * decode): the K and V rows of pass p + 1 are DMA'd while pass p is
 * computed, K behind the P.V products, V behind the next scores; the waits
 * count the wave's own DMAs (issued from inline assembly so that the compiler
 * adds no wait of its own before the LDS reads). */
template <int MODE, int HG, bool APP = false, bool PIPE = false>
__global__ __launch_bounds__(256, 2) void qsa_slab_k(AttnArgs a) {
    constexpr bool STEPL = IS_STEP(MODE) || APP; /* a token's rows are appended */
    static_assert(!PIPE || (HG == 1 && !APP && MODE != MODE_PSTEP && MODE != MODE_DENSE),
                  "the pipelined passes take one head group and a list or descriptors");
    constexpr uint32_t ROWB = 272, NCH = 17;
    constexpr uint32_t NSLAB = 4u / HG, NE = NSLAB * SLAB; /* slabs, entries per pass */
    constexpr uint32_t RBYTES = 2u * NE * ROWB;           /* K rows | V rows */
    constexpr uint32_t MBYTES = 4u * 16u * 8u * 20u * 4u;  /* merge: [wave][tile][head][20] */
    __shared__ __attribute__((aligned(16))) uint8_t rows[RBYTES > MBYTES ? RBYTES : MBYTES];
    /* Q^T operands [head group][block][k-group][column][8 fp16] */
    __shared__ __attribute__((aligned(16))) uint16_t qB[HG][8][4][16][8];
    /* V block scales of each slab, block-major (fp16 bits, 0 at padding) */
    __shared__ __attribute__((aligned(16))) uint16_t vsT[NSLAB][8][SLAB];
    __shared__ __attribute__((aligned(16))) int32_t s_pos[NE];
    __shared__ float s_m[4][8], s_l[4][8];
    /* per head: the power of two 2^e its q was divided by (scores x 2^e) */
    __shared__ float s_qm[8 * HG];
    /* MODE_PSTEP: the prepared query rows and the prepared new key row */
    constexpr bool PREP = MODE == MODE_PSTEP;
    __shared__ __attribute__((aligned(16))) float qst[PREP ? 8u * HG : 1u][PREP ? 256u : 1u];
    __shared__ __attribute__((aligned(16))) float kst[PREP ? 256u : 1u];

    TRACEW(0);
    /* the wave index in a scalar register: the LDS addresses derived from it
     * are then uniform without a readfirstlane per row DMA */
    const uint32_t tid = threadIdx.x, lane = tid & 63u,
                   wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t slab = wave / HG, hg = wave % HG;
    uint32_t s, item;
    if (!xcd_slot(a, s, item)) return; /* padding of the last group row */
    const uint32_t gqa = a.n_head / a.n_kvh, kh = item % a.n_kvh;
    Item it = resolve_item<MODE>(a, item);
    if (APP) {
        it.knew = a.app_k + (size_t)kh * 256u;
        it.vnew = a.app_v + (size_t)kh * 256u;
        it.pos_new = (uint32_t)ldg(a.app_pos);
    }
    const uint32_t c = lane & 15u, jg = lane >> 4; /* MFMA column / row, k-group */
    const float nsel = c >= 8u ? -1.f : 0.f;
    const size_t rstride = (size_t)a.n_kvh * ROWB;
    const uint32_t rstride32 = a.n_kvh * ROWB; /* < 2^32: one 32 x 32 -> 64-bit mad per row */
    const uint8_t *kbase = it.kc + (size_t)kh * ROWB, *vbase = it.vc + (size_t)kh * ROWB;
    const uint32_t k_eoff = jg < 3u ? 4u + 8u * jg : 28u;
    const uint32_t k_esel = jg == 3u ? 0x05040302u : 0x07060504u;
    uint8_t *const krow = rows + slab * SLAB * ROWB;
    uint8_t *const vrow = rows + NE * ROWB + slab * SLAB * ROWB;
    /* with a prefill band, the list entries from the band on are the band
     * kernel's */
    const bool band = MODE == MODE_INDEXED && a.band_nb != nullptr;
    const uint32_t n = band ? min((uint32_t)ldg(a.band_nb + item), it.n) : it.n;
    const uint32_t j0 = (uint32_t)(((uint64_t)s * n) / a.S);
    const uint32_t j1 = (uint32_t)(((uint64_t)(s + 1u) * n) / a.S);
    /* passes: every wave of the workgroup runs the same number (barriers
     * stay matched); pass k covers entries j0 + k * NE + slab * 32 .. + 31 */
    const uint32_t n_pass = j1 > j0 ? (j1 - j0 + NE - 1u) / NE : 0u;

    int32_t raw = -1;
    {
        const uint32_t e = j0 + slab * SLAB + (lane & 31u);
        if (e < j1) raw = it.list ? ldg(it.list + e) : (int32_t)e;
    }
    /* PIPE: the list word of entry e (entry j0 past the split), one load for
     * every lane; a batch item without a list reads a harmless word, and its
     * position (the entry itself) is taken where the word is used */
    auto list_word = [&](uint32_t e) -> int32_t {
        const uint32_t jj = e < j1 ? e : j0;
        if constexpr (IS_BATCH(MODE))
            return ldg(it.lsrc + (jj & it.lmask));
        else
            return ldg(it.list + jj);
    };
    /* MODE_STEP: every lane holds four fp32 of the token's K row and four of
     * its V row (lane l: block l >> 3, part l & 7); split 0's wave 0 writes
     * the quantised rows to the caches, and a wave whose slab lists the
     * position uses the same bytes in LDS instead of the fetched row. */
    float nk[4] = {0.f, 0.f, 0.f, 0.f}, nv[4] = {0.f, 0.f, 0.f, 0.f};
    if (STEPL) {
        const uint32_t off = 32u * (lane >> 3) + 4u * (lane & 7u);
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            nk[i] = ldg(it.knew + off + i);
            nv[i] = ldg(it.vnew + off + i);
        }
    }
    /* this thread's share of the Q operands: head slot hh of head group k,
     * block b, k-group kg (8 dims in q8_kdim order); loaded here so the loads
     * overlap the DMA issue (with the prep: after it, from the prepared rows) */
    float qx[HG][8];
    const uint32_t t_kg = tid & 3u, t_b = (tid >> 2) & 7u, t_hh = tid >> 5;
    auto load_qx = [&]() {
#pragma unroll
        for (uint32_t k = 0; k < HG; k++) {
            const uint32_t h = 8u * k + t_hh;
            const float *qr = PREP ? &qst[h < gqa ? h : 0u][32u * t_b]
                                   : it.q + (size_t)(h < gqa ? h : 0u) * 256u + 32u * t_b;
#pragma unroll
            for (uint32_t kk = 0; kk < 4u; kk++) {
                const fv2 v = PREP ? *(const fv2 *)(qr + q8_kdim(t_b, t_kg, 2u * kk))
                                   : ldg((const fv2 *)(qr + q8_kdim(t_b, t_kg, 2u * kk)));
                qx[k][2u * kk] = h < gqa ? v[0] * a.scale_log2 : 0.f;
                qx[k][2u * kk + 1u] = h < gqa ? v[1] * a.scale_log2 : 0.f;
            }
        }
    };
    if (!PREP) load_qx();

    /* issue pass p: positions into s_pos, the slab's K/V rows by DMA (32 x
     * 17 sixteen-byte pieces per cache, piece u * 64 + lane, row = piece /
     * 17); returns whether the slab holds any valid position */
    /* PIPE: one cache's rows of the slab (9 DMA instructions per wave) */
    auto rows_dma = [&](const uint8_t *base, uint8_t *dst, int32_t p) {
#pragma unroll
        for (uint32_t u = 0; u < 9u; u++) {
            const uint32_t e = u * 64u + lane;
            const uint32_t r = e / NCH, q = e - r * NCH;
            const int32_t pr = __builtin_amdgcn_ds_bpermute((int)((r & 31u) * 4u), p);
            const uint64_t off = (uint64_t)(uint32_t)(pr < 0 ? 0 : pr) * rstride32 + q * 16u;
            if (u < 8u || lane < 32u) dma16_manual(base + off, dst + u * 1024u);
        }
    };
    auto issue = [&](uint32_t pass, uint32_t &ne, int32_t &pos) -> bool {
        const uint32_t e0 = j0 + pass * NE + slab * SLAB;
        ne = e0 < j1 ? min(SLAB, j1 - e0) : 0u;
        int32_t rp = raw;
        if constexpr (PIPE && IS_BATCH(MODE)) {
            const uint32_t ee = e0 + (lane & 31u);
            rp = (int32_t)(((uint32_t)raw & it.lmask) | ((ee < j1 ? ee : j0) & ~it.lmask));
        }
        pos = (rp >= 0 && (uint32_t)rp < it.max_kv && (lane & 31u) < ne) ? rp : -1;
        const bool any = __ballot(pos >= 0) != 0u;
        if (lane < 32u && hg == 0u) s_pos[slab * SLAB + lane] = pos;
        if (hg == 0u && any) {
            if constexpr (PIPE) {
                rows_dma(kbase, krow, pos);
            } else {
#pragma unroll
                for (uint32_t u = 0; u < 9u; u++) {
                    const uint32_t e = u * 64u + lane;
                    const uint32_t r = e / NCH, q = e - r * NCH;
                    const int32_t pr = __builtin_amdgcn_ds_bpermute((int)((r & 31u) * 4u), pos);
                    const uint64_t off =
                        (uint64_t)(uint32_t)(pr < 0 ? 0 : pr) * rstride32 + q * 16u;
                    if (u < 8u || lane < 32u) {
                        dma16(kbase + off, krow + u * 1024u);
                        dma16(vbase + off, vrow + u * 1024u);
                    }
                }
            }
        }
        return any;
    };
    uint32_t ne = 0;
    int32_t pos = -1;
    bool any = n_pass > 0u ? issue(0u, ne, pos) : false;
    if constexpr (PIPE) {
        /* pass 0's V rows, then pass 1's list entries: one load always (a
         * repeat of entry j0 past the split), so the DMA waits below count
         * exactly */
        if (n_pass > 0u && any) rows_dma(vbase, vrow, pos);
        if (n_pass > 0u) raw = list_word(j0 + NE + slab * SLAB + (lane & 31u));
    }
    TRACEW(1);

    if (PREP) {
        /* RMSNorm + RoPE of the query heads (wave w: heads w, w + 4, ..) and,
         * by wave 0, of the new key row, at the token's position, through the
         * routine the separate prep entry points use; split 0 copies the gate
         * halves of the [q | gate] rows to the gate buffer the merge reads */
        for (uint32_t h = wave; h < gqa; h += 4u)
            q4kv_prep_row(it.q + (size_t)h * 512u, qst[h], it.wnq, 256u, a.n_rot,
                          (int32_t)it.pos_new, a.rope_base, a.eps, lane);
        if (wave == 0u)
            q4kv_prep_row(it.knew, kst, it.wnk, 256u, a.n_rot, (int32_t)it.pos_new, a.rope_base,
                          a.eps, lane);
        if (s == 0u && it.gate) {
            for (uint32_t e = tid; e < gqa * 64u; e += 256u) {
                const uint32_t h = e >> 6, d = (e & 63u) * 4u;
                *(float4 *)((float *)it.gate + (size_t)h * 256u + d) =
                    *(const float4 *)(it.q + (size_t)h * 512u + 256u + d);
            }
        }
        __syncthreads();
        load_qx();
        const uint32_t off = 32u * (lane >> 3) + 4u * (lane & 7u);
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) nk[i] = kst[off + i];
    }

    /* ---- Q^T operands, built once per workgroup ----
     * Each head's q (scale folded in) is first divided by the power of two
     * 2^e that brings its largest magnitude into [0.5, 1) (exact), so its
     * fp16 parts neither overflow nor lose relative precision at any
     * magnitude of q; the head's scores are multiplied back by 2^e. The 32
     * threads of a head slot are lanes 32 (t_hh mod 2) .. + 31 of one wave. */
#pragma unroll
    for (uint32_t k = 0; k < HG; k++) {
        float am = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < 8u; i++) am = fmaxf(am, fabsf(qx[k][i]));
#pragma unroll
        for (uint32_t o = 1; o < 32u; o <<= 1) am = fmaxf(am, __shfl_xor(am, (int)o));
        const int e = (am > 0.f && am <= 3.4e38f) ? __builtin_amdgcn_frexp_expf(am) : 0;
        const float f = __builtin_ldexpf(1.f, -e);
#pragma unroll
        for (uint32_t i = 0; i < 8u; i++) qx[k][i] *= f;
        if ((tid & 31u) == 0u) s_qm[8u * k + t_hh] = __builtin_ldexpf(1.f, e);
    }
#pragma unroll
    for (uint32_t k = 0; k < HG; k++) {
        uint32_t hw[4], lw[4];
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            hw[i] = pkrtz(qx[k][2u * i], qx[k][2u * i + 1u]);
            lw[i] = pkrtz(qx[k][2u * i] - h2lo(hw[i]), qx[k][2u * i + 1u] - h2hi(hw[i]));
        }
        *(u4_t *)&qB[k][t_b][t_kg][t_hh][0] = (u4_t){hw[0], hw[1], hw[2], hw[3]};
        *(u4_t *)&qB[k][t_b][t_kg][t_hh + 8u][0] = (u4_t){lw[0], lw[1], lw[2], lw[3]};
    }
    __syncthreads();
    TRACEW(2);

    float m_run = -INFINITY, l_run = 0.f;
    f4_t acc[16];
#pragma unroll
    for (uint32_t t = 0; t < 16u; t++) acc[t] = (f4_t){0.f, 0.f, 0.f, 0.f};
    const h8_t neg = (h8_t)((_Float16)-1152.0f);
    const uint16_t *const qBw = &qB[hg][0][jg][c][0];
    const float qmul = s_qm[8u * hg + (c & 7u)]; /* this lane's column's head */
    const h8_t k_bias = (h8_t)((_Float16)1152.0f);

    /* pass bodies shared by both loops: the scores and softmax of the slab
     * (P, m_run, l_run, the rescaled acc), then its P.V products */
    float P[8];
    auto scores_softmax = [&](uint32_t pass) {
        TRACEW(4);
        /* ---- scores: two 16-position tiles ---- */
        f4_t S[2];
#pragma unroll
        for (uint32_t t = 0; t < 2u; t++) {
            /* this lane's rows 4 jg .. 4 jg + 3 of tile t: padding rows
             * start at -inf (their K scales are zero and their bytes
             * finite, so they stay there; a pass that is computed holds a
             * valid row, so the maximum is finite) */
            const int4 ps = *(const int4 *)&s_pos[slab * SLAB + 16u * t + 4u * jg];
            S[t] = (f4_t){ps.x < 0 ? -INFINITY : 0.f, ps.y < 0 ? -INFINITY : 0.f,
                          ps.z < 0 ? -INFINITY : 0.f, ps.w < 0 ? -INFINITY : 0.f};
        }
#pragma unroll
        for (uint32_t b = 0; b < 8u; b++) {
            const h8_t qb = *(const h8_t *)(qBw + b * 4u * 16u * 8u);
#pragma unroll
            for (uint32_t t = 0; t < 2u; t++) {
                /* exact k: the products need no bias correction, so their
                 * sum rounds at the size of q.k whatever |q| */
                const h8_t kb =
                    k_operand_biased(krow + (16u * t + c) * ROWB, b, jg, k_eoff, k_esel) -
                    k_bias;
                const f4_t C = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    kb, qb, (f4_t){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                const uint8_t *rs = krow + (16u * t + 4u * jg) * ROWB + 34u * b;
#pragma unroll
                for (uint32_t i = 0; i < 4u; i++)
                    S[t][i] = __builtin_fmaf(ld_h(rs + i * ROWB), C[i], S[t][i]);
            }
        }
        TRACEW(5);
        /* ---- softmax over the slab (base 2; scores already scaled) ---- */
        float T[8];
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            T[i] = add_ror8(S[0][i]) * qmul;
            T[4u + i] = add_ror8(S[1][i]) * qmul;
        }
        float mx = fmax3v(fmax3v(T[0], T[1], T[2]), fmax3v(T[3], T[4], T[5]), fmax2(T[6], T[7]));
        mx = max32(max16(mx));
        const float mn = fmax2(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
        const bool grew = mn > m_run;
        m_run = mn;
        float ls = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < 8u; i++) {
            P[i] = __builtin_amdgcn_exp2f(T[i] - mn);
            ls += P[i];
        }
        l_run = l_run * alpha + ls;
        /* later passes: rescale only when some column's maximum grew
         * (alpha is 1 elsewhere) */
        if (pass > 0u && __ballot(grew) != 0u) {
#pragma unroll
            for (uint32_t t = 0; t < 16u; t++) acc[t] *= alpha;
        }
        TRACEW(6);
    };
    auto pv = [&]() {
        /* ---- P.V over the 8 blocks: tiles 2b (even dims), 2b + 1 (odd) ---- */
        /* this lane's 8 positions: 4 jg .. 4 jg + 3, 16 + 4 jg .. 16 + 4 jg + 3 */
        const uint8_t *vp0 = vrow + (4u * jg) * ROWB, *vp1 = vrow + (16u + 4u * jg) * ROWB;
        /* block b's LDS operands: V scales of the lane's 8 positions, and
         * the 16-bit V reads (dims 2c, 2c + 1) at those positions; block
         * b + 1's are requested before block b is computed */
        struct VOps {
            uint32_t vw[4], x[8];
        };
        auto load_v = [&](uint32_t b, VOps &o) {
            const uint2 va = *(const uint2 *)&vsT[slab][b][4u * jg];
            const uint2 vb = *(const uint2 *)&vsT[slab][b][16u + 4u * jg];
            o.vw[0] = va.x;
            o.vw[1] = va.y;
            o.vw[2] = vb.x;
            o.vw[3] = vb.y;
            const uint8_t *s0 = vp0 + 34u * b + 2u + 2u * c, *s1 = vp1 + 34u * b + 2u + 2u * c;
#pragma unroll
            for (uint32_t i = 0; i < 8u; i++)
                o.x[i] = *(const uint16_t *)((i < 4u ? s0 : s1) + (i & 3u) * ROWB);
        };
        VOps cur, nxt;
        load_v(0u, cur);
#pragma unroll
        for (uint32_t b = 0; b < 8u; b++) {
            if (b + 1u < 8u) load_v(b + 1u, nxt);
            __builtin_amdgcn_sched_barrier(0);
            float u[8];
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                u[2u * i] = __builtin_fmaf(P[2u * i], h2lo(cur.vw[i]), 0.f);
                u[2u * i + 1u] = __builtin_fmaf(P[2u * i + 1u], h2hi(cur.vw[i]), 0.f);
            }
            const u4_t bw = {split_pk(u[0], u[1], nsel), split_pk(u[2], u[3], nsel),
                             split_pk(u[4], u[5], nsel), split_pk(u[6], u[7], nsel)};
            const h8_t B = __builtin_bit_cast(h8_t, bw);
            /* V^T: each 16-bit read holds dims 2c, 2c + 1 of one position;
             * two positions' even (odd) bytes go to one fp16 pair, which
             * the xor turns into 1024 + (b ^ 0x80) = 1152 + b */
            u4_t E, O;
#pragma unroll
            for (uint32_t k = 0; k < 4u; k++) {
                E[k] = __builtin_amdgcn_perm(cur.x[2u * k + 1u], cur.x[2u * k], 0x0C040C00u) ^ 0x64806480u;
                O[k] = __builtin_amdgcn_perm(cur.x[2u * k + 1u], cur.x[2u * k], 0x0C050C01u) ^ 0x64806480u;
            }
            acc[2u * b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(h8_t, E), B, acc[2u * b], 0, 0, 0);
            acc[2u * b + 1u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(h8_t, O), B, acc[2u * b + 1u], 0, 0, 0);
            acc[2u * b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(neg, B, acc[2u * b], 0, 0, 0);
            acc[2u * b + 1u] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(neg, B, acc[2u * b + 1u], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            cur = nxt;
        }
    };
    /* the appended token's quantised row (x: this lane's four values of
     * block lane >> 3) stored into the slab rows of mask hit */
    auto subst_rows = [&](uint64_t hit, uint8_t *rows_base, const float (&x)[4]) {
        int q[4];
        const float d = q8_lane_quant(x[0], x[1], x[2], x[3], q);
        for (uint64_t m = hit; m; m &= m - 1u)
            q8_lane_store(rows_base + (uint32_t)__builtin_ctzll(m) * ROWB + 34u * (lane >> 3),
                          lane & 7u, d, q);
    };
    /* padding rows (never fetched, or fetched from row 0): zero their K block
     * scales */
    auto k_fix = [&]() {
        if (lane < 32u && pos < 0) {
#pragma unroll
            for (uint32_t b = 0; b < 8u; b++) *(uint16_t *)(krow + lane * ROWB + 34u * b) = 0;
        }
    };
    /* the V block scales go block-major to vsT, 0 at padding */
    auto v_fix = [&]() {
        const uint32_t p = lane & 31u;
        const bool valid = s_pos[slab * SLAB + p] >= 0;
#pragma unroll
        for (uint32_t k = 0; k < 4u; k++) {
            const uint32_t b = (lane >> 5) + 2u * k;
            vsT[slab][b][p] = valid ? *(const uint16_t *)(vrow + p * ROWB + 34u * b) : 0;
        }
    };

    if constexpr (PIPE) {
        for (uint32_t pass = 0; pass < n_pass; pass++) {
            /* pass p's K rows have landed when at most its V rows (9 DMA
             * instructions) and the next list load are outstanding */
            /* rows at the appended position take the new token's bytes: K
             * once K has landed, V once V has */
            const uint64_t hit =
                STEPL && any ? __ballot(lane < 32u && pos >= 0 && (uint32_t)pos == it.pos_new)
                             : 0ull;
            if (any) {
                __builtin_amdgcn_s_waitcnt(0x0F7A); /* vmcnt(10) */
                TRACEW(3);
                if (STEPL && hit) subst_rows(hit, krow, nk);
                k_fix();
                scores_softmax(pass);
            }
            __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0): V rows, the list load */
            /* the list word is consumed here on every path, so the compiler
             * has no load of its own pending later (its wait would also
             * drain the next pass's DMA) */
            asm volatile("" ::"v"(raw));
            if (STEPL && hit) subst_rows(hit, vrow, nv);
            if (any) v_fix();
            /* pass p + 1: its K rows behind this pass's P.V, its V rows behind
             * its own scores, then pass p + 2's list entries (one load always) */
            uint32_t ne_n = 0;
            int32_t pos_n = -1;
            const bool any_n = pass + 1u < n_pass ? issue(pass + 1u, ne_n, pos_n) : false;
            if (any) pv();
            if (any_n) rows_dma(vbase, vrow, pos_n);
            raw = list_word(j0 + (pass + 2u) * NE + slab * SLAB + (lane & 31u));
            any = any_n;
            pos = pos_n;
            ne = ne_n;
        }
        __builtin_amdgcn_s_waitcnt(0x0F70); /* the last (unused) list load */
    } else {
        for (uint32_t pass = 0; pass < n_pass; pass++) {
            if (pass > 0u) any = issue(pass, ne, pos);
            /* the next pass's list entries (a wave rarely has more than one) */
            raw = -1;
            {
                const uint32_t e = j0 + (pass + 1u) * NE + slab * SLAB + (lane & 31u);
                if (pass + 1u < n_pass && e < j1) raw = it.list ? ldg(it.list + e) : (int32_t)e;
            }
            __builtin_amdgcn_s_waitcnt(0);
            TRACEW(3);
            if (HG > 1) __syncthreads(); /* the head-group waves share the slab's rows */
            if (hg == 0u && any) {
                if (STEPL) {
                    /* rows at the appended position take the new token's bytes */
                    uint64_t hit = __ballot(lane < 32u && pos >= 0 && (uint32_t)pos == it.pos_new);
                    if (hit) {
                        int q[4], qv[4];
                        const float dk = q8_lane_quant(nk[0], nk[1], nk[2], nk[3], q);
                        const float dv = q8_lane_quant(nv[0], nv[1], nv[2], nv[3], qv);
                        while (hit) {
                            const uint32_t r = __builtin_ctzll(hit);
                            hit &= hit - 1u;
                            q8_lane_store(krow + r * ROWB + 34u * (lane >> 3), lane & 7u, dk, q);
                            q8_lane_store(vrow + r * ROWB + 34u * (lane >> 3), lane & 7u, dv, qv);
                        }
                    }
                }
                k_fix();
                v_fix();
            }
            if (HG > 1) __syncthreads();
            if (any) {
                scores_softmax(pass);
                pv();
            }
            if (HG > 1) __syncthreads(); /* the slab's rows are refilled next pass */
        }
    }
    TRACEW(7);

    /* ---- merge the waves: (m, l) per head, acc to the common max ---- */
    const float lw = pair32_sum(sum16(l_run));
    if (lane < 8u) {
        s_m[wave][lane] = m_run;
        s_l[wave][lane] = lw;
    }
    __syncthreads(); /* every wave is done with the rows: the merge reuses them */
    TRACEW(8);
    float *const mrg = (float *)rows;
#pragma unroll
    for (uint32_t t = 0; t < 16u; t++) {
        f4_t v;
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) v[i] = add_ror8(acc[t][i]);
        if (c < 8u) *(f4_t *)(mrg + ((wave * 16u + t) * 8u + c) * 20u + 4u * jg) = v;
    }
    __syncthreads();
    TRACEW(9);
#pragma unroll
    for (uint32_t k = 0; k < 2u * HG; k++) {
        const uint32_t task = tid + 256u * k;
        const uint32_t thg = task >> 9, hh = (task >> 6) & 7u, t = (task >> 2) & 15u, jq = task & 3u;
        const uint32_t g = 8u * thg + hh;
        if (g >= gqa) continue;
        const uint32_t col = 16u * t + 4u * jq;
        float Mh = -INFINITY;
#pragma unroll
        for (uint32_t w = thg; w < 4u; w += HG) Mh = fmax2(Mh, s_m[w][hh]);
        /* the band's partial of this (item, head), if any (single split) */
        float mb = -INFINITY, lb = 0.f;
        if (band && a.S == 1u) {
            const fv2 ml = ldg((const fv2 *)(a.band_ml + ((size_t)item * gqa + g) * 2u));
            mb = ml[0];
            lb = ml[1];
            if (lb > 0.f) Mh = fmax2(Mh, mb);
        }
        float L = 0.f;
        f4_t v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t w = thg; w < 4u; w += HG) {
            const float mw = s_m[w][hh];
            const float fw = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - Mh);
            L += fw * s_l[w][hh];
            v += fw * *(const f4_t *)(mrg + ((w * 16u + t) * 8u + hh) * 20u + 4u * jq);
        }
        if (lb > 0.f) {
            const float fb = __builtin_amdgcn_exp2f(mb - Mh);
            L += fb * lb;
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++)
                v[i] += fb * ldg(it.out + (size_t)g * 256u + col_dim<Q4KV_Q8>(col + i));
        }
        if (a.S == 1u) {
            const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                const uint32_t d = col_dim<Q4KV_Q8>(col + i);
                float r = v[i] * inv;
                if (it.gate) {
                    /* with the prep: the gate half of the source row (the copy
                     * above is for the merge kernel) */
                    const float gv = PREP ? ldg(it.q + (size_t)g * 512u + 256u + d)
                                          : ldg(it.gate + (size_t)g * 256u + d);
                    r *= 1.f / (1.f + expf(-gv));
                }
                stg(it.out + (size_t)g * 256u + d, r);
            }
        } else {
            float *pb = a.part + ((size_t)item * a.S + s) * gqa * PSTRIDE + (size_t)g * PSTRIDE;
            stg((fv2 *)(pb + 2u + col), (fv2){v[0], v[1]});
            stg((fv2 *)(pb + 4u + col), (fv2){v[2], v[3]});
            if (t == 0u && jq == 0u) stg((fv2 *)pb, (fv2){Mh, L});
        }
    }
    /* MODE_STEP: split 0 writes the quantised rows (K after its prep) last,
     * so no wait inside the kernel covers these stores */
    if (STEPL && s == 0u && wave == 0u && (APP ? item < a.n_kvh : it.pos_new < it.max_kv)) {
        int q[4];
        float d = q8_lane_quant(nk[0], nk[1], nk[2], nk[3], q);
        q8_lane_store((uint8_t *)kbase + (size_t)it.pos_new * rstride + 34u * (lane >> 3),
                      lane & 7u, d, q);
        d = q8_lane_quant(nv[0], nv[1], nv[2], nv[3], q);
        q8_lane_store((uint8_t *)vbase + (size_t)it.pos_new * rstride + 34u * (lane >> 3),
                      lane & 7u, d, q);
    }
    TRACEW(10);
}

/* ------------------------------------------------------------------------
 * f16 cache, hd 256: the slab kernel's structure on plain fp16 MFMA. The
 * cache values are fp16 already, so K rows are the score MFMA's A operand
 * as stored (one 16-byte LDS read each) and V rows need only a 16-bit
 * regroup; there are no block scales. Each wave owns a slab of 16 list
 * entries per pass (4 slabs, or 2 slabs x 2 head groups for 9-16 query
 * heads per KV head):
 *  - scores S^T (16 positions x 8 heads hi | lo) = K (16 x 256) . Q^T over
 *    eight v_mfma_f32_16x16x32_f16, Q split hi/lo (fp16 x 2, ~22 bits);
 *  - the softmax weights P^T come out of the score tile in the lane layout
 *    the P.V B operand needs (split hi/lo in place);
 *  - O^T (dims x heads) += V^T . P^T over sixteen v_mfma_f32_16x16x16_f16:
 *    per 32-dim block, four 32-bit reads (dims 2c, 2c + 1 at the lane's
 *    four positions) regroup into the even-dim and odd-dim operands.
 * Rows are 512 bytes in HBM and 528 in LDS (one 16-byte pad keeps the
 * 16-row operand reads off a single bank group); padding entries are never
 * fetched and their V rows are zeroed in LDS. MODE_STEP appends the token's
 * K/V rows (fp16, round to nearest even, as q4_hip_kv_append_d) from split
 * 0 and patches the LDS rows of any slab that lists the new position. */
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
constexpr uint32_t H16_SL = 16;  /* list entries per slab */

/* Q4KV_SLAB_PIPE=0 keeps the prefill slab passes unpipelined. */
static bool slab_pipe_enabled(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4KV_SLAB_PIPE");
        v = (e && e[0] == '0') ? 0 : 1;
    }
    return v != 0;
}

static bool h16_enabled(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4KV_H16");
        v = (e && e[0] == '0') ? 0 : 1;
    }
    return v != 0;
}

template <int MODE, int HG>
__global__ __launch_bounds__(256, 2) void qsa_h16_k(AttnArgs a) {
    constexpr uint32_t SL = H16_SL, ROWB = 528, NCH = 33;
    constexpr uint32_t NSLAB = 4u / HG, NE = NSLAB * SL;
    constexpr uint32_t RBYTES = 2u * NE * ROWB;
    constexpr uint32_t MBYTES = 4u * 16u * 8u * 20u * 4u; /* merge: [wave][tile][head][20] */
    __shared__ __attribute__((aligned(16))) uint8_t rows[RBYTES > MBYTES ? RBYTES : MBYTES];
    /* Q^T operands [head group][block][k-group][column][8 fp16] */
    __shared__ __attribute__((aligned(16))) uint16_t qB[HG][8][4][16][8];
    __shared__ float s_m[4][8], s_l[4][8];
    /* per head: the power of two 2^e its q was divided by (scores x 2^e) */
    __shared__ float s_qm[8 * HG];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t slab = wave / HG, hg = wave % HG;
    uint32_t s, item;
    if (!xcd_slot(a, s, item)) return; /* padding of the last group row */
    const uint32_t gqa = a.n_head / a.n_kvh, kh = item % a.n_kvh;
    const Item it = resolve_item<MODE>(a, item);
    const uint32_t c = lane & 15u, jg = lane >> 4;
    const float nsel = c >= 8u ? -1.f : 0.f;
    const size_t rstride = (size_t)a.n_kvh * 512u;
    const uint8_t *kbase = it.kc + (size_t)kh * 512u, *vbase = it.vc + (size_t)kh * 512u;
    uint8_t *const krow = rows + slab * SL * ROWB;
    uint8_t *const vrow = rows + NE * ROWB + slab * SL * ROWB;
    const uint32_t n = it.n;
    const uint32_t j0 = (uint32_t)(((uint64_t)s * n) / a.S);
    const uint32_t j1 = (uint32_t)(((uint64_t)(s + 1u) * n) / a.S);
    const uint32_t n_pass = j1 > j0 ? (j1 - j0 + NE - 1u) / NE : 0u;

    /* lane l's list entry: slab position l & 15 */
    int32_t raw = -1;
    {
        const uint32_t e = j0 + slab * SL + c;
        if (e < j1) raw = it.list ? ldg(it.list + e) : (int32_t)e;
    }
    /* MODE_STEP: lane l holds dims 4 l .. 4 l + 3 of the new K and V rows,
     * as fp16 */
    uint32_t nk2[2] = {0u, 0u}, nv2[2] = {0u, 0u};
    if (IS_STEP(MODE)) {
        const f4_t k4 = ldg((const f4_t *)(it.knew + 4u * lane));
        const f4_t v4 = ldg((const f4_t *)(it.vnew + 4u * lane));
        auto h2 = [](float x, float y) {
            return (uint32_t)__half_as_ushort(__float2half_rn(x)) |
                   ((uint32_t)__half_as_ushort(__float2half_rn(y)) << 16);
        };
        nk2[0] = h2(k4[0], k4[1]);
        nk2[1] = h2(k4[2], k4[3]);
        nv2[0] = h2(v4[0], v4[1]);
        nv2[1] = h2(v4[2], v4[3]);
    }
    /* this thread's share of the Q operands: head slot hh of head group k,
     * block b, k-group kg (dims 32 b + 8 kg .. + 7) */
    float qx[HG][8];
    const uint32_t t_kg = tid & 3u, t_b = (tid >> 2) & 7u, t_hh = tid >> 5;
#pragma unroll
    for (uint32_t k = 0; k < HG; k++) {
        const uint32_t h = 8u * k + t_hh;
        const float *qr = it.q + (size_t)(h < gqa ? h : 0u) * 256u + 32u * t_b + 8u * t_kg;
        const f4_t x0 = ldg((const f4_t *)qr), x1 = ldg((const f4_t *)(qr + 4));
        const float sc = h < gqa ? a.scale_log2 : 0.f;
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            qx[k][i] = x0[i] * sc;
            qx[k][4u + i] = x1[i] * sc;
        }
    }

    /* issue pass p: the slab's K/V rows by DMA (16 x 33 sixteen-byte slots
     * per cache, slot u * 64 + lane, row = slot / 33; slot 32 of a row is
     * its pad). Padding entries are not fetched. Returns whether the slab
     * holds any valid position. */
    auto issue = [&](uint32_t pass, int32_t &pos) -> bool {
        const uint32_t e0 = j0 + pass * NE + slab * SL;
        const uint32_t ne = e0 < j1 ? min(SL, j1 - e0) : 0u;
        pos = (raw >= 0 && (uint32_t)raw < it.max_kv && c < ne) ? raw : -1;
        const bool any = __ballot(pos >= 0) != 0u;
        if (hg == 0u && any) {
#pragma unroll
            for (uint32_t u = 0; u < 9u; u++) {
                const uint32_t e = u * 64u + lane;
                const uint32_t r = e / NCH, q = e - r * NCH;
                const int32_t pr = __builtin_amdgcn_ds_bpermute((int)((r & 15u) * 4u), pos);
                const size_t off = (size_t)(pr < 0 ? 0 : pr) * rstride + q * 16u;
                if (r < SL && q < 32u && pr >= 0) {
                    dma16(kbase + off, krow + u * 1024u);
                    dma16(vbase + off, vrow + u * 1024u);
                }
            }
        }
        return any;
    };
    int32_t pos = -1;
    bool any = n_pass > 0u ? issue(0u, pos) : false;

    /* ---- Q^T operands, built once per workgroup ----
     * Each head's q (scale folded in) is first divided by the power of two
     * 2^e that brings its largest magnitude into [0.5, 1) (exact), so its
     * fp16 parts neither overflow nor lose relative precision at any
     * magnitude of q; the head's scores are multiplied back by 2^e. The 32
     * threads of a head slot are lanes 32 (t_hh mod 2) .. + 31 of one wave. */
#pragma unroll
    for (uint32_t k = 0; k < HG; k++) {
        float am = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < 8u; i++) am = fmaxf(am, fabsf(qx[k][i]));
#pragma unroll
        for (uint32_t o = 1; o < 32u; o <<= 1) am = fmaxf(am, __shfl_xor(am, (int)o));
        const int e = (am > 0.f && am <= 3.4e38f) ? __builtin_amdgcn_frexp_expf(am) : 0;
        const float f = __builtin_ldexpf(1.f, -e);
#pragma unroll
        for (uint32_t i = 0; i < 8u; i++) qx[k][i] *= f;
        if ((tid & 31u) == 0u) s_qm[8u * k + t_hh] = __builtin_ldexpf(1.f, e);
    }
#pragma unroll
    for (uint32_t k = 0; k < HG; k++) {
        uint32_t hw[4], lw[4];
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            hw[i] = pkrtz(qx[k][2u * i], qx[k][2u * i + 1u]);
            lw[i] = pkrtz(qx[k][2u * i] - h2lo(hw[i]), qx[k][2u * i + 1u] - h2hi(hw[i]));
        }
        *(u4_t *)&qB[k][t_b][t_kg][t_hh][0] = (u4_t){hw[0], hw[1], hw[2], hw[3]};
        *(u4_t *)&qB[k][t_b][t_kg][t_hh + 8u][0] = (u4_t){lw[0], lw[1], lw[2], lw[3]};
    }
    __syncthreads();

    float m_run = -INFINITY, l_run = 0.f;
    f4_t acc[16];
#pragma unroll
    for (uint32_t t = 0; t < 16u; t++) acc[t] = (f4_t){0.f, 0.f, 0.f, 0.f};
    const uint16_t *const qBw = &qB[hg][0][jg][c][0];
    const float qmul = s_qm[8u * hg + (c & 7u)]; /* this lane's column's head */

    for (uint32_t pass = 0; pass < n_pass; pass++) {
        if (pass > 0u) any = issue(pass, pos);
        raw = -1;
        {
            const uint32_t e = j0 + (pass + 1u) * NE + slab * SL + c;
            if (pass + 1u < n_pass && e < j1) raw = it.list ? ldg(it.list + e) : (int32_t)e;
        }
        /* valid positions of the slab (bit p: entry p) */
        const uint32_t vmask = (uint32_t)__ballot(pos >= 0) & 0xFFFFu;
        __builtin_amdgcn_s_waitcnt(0);
        if (HG > 1) __syncthreads(); /* the head-group waves share the slab's rows */
        if (hg == 0u && any) {
            /* padding entries: zero V rows (their weights are 0; stale LDS
             * must not turn that into NaN) */
            uint32_t padm = ~vmask & 0xFFFFu;
            while (padm) {
                const uint32_t r = (uint32_t)__builtin_ctz(padm);
                padm &= padm - 1u;
                if (lane < 32u) *(u4_t *)(vrow + r * ROWB + 16u * lane) = (u4_t){0u, 0u, 0u, 0u};
            }
            if (IS_STEP(MODE)) {
                /* rows at the appended position take the new token's bytes */
                uint32_t hit = (uint32_t)__ballot(lane < 16u && pos >= 0 &&
                                                  (uint32_t)pos == it.pos_new);
                while (hit) {
                    const uint32_t r = (uint32_t)__builtin_ctz(hit);
                    hit &= hit - 1u;
                    *(u2_t *)(krow + r * ROWB + 8u * lane) = (u2_t){nk2[0], nk2[1]};
                    *(u2_t *)(vrow + r * ROWB + 8u * lane) = (u2_t){nv2[0], nv2[1]};
                }
            }
        }
        if (HG > 1) __syncthreads();
        if (any) {
            /* ---- scores: S^T (positions x [heads hi | heads lo]) ---- */
            f4_t S = {0.f, 0.f, 0.f, 0.f};
            const uint8_t *kr = krow + c * ROWB + 16u * jg;
#pragma unroll
            for (uint32_t b = 0; b < 8u; b++) {
                const h8_t A = *(const h8_t *)(kr + 64u * b);
                const h8_t B = *(const h8_t *)(qBw + b * 4u * 16u * 8u);
                S = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, S, 0, 0, 0);
            }
            /* ---- softmax over the slab (base 2; scores already scaled) ---- */
            float T[4];
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                const float x = add_ror8(S[i]) * qmul;
                T[i] = (vmask >> (4u * jg + i)) & 1u ? x : -INFINITY;
            }
            float mx = fmax2(fmax2(T[0], T[1]), fmax2(T[2], T[3]));
            mx = max32(max16(mx));
            const float mn = fmax2(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
            const bool grew = mn > m_run;
            m_run = mn;
            float P[4];
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) P[i] = __builtin_amdgcn_exp2f(T[i] - mn);
            l_run = l_run * alpha + ((P[0] + P[1]) + (P[2] + P[3]));
            if (pass > 0u && __ballot(grew) != 0u) {
#pragma unroll
                for (uint32_t t = 0; t < 16u; t++) acc[t] *= alpha;
            }
            /* P^T operand: the lane's four positions, hi (columns < 8) or
             * lo (columns >= 8) */
            const h4_t Bp = __builtin_bit_cast(
                h4_t, (u2_t){split_pk(P[0], P[1], nsel), split_pk(P[2], P[3], nsel)});
            /* ---- P.V: per 32-dim block b, tiles 2b (even dims), 2b + 1 (odd) ---- */
            const uint8_t *vr = vrow + (4u * jg) * ROWB + 4u * c;
#pragma unroll
            for (uint32_t b = 0; b < 8u; b++) {
                uint32_t x[4];
#pragma unroll
                for (uint32_t i = 0; i < 4u; i++) x[i] = *(const uint32_t *)(vr + i * ROWB + 64u * b);
                const u2_t E = {__builtin_amdgcn_perm(x[1], x[0], 0x05040100u),
                                 __builtin_amdgcn_perm(x[3], x[2], 0x05040100u)};
                const u2_t O = {__builtin_amdgcn_perm(x[1], x[0], 0x07060302u),
                                 __builtin_amdgcn_perm(x[3], x[2], 0x07060302u)};
                acc[2u * b] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                    __builtin_bit_cast(h4_t, E), Bp, acc[2u * b], 0, 0, 0);
                acc[2u * b + 1u] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                    __builtin_bit_cast(h4_t, O), Bp, acc[2u * b + 1u], 0, 0, 0);
            }
        }
        if (HG > 1) __syncthreads(); /* the slab's rows are refilled next pass */
    }

    /* ---- merge the waves: (m, l) per head, acc to the common max ---- */
    const float lw = pair32_sum(sum16(l_run));
    if (lane < 8u) {
        s_m[wave][lane] = m_run;
        s_l[wave][lane] = lw;
    }
    __syncthreads(); /* every wave is done with the rows: the merge reuses them */
    float *const mrg = (float *)rows;
#pragma unroll
    for (uint32_t t = 0; t < 16u; t++) {
        f4_t v;
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) v[i] = add_ror8(acc[t][i]);
        if (c < 8u) *(f4_t *)(mrg + ((wave * 16u + t) * 8u + c) * 20u + 4u * jg) = v;
    }
    __syncthreads();
    /* output column 16 t + r of a head is dim 32 (t >> 1) + 2 r + (t & 1):
     * the q8_0 kernels' column order, so qsa_comb_k<Q4KV_Q8> merges splits */
#pragma unroll
    for (uint32_t k = 0; k < 2u * HG; k++) {
        const uint32_t task = tid + 256u * k;
        const uint32_t thg = task >> 9, hh = (task >> 6) & 7u, t = (task >> 2) & 15u, jq = task & 3u;
        const uint32_t g = 8u * thg + hh;
        if (g >= gqa) continue;
        const uint32_t col = 16u * t + 4u * jq;
        float Mh = -INFINITY;
#pragma unroll
        for (uint32_t w = thg; w < 4u; w += HG) Mh = fmax2(Mh, s_m[w][hh]);
        float L = 0.f;
        f4_t v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t w = thg; w < 4u; w += HG) {
            const float mw = s_m[w][hh];
            const float fw = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - Mh);
            L += fw * s_l[w][hh];
            v += fw * *(const f4_t *)(mrg + ((w * 16u + t) * 8u + hh) * 20u + 4u * jq);
        }
        if (a.S == 1u) {
            const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                const uint32_t d = col_dim<Q4KV_Q8>(col + i);
                float r = v[i] * inv;
                if (it.gate) r *= 1.f / (1.f + expf(-ldg(it.gate + (size_t)g * 256u + d)));
                stg(it.out + (size_t)g * 256u + d, r);
            }
        } else {
            float *pb = a.part + ((size_t)item * a.S + s) * gqa * PSTRIDE + (size_t)g * PSTRIDE;
            stg((fv2 *)(pb + 2u + col), (fv2){v[0], v[1]});
            stg((fv2 *)(pb + 4u + col), (fv2){v[2], v[3]});
            if (t == 0u && jq == 0u) stg((fv2 *)pb, (fv2){Mh, L});
        }
    }
    /* MODE_STEP: split 0 writes the new rows last (no wait covers them) */
    if (IS_STEP(MODE) && s == 0u && wave == 0u && it.pos_new < it.max_kv) {
        stg((u2_t *)(kbase + (size_t)it.pos_new * rstride + 8u * lane), (u2_t){nk2[0], nk2[1]});
        stg((u2_t *)(vbase + (size_t)it.pos_new * rstride + 8u * lane), (u2_t){nv2[0], nv2[1]});
    }
}

/* ------------------------------------------------------------------------
 * f32 cache, hd 256: rows of 1 KB, contracted on fp32 MFMA
 * (v_mfma_f32_16x16x4_f32: exact fp32 products, no hi/lo split). A 64-entry
 * pass of K and V rows would need 128 KB of LDS, so each wave loads its 16
 * entries' rows straight into registers (16 + 16 sixteen-byte loads per
 * lane, all issued before the first is used) and the four waves never
 * synchronise inside the loop:
 *  - scores S^T (16 positions x 16 heads) = K . Q^T over 64 MFMAs; lane
 *    (c, g) holds K[position c][16 m + 4 g .. + 3] for m < 16, and the
 *    matching Q^T operands come from LDS;
 *  - the softmax weights are the P.V B operand in place (lane (c, g),
 *    MFMA i: position 4 g + i, head c);
 *  - O^T (16 tiles of 16 dims x 16 heads) += V^T . P^T over 64 MFMAs; lane
 *    (c, g) holds V[position 4 g + i][64 t' + 4 c .. + 3] for i, t' < 4, so
 *    tile 4 t' + u has dims 64 t' + 4 c + u on its rows.
 * Padding entries load nothing (zero rows, weight 0). MODE_STEP appends the
 * token's rows (fp32, as stored) from split 0 and substitutes them in the
 * registers of any lane whose entry is the new position. */
static bool f32w_enabled(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4KV_F32W");
        v = (e && e[0] == '0') ? 0 : 1;
    }
    return v != 0;
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void qsa_f32w_k(AttnArgs a) {
    constexpr uint32_t SL = 16u, NE = 64u;
    /* the Q^T operands [m][g][head][4] during the loop; the waves' output
     * tiles [wave][tile][lane][4] for the merge */
    __shared__ __attribute__((aligned(16))) float lds[4u * 16u * 64u * 4u];
    __shared__ float s_m[4][16], s_l[4][16];
    float(*qT)[4][16][4] = (float(*)[4][16][4])lds;

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    uint32_t s, item;
    if (!xcd_slot(a, s, item)) return; /* padding of the last group row */
    const uint32_t gqa = a.n_head / a.n_kvh, kh = item % a.n_kvh;
    const Item it = resolve_item<MODE>(a, item);
    const uint32_t c = lane & 15u, jg = lane >> 4;
    const size_t rstride = (size_t)a.n_kvh * 1024u;
    const uint8_t *kbase = it.kc + (size_t)kh * 1024u, *vbase = it.vc + (size_t)kh * 1024u;
    const uint32_t n = it.n;
    const uint32_t j0 = (uint32_t)(((uint64_t)s * n) / a.S);
    const uint32_t j1 = (uint32_t)(((uint64_t)(s + 1u) * n) / a.S);
    const uint32_t n_pass = j1 > j0 ? (j1 - j0 + NE - 1u) / NE : 0u;

    /* MODE_STEP: split 0's wave 0 holds the new rows (lane l: floats
     * 4 l .. 4 l + 3) and writes them last, so no wait covers the stores */
    const bool step_wr = IS_STEP(MODE) && s == 0u && wave == 0u && it.pos_new < it.max_kv;
    f4_t nk4 = {0.f, 0.f, 0.f, 0.f}, nv4 = nk4;
    if (step_wr) {
        nk4 = ldg((const f4_t *)it.knew + lane);
        nv4 = ldg((const f4_t *)it.vnew + lane);
    }
    for (uint32_t e = tid; e < 16u * 256u; e += 256u) {
        const uint32_t h = e >> 8, d = e & 255u;
        qT[d >> 4][(d >> 2) & 3u][h][d & 3u] =
            h < gqa ? ldg(it.q + (size_t)h * 256u + d) * a.scale_log2 : 0.f;
    }
    __syncthreads();

    float m_run = -INFINITY, l_run = 0.f;
    f4_t acc[16];
#pragma unroll
    for (uint32_t t = 0; t < 16u; t++) acc[t] = (f4_t){0.f, 0.f, 0.f, 0.f};
    const f4_t z4 = {0.f, 0.f, 0.f, 0.f};

    for (uint32_t pass = 0; pass < n_pass; pass++) {
        /* lane l's entry: slab position l & 15 */
        const uint32_t e = j0 + pass * NE + wave * SL + c;
        int32_t pk = -1;
        if (e < j1) pk = it.list ? ldg(it.list + e) : (int32_t)e;
        if (pk >= 0 && (uint32_t)pk >= it.max_kv) pk = -1;
        const uint32_t vmask = (uint32_t)__ballot(pk >= 0) & 0xFFFFu;
        if (!vmask) continue; /* wave-uniform */
        int32_t pv[4];
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) pv[i] = __shfl(pk, (int)(4u * jg + i));
        /* K: position c, dims 16 m + 4 jg .. + 3; V: positions 4 jg + i,
         * dims 64 t + 4 c .. + 3 */
        f4_t kr[16], vr[4][4];
        const f4_t *kp = (const f4_t *)(kbase + (size_t)(pk < 0 ? 0 : pk) * rstride) + jg;
#pragma unroll
        for (uint32_t m = 0; m < 16u; m++) kr[m] = pk >= 0 ? ldg(kp + 4u * m) : z4;
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) {
            const f4_t *vp = (const f4_t *)(vbase + (size_t)(pv[i] < 0 ? 0 : pv[i]) * rstride) + c;
#pragma unroll
            for (uint32_t t = 0; t < 4u; t++) vr[i][t] = pv[i] >= 0 ? ldg(vp + 16u * t) : z4;
        }
        if (IS_STEP(MODE)) {
            if (pk >= 0 && (uint32_t)pk == it.pos_new) {
#pragma unroll
                for (uint32_t m = 0; m < 16u; m++) kr[m] = ldg((const f4_t *)it.knew + 4u * m + jg);
            }
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++)
                if (pv[i] >= 0 && (uint32_t)pv[i] == it.pos_new) {
#pragma unroll
                    for (uint32_t t = 0; t < 4u; t++) vr[i][t] = ldg((const f4_t *)it.vnew + 16u * t + c);
                }
        }
        /* ---- scores ---- */
        f4_t S = z4;
#pragma unroll
        for (uint32_t m = 0; m < 16u; m++) {
            const f4_t qb = *(const f4_t *)&qT[m][jg][c][0];
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++)
                S = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[m][i], qb[i], S, 0, 0, 0);
        }
        /* ---- softmax (base 2; scores already scaled) ---- */
        float T[4];
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) T[i] = (vmask >> (4u * jg + i)) & 1u ? S[i] : -INFINITY;
        float mx = fmax2(fmax2(T[0], T[1]), fmax2(T[2], T[3]));
        mx = max32(max16(mx));
        const float mn = fmax2(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - mn);
        const bool grew = mn > m_run;
        m_run = mn;
        float P[4];
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) P[i] = __builtin_amdgcn_exp2f(T[i] - mn);
        l_run = l_run * alpha + ((P[0] + P[1]) + (P[2] + P[3]));
        if (__ballot(grew) != 0u) {
#pragma unroll
            for (uint32_t t = 0; t < 16u; t++) acc[t] *= alpha;
        }
        /* ---- P.V ---- */
#pragma unroll
        for (uint32_t t = 0; t < 4u; t++)
#pragma unroll
            for (uint32_t u = 0; u < 4u; u++)
#pragma unroll
                for (uint32_t i = 0; i < 4u; i++)
                    acc[4u * t + u] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[i][t][u], P[i],
                                                                          acc[4u * t + u], 0, 0, 0);
    }

    /* ---- merge the waves ---- */
    const float lw = pair32_sum(sum16(l_run));
    if (lane < 16u) {
        s_m[wave][lane] = m_run;
        s_l[wave][lane] = lw;
    }
    __syncthreads(); /* every wave is done with the Q^T operands */
    f4_t *const mrg = (f4_t *)lds;
#pragma unroll
    for (uint32_t t = 0; t < 16u; t++) mrg[(wave * 16u + t) * 64u + lane] = acc[t];
    __syncthreads();
    const bool fin = a.S == 1u;
    float *pbase = fin ? nullptr : a.part + ((size_t)item * a.S + s) * gqa * PSTRIDE;
    for (uint32_t e = tid; e < 16u * 256u; e += 256u) {
        const uint32_t h = e >> 8, d = e & 255u;
        if (h >= gqa) break; /* h grows with e */
        /* dim d = 64 t + 4 (4 g + r) + u: tile 4 t + u, lane 16 g + h, row r */
        const uint32_t t = d >> 6, g = (d >> 4) & 3u, r = (d >> 2) & 3u, u = d & 3u;
        const uint32_t slot = (4u * t + u) * 64u + 16u * g + h;
        float M = -INFINITY;
#pragma unroll
        for (uint32_t w = 0; w < 4u; w++) M = fmax2(M, s_m[w][h]);
        float L = 0.f, x = 0.f;
#pragma unroll
        for (uint32_t w = 0; w < 4u; w++) {
            const float mw = s_m[w][h];
            const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
            L += f * s_l[w][h];
            x += f * mrg[w * 16u * 64u + slot][r];
        }
        if (fin) {
            float rv = L > 0.f ? x / L : 0.f;
            if (it.gate) rv *= 1.f / (1.f + expf(-ldg(it.gate + (size_t)h * 256u + d)));
            stg(it.out + (size_t)h * 256u + d, rv);
        } else {
            stg(pbase + h * PSTRIDE + 2u + d, x);
            if (d == 0u) stg((fv2 *)(pbase + h * PSTRIDE), (fv2){M, L});
        }
    }
    if (step_wr) {
        stg((f4_t *)(kbase + (size_t)it.pos_new * rstride) + lane, nk4);
        stg((f4_t *)(vbase + (size_t)it.pos_new * rstride) + lane, nv4);
    }
}

/* ------------------------------------------------------------------------
 * Prefill band kernel: the recent window that consecutive prefill tokens'
 * lists share, as dense MFMA tiles. A token's band is the longest run of
 * consecutive positions that ends its list (the causal recent window); the
 * slab kernel then attends only the list entries before it. One workgroup
 * takes BAND_TOK consecutive tokens of one KV head (two per wave): the union
 * of their bands (at most BAND_SPAN positions) streams through LDS 32
 * positions per pass (two passes in flight), where the workgroup dequantises
 * the K and V rows once into fp16 hi + lo parts (k * scale, exact to
 * ~2^-22), shared by every token and head of the tile. Each wave then runs,
 * for its two tokens with every LDS operand read once for both,
 *   S^T = K' Q^T   (A = K' hi / lo rows, B = a token's Q^T, columns 0-7 the
 *                   fp16 part of 8 heads' q, 8-15 the residual),
 *   softmax over the token's band positions only (the rest -inf),
 *   O^T += V'^T P^T (A = V'^T hi / lo, B = the weights split hi / lo),
 * with no per-position scale work on the VALU. The result is the (m, l,
 * unnormalised acc) partial of each (token, head), handed to the slab
 * kernel's final merge.
 * ------------------------------------------------------------------------ */
constexpr uint32_t BAND_TPW = 2;                /* tokens per wave */
constexpr uint32_t BAND_WAVES = 8;              /* waves per workgroup */
constexpr uint32_t BAND_TOK = BAND_WAVES * BAND_TPW; /* tokens per workgroup */
constexpr uint32_t BAND_MIN = 64;               /* shortest run worth a band */
constexpr uint32_t BAND_SPAN = 1024;            /* widest union of a workgroup's bands */
constexpr uint32_t BP = 32;                     /* positions per pass */

/* workgroup barrier that waits for this wave's LDS accesses only (the
 * __syncthreads fence also drains every outstanding global load, including
 * the next pass's DMA) */
__device__ static inline void barrier_lds(void) {
    __builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) */
    __builtin_amdgcn_s_barrier();
}

/* The band of one token's list (wave-uniform): the run of consecutive
 * positions that ends it (after any padding), at least BAND_MIN long.
 * Returns the list index where the run starts (width if there is none) and
 * the run's first and last positions (ps > pe if none). */
__device__ static inline uint32_t band_of(const int32_t *list, uint32_t width, uint32_t max_kv,
                                          uint32_t lane, int32_t &ps, int32_t &pe) {
    ps = 1;
    pe = 0;
    int32_t e = -1, vend = 0;
    for (int32_t base = (int32_t)width - 64;; base -= 64) {
        const int32_t j = base + (int32_t)lane;
        const int32_t v = j >= 0 ? ldg(list + j) : -1;
        const bool ok = j >= 0 && v >= 0 && (uint32_t)v < max_kv;
        const uint64_t bal = __ballot(ok);
        if (bal) {
            const uint32_t hi = 63u - (uint32_t)__builtin_clzll(bal);
            e = base + (int32_t)hi;
            vend = __shfl(v, (int)hi);
            break;
        }
        if (base <= 0) break;
    }
    if (e < 0) return width;
    uint32_t run = 0;
    for (uint32_t w0 = 0; w0 < BAND_SPAN; w0 += 64u) {
        const int32_t j = e - (int32_t)(w0 + lane);
        const bool ok = j >= 0 && ldg(list + j) == vend - (int32_t)(w0 + lane);
        const uint64_t bad = __ballot(!ok);
        if (bad) {
            run = w0 + (uint32_t)__builtin_ctzll(bad);
            break;
        }
        run = w0 + 64u;
    }
    /* a run stops at position 0 (a -1 entry before it equals vend - run too) */
    if ((int64_t)run > (int64_t)vend + 1) run = (uint32_t)vend + 1u;
    if (run > BAND_SPAN) run = BAND_SPAN;
    if (run < BAND_MIN) return width;
    ps = vend - (int32_t)run + 1;
    pe = vend;
    return (uint32_t)(e - (int32_t)run + 1);
}

/* band_of with every load issued at once: the last BAND_NJ x 64 entries of
 * the list (one load per lane each) cover the run whenever the list's last
 * valid entry is among its final 64 (no more than 63 trailing padding or
 * out-of-range entries); otherwise the chained band_of runs. Same result. */
constexpr uint32_t BAND_NJ = BAND_SPAN / 64u + 1u;
__device__ static inline uint32_t band_of_tail(const int32_t *list, uint32_t width,
                                               uint32_t max_kv, uint32_t lane, int32_t &ps,
                                               int32_t &pe) {
    int32_t v[BAND_NJ];
#pragma unroll
    for (uint32_t i = 0; i < BAND_NJ; i++) {
        const uint32_t j = 64u * i + lane; /* entry width - 1 - j */
        v[i] = j < width ? ldg(list + (width - 1u - j)) : -1;
    }
    /* the last valid entry: the smallest j with a valid position */
    const uint64_t okb = __ballot(v[0] >= 0 && (uint32_t)v[0] < max_kv);
    if (!okb) return band_of(list, width, max_kv, lane, ps, pe);
    const uint32_t jf = (uint32_t)__builtin_ctzll(okb);
    const int32_t vend = __shfl(v[0], (int)jf);
    /* the run: entry width - 1 - j holds vend - (j - jf) for j = jf, jf + 1, .. */
    uint32_t run = BAND_NJ * 64u - jf; /* every loaded entry from jf on matches */
#pragma unroll
    for (uint32_t i = 0; i < BAND_NJ; i++) {
        const uint32_t j = 64u * i + lane;
        const bool bad = j >= jf && (j >= width || v[i] != vend - (int32_t)(j - jf));
        const uint64_t bb = __ballot(bad);
        if (bb) {
            run = min(run, 64u * i + (uint32_t)__builtin_ctzll(bb) - jf);
            break;
        }
    }
    ps = 1;
    pe = 0;
    /* a run stops at position 0 (a -1 entry before it equals vend - run too) */
    if ((int64_t)run > (int64_t)vend + 1) run = (uint32_t)vend + 1u;
    if (run > BAND_SPAN) run = BAND_SPAN;
    if (run < BAND_MIN) return width;
    ps = vend - (int32_t)run + 1;
    pe = vend;
    return width - 1u - jf - run + 1u;
}

__global__ __launch_bounds__(512, 2) void qsa_band_k(AttnArgs a) {
    constexpr uint32_t ROWB = 272, NCH = 17, KPAD = 264, VPAD = 40, TW = BAND_TPW;
    /* K rows | V rows of even and odd passes: two passes in flight (two
     * objects, so the LDS-DMA wait before reading one buffer does not cover
     * the other's DMA) */
    __shared__ __attribute__((aligned(16))) uint8_t rawA[2 * BP * ROWB];
    __shared__ __attribute__((aligned(16))) uint8_t rawB[2 * BP * ROWB];
    /* K' [hi/lo][position][dim] and V'^T [hi/lo][dim][slot] (fp16); V slot
     * 8 g + i holds position 4 g + i (i < 4) or 16 + 4 g + i - 4, the
     * positions a lane of k-group g holds in the score tiles */
    __shared__ __attribute__((aligned(16))) _Float16 kp[2][BP][KPAD];
    __shared__ __attribute__((aligned(16))) _Float16 vt[2][256][VPAD];
    __shared__ int32_t s_ps[BAND_TOK], s_pe[BAND_TOK];

    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t kh = blockIdx.y, t0 = blockIdx.x * BAND_TOK + wave * TW;
    const uint32_t n_tok = a.kv_base; /* tokens of the launch (set by the host) */
    const uint32_t gqa = a.n_head / a.n_kvh, width = a.width;
    const uint32_t c = lane & 15u, jg = lane >> 4;
    const float nsel = c >= 8u ? -1.f : 0.f;
    const size_t rstride = (size_t)a.n_kvh * ROWB;
    const uint8_t *kbase = a.kc + (size_t)kh * ROWB, *vbase = a.vc + (size_t)kh * ROWB;

    TRACEB(0);
    /* ---- the bands of this wave's tokens ---- */
    int32_t ps[TW], pe[TW];
    uint32_t nb[TW];
#pragma unroll
    for (uint32_t k = 0; k < TW; k++) {
        const uint32_t t = t0 + k;
        ps[k] = 1;
        pe[k] = 0;
        nb[k] = width;
        if (t < n_tok)
            nb[k] = band_of_tail(a.idx + (size_t)t * a.tok_stride + (size_t)kh * a.kvh_stride,
                                 width, a.max_kv, lane, ps[k], pe[k]);
        if (lane == 0) {
            s_ps[wave * TW + k] = ps[k];
            s_pe[wave * TW + k] = pe[k];
        }
    }
    __syncthreads();
    int32_t lo = INT32_MAX, hi = INT32_MIN;
#pragma unroll
    for (uint32_t w = 0; w < BAND_TOK; w++)
        if (s_ps[w] <= s_pe[w]) {
            lo = min(lo, s_ps[w]);
            hi = max(hi, s_pe[w]);
        }
    const bool tile = lo <= hi && (int64_t)hi - lo + 1 <= (int64_t)BAND_SPAN;
#pragma unroll
    for (uint32_t k = 0; k < TW; k++) {
        const uint32_t t = t0 + k;
        if (!tile) {
            ps[k] = 1;
            pe[k] = 0;
            nb[k] = width;
        }
        if (t < n_tok) {
            const uint32_t item = t * a.n_kvh + kh;
            if (lane == 0) a.band_nb[item] = (int32_t)nb[k];
            if (ps[k] > pe[k] && lane < gqa)
                stg((fv2 *)(a.band_ml + ((size_t)item * gqa + lane) * 2u), (fv2){-INFINITY, 0.f});
        }
    }
    if (!tile) return; /* uniform over the workgroup */
    TRACEB(1);
    const uint32_t n_pass = (uint32_t)(hi - lo) / BP + 1u;

    /* the Q^T operands of this wave's tokens, natural dim order. Each head's
     * q x scale is divided by the power of two 2^e that brings its largest
     * magnitude into [0.5, 1) (exact: the fp16 parts neither overflow nor
     * lose relative precision), and its scores are multiplied by qmul = 2^e;
     * the eight lanes holding a head (columns c, c + 8, k-groups 0-3) find
     * its maximum together. */
    h8_t qB[TW][8];
    float qmul[TW];
#pragma unroll
    for (uint32_t k = 0; k < TW; k++) {
        const uint32_t t = t0 + k, h = c & 7u;
        const bool hv = t < n_tok && h < gqa;
        const float *qr = a.q + ((size_t)(t < n_tok ? t : 0u) * a.n_head + kh * gqa + (hv ? h : 0u)) * 256u;
        float am = 0.f;
#pragma unroll
        for (uint32_t b = 0; b < 8u; b++) {
            const f4_t x0 = ldg((const f4_t *)(qr + 32u * b + 8u * jg));
            const f4_t x1 = ldg((const f4_t *)(qr + 32u * b + 8u * jg + 4u));
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) am = fmaxf(am, fmaxf(fabsf(x0[i]), fabsf(x1[i])));
        }
        am = fmaxf(am, __shfl_xor(am, 8));
        am = fmaxf(am, __shfl_xor(am, 16));
        am = fmaxf(am, __shfl_xor(am, 32));
        am *= a.scale_log2;
        const int e = (am > 0.f && am <= 3.4e38f) ? __builtin_amdgcn_frexp_expf(am) : 0;
        qmul[k] = __builtin_ldexpf(1.f, e);
        const float qs = hv ? __builtin_ldexpf(a.scale_log2, -e) : 0.f;
#pragma unroll
        for (uint32_t b = 0; b < 8u; b++) {
            const f4_t x0 = ldg((const f4_t *)(qr + 32u * b + 8u * jg));
            const f4_t x1 = ldg((const f4_t *)(qr + 32u * b + 8u * jg + 4u));
            qB[k][b] = __builtin_bit_cast(
                h8_t, (u4_t){split_pk(x0[0] * qs, x0[1] * qs, nsel), split_pk(x0[2] * qs, x0[3] * qs, nsel),
                             split_pk(x1[0] * qs, x1[1] * qs, nsel), split_pk(x1[2] * qs, x1[3] * qs, nsel)});
        }
    }

    /* the rows of pass p: 32 positions x 17 sixteen-byte pieces per cache;
     * wave w issues K and V instruction w (and wave 0 / 1 the ninth) */
    auto issue = [&](uint32_t pass, uint8_t *rawb) {
        const int32_t base = lo + (int32_t)(pass * BP);
        /* K and V instruction u = wave; wave 0 / 1 also the ninth K / V
         * instruction */
#pragma unroll
        for (uint32_t k = 0; k < 2u; k++) {
            const uint32_t u = k == 0u ? wave : 8u;
            if (k == 1u && wave > 1u) break;
            const uint32_t e = u * 64u + lane;
            const uint32_t r = e / NCH, q = e - r * NCH;
            int32_t p = base + (int32_t)r;
            if (p > hi || (uint32_t)p >= a.max_kv) p = lo; /* outside every band: masked */
            const size_t off = (size_t)p * rstride + q * 16u;
            if (u < 8u || lane < 32u) {
                if (k == 0u || wave == 0u) dma16_manual(kbase + off, rawb + u * 1024u);
                if (k == 0u || wave == 1u) dma16_manual(vbase + off, rawb + BP * ROWB + u * 1024u);
            }
        }
    };
    /* the Q operands are complete before the first DMA: a compiler wait for
     * a load issued after the (assembly) DMAs would drain those too */
#pragma unroll
    for (uint32_t k = 0; k < TW; k++)
#pragma unroll
        for (uint32_t bb = 0; bb < 8u; bb++) asm volatile("" ::"v"(qB[k][bb]));
    TRACEB(2);
    issue(0u, rawA);
    if (n_pass > 1u) issue(1u, rawB);

    float m_run[TW], l_run[TW];
    f4_t acc[TW][16];
#pragma unroll
    for (uint32_t k = 0; k < TW; k++) {
        m_run[k] = -INFINITY;
        l_run[k] = 0.f;
#pragma unroll
        for (uint32_t T = 0; T < 16u; T++) acc[k][T] = (f4_t){0.f, 0.f, 0.f, 0.f};
    }

    auto run_pass = [&](uint32_t pass, uint8_t *rawb) {
        /* this pass's rows landed (the next pass's may still be in flight:
         * s_waitcnt vmcnt(n) with the lgkm / exp counts unconstrained; waves
         * 0 and 1 issue three DMA instructions per pass, the others two) */
        if (pass + 1u < n_pass) {
            if (wave <= 1u)
                __builtin_amdgcn_s_waitcnt(0x0F73);
            else
                __builtin_amdgcn_s_waitcnt(0x0F72);
        } else {
            __builtin_amdgcn_s_waitcnt(0);
        }
        barrier_lds(); /* rows landed; every wave done with the last pass */
        if (pass == 4u) TRACEB(3);
        /* ---- dequantise: K' rows (work item: position x >> 4, 16 dims) ---- */
#pragma unroll
        for (uint32_t x = tid; x < 512u; x += 64u * BAND_WAVES) {
            const uint32_t p = x >> 4, d0 = 16u * (x & 15u), b = d0 >> 5;
            const uint8_t *src = rawb + p * ROWB + 34u * b + 2u + (d0 & 31u);
            const float ks = ld_h(rawb + p * ROWB + 34u * b);
            uint32_t hw[8], lw[8];
#pragma unroll
            for (uint32_t i = 0; i < 8u; i++) {
                const uint32_t w = *(const uint16_t *)(src + 2u * i);
                const float x0 = (float)(int32_t)(int8_t)(w & 0xffu) * ks;
                const float x1 = (float)(int32_t)(int8_t)(w >> 8) * ks;
                hw[i] = pkrtz(x0, x1);
                lw[i] = pkrtz(x0 - h2lo(hw[i]), x1 - h2hi(hw[i]));
            }
            *(u4_t *)&kp[0][p][d0] = (u4_t){hw[0], hw[1], hw[2], hw[3]};
            *(u4_t *)&kp[0][p][d0 + 8u] = (u4_t){hw[4], hw[5], hw[6], hw[7]};
            *(u4_t *)&kp[1][p][d0] = (u4_t){lw[0], lw[1], lw[2], lw[3]};
            *(u4_t *)&kp[1][p][d0 + 8u] = (u4_t){lw[4], lw[5], lw[6], lw[7]};
        }
        /* ---- V'^T (work item: dims 2 dp, 2 dp + 1, slots 8 g .. 8 g + 7) ---- */
#pragma unroll
        for (uint32_t x = tid; x < 512u; x += 64u * BAND_WAVES) {
            const uint32_t dp = x & 127u, g = x >> 7, b = dp >> 4;
            const uint8_t *vr = rawb + BP * ROWB;
            uint32_t he[4], le[4], ho[4], lo4[4];
#pragma unroll
            for (uint32_t i2 = 0; i2 < 4u; i2++) {
                float xe[2], xo[2];
#pragma unroll
                for (uint32_t k = 0; k < 2u; k++) {
                    const uint32_t i = 2u * i2 + k;
                    const uint32_t p = i < 4u ? 4u * g + i : 16u + 4u * g + i - 4u;
                    const uint8_t *row = vr + p * ROWB + 34u * b;
                    const float vs = ld_h(row);
                    const uint32_t w = *(const uint16_t *)(row + 2u + 2u * (dp & 15u));
                    xe[k] = (float)(int32_t)(int8_t)(w & 0xffu) * vs;
                    xo[k] = (float)(int32_t)(int8_t)(w >> 8) * vs;
                }
                he[i2] = pkrtz(xe[0], xe[1]);
                le[i2] = pkrtz(xe[0] - h2lo(he[i2]), xe[1] - h2hi(he[i2]));
                ho[i2] = pkrtz(xo[0], xo[1]);
                lo4[i2] = pkrtz(xo[0] - h2lo(ho[i2]), xo[1] - h2hi(ho[i2]));
            }
            *(u4_t *)&vt[0][2u * dp][8u * g] = (u4_t){he[0], he[1], he[2], he[3]};
            *(u4_t *)&vt[1][2u * dp][8u * g] = (u4_t){le[0], le[1], le[2], le[3]};
            *(u4_t *)&vt[0][2u * dp + 1u][8u * g] = (u4_t){ho[0], ho[1], ho[2], ho[3]};
            *(u4_t *)&vt[1][2u * dp + 1u][8u * g] = (u4_t){lo4[0], lo4[1], lo4[2], lo4[3]};
        }
        barrier_lds(); /* K', V'^T ready; this pass's raw rows are free */
        if (pass == 4u) TRACEB(4);
        if (pass + 2u < n_pass) issue(pass + 2u, rawb);
        const int32_t base = lo + (int32_t)(pass * BP);
        bool live[TW], any = false;
#pragma unroll
        for (uint32_t k = 0; k < TW; k++) {
            live[k] = ps[k] <= pe[k] && base <= pe[k] && base + (int32_t)BP - 1 >= ps[k];
            any = any || live[k];
        }
        if (!any) return; /* wave-uniform */
        if (pass == 4u) TRACEB(5);
        /* ---- scores of the tokens' 8 heads at the pass's 32 positions ---- */
        f4_t S[TW][2];
#pragma unroll
        for (uint32_t k = 0; k < TW; k++) S[k][0] = S[k][1] = (f4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t b = 0; b < 8u; b++) {
#pragma unroll
            for (uint32_t tt = 0; tt < 2u; tt++) {
#pragma unroll
                for (uint32_t hl = 0; hl < 2u; hl++) {
                    const h8_t A = *(const h8_t *)&kp[hl][16u * tt + c][32u * b + 8u * jg];
#pragma unroll
                    for (uint32_t k = 0; k < TW; k++)
                        S[k][tt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, qB[k][b], S[k][tt], 0, 0, 0);
                }
            }
        }
        h8_t B[TW];
#pragma unroll
        for (uint32_t k = 0; k < TW; k++) {
            float T[8];
#pragma unroll
            for (uint32_t i = 0; i < 8u; i++) {
                const int32_t P = base + (int32_t)((i < 4u ? 0u : 16u) + 4u * jg + (i & 3u));
                const float x = add_ror8(S[k][i >> 2][i & 3u]) * qmul[k];
                T[i] = (P >= ps[k] && P <= pe[k]) ? x : -INFINITY;
            }
            float mx = fmax3v(fmax3v(T[0], T[1], T[2]), fmax3v(T[3], T[4], T[5]), fmax2(T[6], T[7]));
            mx = max32(max16(mx));
            const float mn = fmax2(m_run[k], mx);
            const float ms = mn == -INFINITY ? 0.f : mn;
            const float alpha = __builtin_amdgcn_exp2f(m_run[k] - ms);
            const bool grew = mn > m_run[k];
            m_run[k] = mn;
            float P[8], ls = 0.f;
#pragma unroll
            for (uint32_t i = 0; i < 8u; i++) {
                P[i] = __builtin_amdgcn_exp2f(T[i] - ms);
                ls += P[i];
            }
            l_run[k] = l_run[k] * alpha + ls;
            if (__ballot(grew) != 0u) {
#pragma unroll
                for (uint32_t T2 = 0; T2 < 16u; T2++) acc[k][T2] *= alpha;
            }
            B[k] = __builtin_bit_cast(
                h8_t, (u4_t){split_pk(P[0], P[1], nsel), split_pk(P[2], P[3], nsel),
                             split_pk(P[4], P[5], nsel), split_pk(P[6], P[7], nsel)});
        }
#pragma unroll
        for (uint32_t T2 = 0; T2 < 16u; T2++) {
#pragma unroll
            for (uint32_t hl = 0; hl < 2u; hl++) {
                const h8_t A = *(const h8_t *)&vt[hl][16u * T2 + c][8u * jg];
#pragma unroll
                for (uint32_t k = 0; k < TW; k++)
                    acc[k][T2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[k], acc[k][T2], 0, 0, 0);
            }
        }
        TRACEB(8u + (pass < 7u ? pass : 7u));
    };
    for (uint32_t pass = 0; pass < n_pass; pass += 2u) {
        run_pass(pass, rawA);
        if (pass == 4u) TRACEB(6);
        if (pass + 1u < n_pass) run_pass(pass + 1u, rawB);
    }
    TRACEB(7);
    /* ---- the partials: (m, l) per head, unnormalised rows in out ---- */
#pragma unroll
    for (uint32_t k = 0; k < TW; k++) {
        const uint32_t t = t0 + k;
        if (t >= n_tok || ps[k] > pe[k]) continue;
        const uint32_t item = t * a.n_kvh + kh;
        const float lw = pair32_sum(sum16(l_run[k]));
        if (lane < gqa) stg((fv2 *)(a.band_ml + ((size_t)item * gqa + lane) * 2u), (fv2){m_run[k], lw});
        float *orow = a.out + ((size_t)t * a.n_head + kh * gqa) * 256u;
#pragma unroll
        for (uint32_t T2 = 0; T2 < 16u; T2++) {
            f4_t v;
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) v[i] = add_ror8(acc[k][T2][i]);
            if (c < gqa) stg((f4_t *)(orow + (size_t)c * 256u + 16u * T2 + 4u * jg), v);
        }
    }
}

/* Merge the S split partials of one (item, head): weights 2^(m_s - M) over
 * splits with l_s > 0, then the sigmoid gate (src/q4_rocm.cu:6968-7013).
 * Thread c owns output column c. For S <= COMB_REG every partial load
 * (its columns, and one split's m_s, l_s per lane) is issued before the
 * first is used and the merge needs neither LDS nor barriers. */
#define COMB_MAXS 1024u
#define COMB_REG 64u

/* R >= S: all S partials in registers (indices past S re-read split S-1 and
 * get weight 0). Lane k of every wave loads split k's (m, l) (S <= 64), so a
 * thread has R + 2 loads in flight (within the 63 the vmcnt counter holds,
 * one memory round trip); the weights 2^(m_k - M) are formed once per lane
 * and read back per split with v_readlane. xv = *xp is loaded in the same
 * round trip (the gate value, where there is one). */
template <uint32_t R>
__device__ static inline float comb_reg(const float *pb, size_t sst, uint32_t S, uint32_t col,
                                        float &L, const float *xp, float &xv) {
    static_assert(R <= 64u, "one split per lane");
    const uint32_t lane = threadIdx.x & 63u;
    const float *pm = pb + (lane < S ? lane : S - 1u) * sst;
    const float mk = ldg(pm), lk = ldg(pm + 1u);
    float v[R];
#pragma unroll
    for (uint32_t k = 0; k < R; k++) v[k] = ldg(pb + (k < S ? k : S - 1u) * sst + 2u + col);
    xv = ldg(xp);
    /* every load above is issued before the wait for (m, l) */
    __builtin_amdgcn_sched_barrier(0);
    const bool ok = lane < S && lk > 0.f;
    const float M = wave_max64(ok ? mk : -INFINITY);
    const float w = ok ? __builtin_amdgcn_exp2f(mk - M) : 0.f;
    L = wave_sum64(w * lk);
    float acc = 0.f;
#pragma unroll
    for (uint32_t k = 0; k < R; k++)
        acc += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), (int)k)) * v[k];
    return acc;
}

/* The merged (unnormalised) column col of one (item, head) from its S split
 * partials at pb (stride sst), L the merged denominator; xv = *xp, loaded
 * with the partials. */
__device__ static inline float comb_cols(const float *pb, size_t sst, uint32_t S, uint32_t col,
                                         float &L, const float *xp, float &xv) {
    if (S <= 8u) return comb_reg<8>(pb, sst, S, col, L, xp, xv);
    if (S <= 16u) return comb_reg<16>(pb, sst, S, col, L, xp, xv);
    if (S <= 20u) return comb_reg<20>(pb, sst, S, col, L, xp, xv);
    if (S <= 24u) return comb_reg<24>(pb, sst, S, col, L, xp, xv);
    if (S <= 32u) return comb_reg<32>(pb, sst, S, col, L, xp, xv);
    if (S <= 36u) return comb_reg<36>(pb, sst, S, col, L, xp, xv);
    if (S <= 48u) return comb_reg<48>(pb, sst, S, col, L, xp, xv);
    if (S <= COMB_REG) return comb_reg<COMB_REG>(pb, sst, S, col, L, xp, xv);
    /* long split lists: two passes over the partials */
    xv = ldg(xp);
    float M = -INFINITY, acc = 0.f;
    L = 0.f;
    for (uint32_t sp = 0; sp < S; sp++)
        if (ldg(pb + sp * sst + 1u) > 0.f) M = fmax2(M, ldg(pb + sp * sst));
    for (uint32_t sp = 0; sp < S; sp++) {
        const float l = ldg(pb + sp * sst + 1u);
        if (l > 0.f) {
            const float w = __builtin_amdgcn_exp2f(ldg(pb + sp * sst) - M);
            L += w * l;
            acc += w * ldg(pb + sp * sst + 2u + col);
        }
    }
    return acc;
}

template <int KIND, int MODE>
__global__ __launch_bounds__(256) void qsa_comb_k(AttnArgs a) {
    const uint32_t g = blockIdx.x, item = a.item0 + blockIdx.y, tid = threadIdx.x;
    const uint32_t gqa = a.n_head / a.n_kvh, hd = a.hd, S = a.S;
    const float *pb = a.part + ((size_t)item * S * gqa + g) * PSTRIDE;
    const size_t sst = (size_t)gqa * PSTRIDE;
    const uint32_t dim = col_dim<KIND>(tid);
    const bool dvalid = dim < hd;
    const uint32_t col = dvalid ? tid : 0u;
    const Item it = resolve_item<MODE>(a, item);
    /* the gate value is loaded with the partials (any readable word when
     * there is no gate) */
    const float *gp = it.gate && dvalid ? it.gate + (size_t)g * hd + dim : pb;
    float L, gv;
    const float acc = comb_cols(pb, sst, S, col, L, gp, gv);
    if (!dvalid) return;
    float r = L > 0.f ? acc / L : 0.f;
    if (it.gate) r *= 1.f / (1.f + expf(-gv));
    stg(it.out + (size_t)g * hd + dim, r);
}

/* The merge epilogue fused with the attention output projection
 * (src/q4_fwd.c:922-927: the split merge with its gate, then the q8_0
 * attn_output GEMV): workgroup (head, row block) of item seq merges that
 * head's split partials exactly as qsa_comb_k does (or, with one split,
 * reads the finished output), keeps the gated head row in LDS, writes it to
 * the output buffer (row block 0), and adds y_scale * W[rows][head cols] x_h
 * into y with fp32 atomics: four lanes per row, two q8_0 blocks each. The
 * sixteen heads' contributions to a row are summed in arrival order. */
constexpr uint32_t OUT_RPB = 256; /* W rows per workgroup */

template <int MODE>
__global__ __launch_bounds__(256) void qsa_comb_gemv_k(AttnArgs a, const q4kv_out_desc *od,
                                                       uint32_t n_embd, uint32_t n_rb,
                                                       float y_scale) {
    __shared__ __attribute__((aligned(16))) float xh[256];
    __shared__ float xsum[8];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t h = blockIdx.x / n_rb, rb = blockIdx.x - h * n_rb, seq = blockIdx.y;
    const uint32_t gqa = a.n_head / a.n_kvh, hd = a.hd, S = a.S;
    const uint32_t kh = h / gqa, g = h - kh * gqa, item = seq * a.n_kvh + kh;
    const uint32_t dim = col_dim<Q4KV_Q8>(tid);
    const Item it = resolve_item<MODE>(a, item);
    float r;
    if (S > 1u) {
        const float *pb = a.part + ((size_t)item * S * gqa + g) * PSTRIDE;
        const size_t sst = (size_t)gqa * PSTRIDE;
        const float *gp = it.gate ? it.gate + (size_t)g * hd + dim : pb;
        float L, gv;
        const float acc = comb_cols(pb, sst, S, tid, L, gp, gv);
        r = L > 0.f ? acc / L : 0.f;
        if (it.gate) r *= 1.f / (1.f + expf(-gv));
        if (rb == 0) stg(it.out + (size_t)g * hd + dim, r);
    } else {
        r = ldg(it.out + (size_t)g * hd + dim); /* one split: already merged and gated */
    }
    xh[dim] = r;
    __syncthreads();
    if (tid < 8u) {
        float sx = 0.f;
        for (int i = 0; i < 32; i++) sx += xh[32u * tid + i];
        xsum[tid] = sx;
    }
    __syncthreads();
    const uint8_t *w = (const uint8_t *)ldg(&od[seq].w_o);
    float *y = q4kv_gptr_at(&od[seq].y);
    const size_t rowb = (size_t)(a.n_head * hd / 32u) * 34u;
    const uint32_t pr = lane & 3u; /* this lane's block pair (64 columns) */
    const uint32_t rend = min(n_embd, (rb + 1u) * OUT_RPB);
    const float xa = xsum[2u * pr], xb = xsum[2u * pr + 1u];
    for (uint32_t row = rb * OUT_RPB + wave * 16u + (lane >> 2); row < rend; row += 64u) {
        uint32_t dw[17];
        const uint32_t *src = (const uint32_t *)(w + (size_t)row * rowb + (size_t)h * 272u + 68u * pr);
#pragma unroll
        for (int k = 0; k < 17; k++) dw[k] = ldg(src + k);
        float part = q4kv_q8_pair_dot(dw, xh, pr, xa, xb);
        part += q4kv_dpp<0xB1>(part); /* the row's four lanes */
        part += q4kv_dpp<0x4E>(part);
        if (pr == 0) atomicAdd(y + row, y_scale * part);
    }
}

/* ------------------------------------------------------------------------ */

/* Live timing of the split-KV kernel: HIP events recorded on the library
 * stream around each launch while armed (never inside a capture). */
#define Q4KV_PROF_MAX 4096
static hipEvent_t g_pev[2 * Q4KV_PROF_MAX];
static int g_pev_made = 0, g_prof_on = 0, g_prof_n = 0, g_prof_max = 0;

extern "C" bool q4kv_prof_begin(int max_launches) {
    if (!q4kv_ok || q4kv_capturing || max_launches <= 0 || max_launches > Q4KV_PROF_MAX)
        return false;
    for (; g_pev_made < 2 * max_launches; g_pev_made++)
        /* timing-only events: no system-scope fence (cache writeback and
         * invalidate) when they complete, which would add to the interval */
        if (hipEventCreateWithFlags(&g_pev[g_pev_made], hipEventDisableSystemFence) !=
            hipSuccess)
            return false;
    g_prof_on = 1;
    g_prof_n = 0;
    g_prof_max = max_launches;
    return true;
}

extern "C" int q4kv_prof_end(double *total_ms) {
    if (!q4kv_flush()) return -1;
    g_prof_on = 0;
    if (total_ms) *total_ms = 0.0;
    if (!g_prof_n) return 0;
    if (hipEventSynchronize(g_pev[2 * g_prof_n - 1]) != hipSuccess) return -1;
    double t = 0.0;
    for (int i = 0; i < g_prof_n; i++) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, g_pev[2 * i], g_pev[2 * i + 1]) != hipSuccess) return -1;
        t += ms;
    }
    if (total_ms) *total_ms = t;
    return g_prof_n;
}

static inline bool prof_armed(void) {
    return g_prof_on && !q4kv_capturing && g_prof_n < g_prof_max;
}

/* Workgroups a launch aims for (Q4KV_SPLIT_TARGET overrides, like the
 * reference's Q4_DEC_SPLIT_S tuning knob). */
static uint32_t split_target(void) {
    static uint32_t t = 0;
    if (!t) {
        const char *e = getenv("Q4KV_SPLIT_TARGET");
        const long v = e ? strtol(e, nullptr, 10) : 0;
        t = (v >= 1 && v <= 1 << 20) ? (uint32_t)v : 512u;
    }
    return t;
}
#define Q4KV_MAX_GRID_Y 65535u

/* Chunks per workgroup from which the fast kernel double-buffers its rows
 * (Q4KV_DB_MIN overrides, for measurement). */
static uint32_t db_min_chunks(void) {
    static uint32_t t = 0;
    if (!t) {
        const char *e = getenv("Q4KV_DB_MIN");
        const long v = e ? strtol(e, nullptr, 10) : 0;
        t = (v >= 1 && v <= 1 << 20) ? (uint32_t)v : 3u;
    }
    return t;
}

struct OutProj {
    const q4kv_out_desc *od;
    uint32_t n_embd;
    float y_scale;
};

/* Where a launch's split partials go: the library's buffer (allocated by
 * q4_hip_init), or the static scratch of the no-allocation entry point. */
struct PartBuf {
    float *ptr;
    size_t cap; /* floats */
};
static PartBuf lib_part(void) { return PartBuf{q4kv_part, q4kv_part_cap}; }

/* The split count S and chunks per split for n_items items of up to max_n
 * list entries, bounded by a partial buffer of cap floats (0 or no buffer:
 * one split, finalised in place). The same inputs always give the same
 * division, so two entry points that share it give identical results. */
static void choose_split(uint32_t n_items, uint32_t n_chunks, uint32_t gqa, bool have_part,
                         size_t cap, uint32_t &S, uint32_t &cps) {
    /* Fill the chip once: the fast q8 kernel keeps 2 workgroups per CU
     * resident, the generic one about as many; more splits than that only
     * add a second round of workgroups and more partials to merge. */
    S = (split_target() + n_items - 1u) / n_items;
    if (S > n_chunks) S = n_chunks;
    if (S < 1u) S = 1u;
    /* at most COMB_REG splits: the merge then holds every partial in
     * registers (one memory round trip; past that it walks them) */
    if (S > COMB_REG) S = COMB_REG;
    const size_t per = (size_t)gqa * PSTRIDE;
    while (S > 1u && (size_t)n_items * S * per > cap) S--;
    if (!have_part) S = 1u;
    cps = n_chunks ? (n_chunks + S - 1u) / S : 1u;
    if (n_chunks) S = (n_chunks + cps - 1u) / cps;
    if (S < 1u) S = 1u;
}

/* ---- shapes outside the MFMA kernels' tiling ----
 * head_dim not a multiple of 32 (f16 / f32 caches, any hd <= 256), or more
 * than 16 query heads per KV head (any width). The reference runs these on
 * its one-block-per-head fallback (src/q4_rocm.cu:7286-7297); here one
 * workgroup (4 x wave64) owns one (item, split, group of up to 8 query heads)
 * and walks its list 256 entries at a time, 64 per wave:
 *  - scores: lane = list entry; it reads its own K row element by element
 *    (dequantised) against the group's query rows, held pre-scaled in LDS
 *    and read as broadcasts;
 *  - online softmax in base 2 per wave and head (wave max / sum over the
 *    64 entries), the weights through LDS;
 *  - P.V: lane = dimension (4 per lane), one V row per valid entry of the
 *    wave's 64, coalesced across the wave;
 *  - the four waves' (m, l, acc) merge in LDS; one split finalises (gate,
 *    output), several write the partial rows qsa_comb_k merges (natural
 *    column order). */
constexpr uint32_t ANY_HEADS = 8u;

__device__ static inline float ld_f16_g(const uint8_t *p) {
    return __half2float(__ushort_as_half(ldg((const uint16_t *)p)));
}

template <int KIND>
__device__ static inline float any_elem(const uint8_t *row, uint32_t d) {
    if (KIND == Q4KV_F32) return ldg((const float *)row + d);
    if (KIND == Q4KV_F16) return ld_f16_g(row + 2u * d);
    const uint8_t *blk = row + 34u * (d >> 5);
    return ld_f16_g(blk) * (float)(int8_t)ldg(blk + 2u + (d & 31u));
}


template <int KIND, int MODE>
__global__ __launch_bounds__(256) void qsa_any_k(AttnArgs a) {
    constexpr uint32_t NH = ANY_HEADS;
    __shared__ float qs[NH][256];
    __shared__ float pw[4][64][NH];
    __shared__ float wm[4][NH], wl[4][NH];
    __shared__ float wacc[4][NH][256];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t s = blockIdx.x, item = a.item0 + blockIdx.y, h0 = blockIdx.z * NH;
    const uint32_t gqa = a.n_head / a.n_kvh, hd = a.hd, kh = item % a.n_kvh;
    const uint32_t nh = gqa - h0 < NH ? gqa - h0 : NH;
    const Item it = resolve_item<MODE>(a, item);
    const uint32_t rowb = KIND == Q4KV_Q8 ? hd / 32u * 34u : hd * (KIND == Q4KV_F16 ? 2u : 4u);
    const size_t rstride = (size_t)a.n_kvh * rowb;
    const uint8_t *kbase = it.kc + (size_t)kh * rowb, *vbase = it.vc + (size_t)kh * rowb;

    for (uint32_t e = tid; e < NH * 256u; e += 256u) {
        const uint32_t h = e >> 8, d = e & 255u;
        qs[h][d] = (h < nh && d < hd) ? ldg(it.q + (size_t)(h0 + h) * hd + d) * a.scale_log2 : 0.f;
    }
    __syncthreads();

    const uint32_t n = it.n;
    const uint32_t j0 = (uint32_t)(((uint64_t)s * n) / a.S);
    const uint32_t j1 = (uint32_t)(((uint64_t)(s + 1u) * n) / a.S);
    float m[NH], l[NH], acc[NH][4];
#pragma unroll
    for (uint32_t h = 0; h < NH; h++) {
        m[h] = -INFINITY;
        l[h] = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) acc[h][i] = 0.f;
    }
    /* every wave runs the same iterations (the barriers stay matched) */
    for (uint32_t c0 = j0; c0 < j1; c0 += 256u) {
        const uint32_t j = c0 + 64u * wave + lane;
        int32_t p = -1;
        if (j < j1) p = it.list ? ldg(it.list + j) : (int32_t)j;
        const bool ok = p >= 0 && (uint32_t)p < it.max_kv;
        float sc[NH];
#pragma unroll
        for (uint32_t h = 0; h < NH; h++) sc[h] = 0.f;
        if (ok) {
            const uint8_t *kr = kbase + (size_t)p * rstride;
            for (uint32_t d = 0; d < hd; d++) {
                const float kv = any_elem<KIND>(kr, d);
#pragma unroll
                for (uint32_t h = 0; h < NH; h++) sc[h] = __builtin_fmaf(qs[h][d], kv, sc[h]);
            }
        }
#pragma unroll
        for (uint32_t h = 0; h < NH; h++) {
            const float x = ok ? sc[h] : -INFINITY;
            const float mn = fmaxf(m[h], wave_max64(x));
            const float ms = mn == -INFINITY ? 0.f : mn;
            const float alpha = __builtin_amdgcn_exp2f(m[h] - ms);
            const float pv = __builtin_amdgcn_exp2f(x - ms);
            l[h] = l[h] * alpha + wave_sum64(pv);
            m[h] = mn;
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) acc[h][i] *= alpha;
            pw[wave][lane][h] = pv;
        }
        __syncthreads();
        uint64_t vm = __ballot(ok);
        while (vm) {
            const uint32_t jj = (uint32_t)__builtin_ctzll(vm);
            vm &= vm - 1u;
            const int32_t pj = __shfl(p, (int)jj);
            const uint8_t *vr = vbase + (size_t)pj * rstride;
#pragma unroll
            for (uint32_t i = 0; i < 4u; i++) {
                const uint32_t d = lane + 64u * i;
                if (d < hd) {
                    const float vv = any_elem<KIND>(vr, d);
#pragma unroll
                    for (uint32_t h = 0; h < NH; h++)
                        acc[h][i] = __builtin_fmaf(pw[wave][jj][h], vv, acc[h][i]);
                }
            }
        }
        __syncthreads(); /* pw is rewritten by the next iteration */
    }

    /* merge the four waves */
#pragma unroll
    for (uint32_t h = 0; h < NH; h++) {
        if (lane == 0u) {
            wm[wave][h] = m[h];
            wl[wave][h] = l[h];
        }
#pragma unroll
        for (uint32_t i = 0; i < 4u; i++) wacc[wave][h][lane + 64u * i] = acc[h][i];
    }
    __syncthreads();
    const bool fin = a.S == 1u;
    float *pbase = fin ? nullptr : a.part + ((size_t)item * a.S + s) * gqa * PSTRIDE;
    for (uint32_t e = tid; e < NH * 256u; e += 256u) {
        const uint32_t h = e >> 8, d = e & 255u;
        if (h >= nh || d >= hd) continue;
        float M = -INFINITY;
#pragma unroll
        for (uint32_t w = 0; w < 4u; w++) M = fmaxf(M, wm[w][h]);
        const float ms = M == -INFINITY ? 0.f : M;
        float L = 0.f, x = 0.f;
#pragma unroll
        for (uint32_t w = 0; w < 4u; w++) {
            const float f = __builtin_amdgcn_exp2f(wm[w][h] - ms);
            L += f * wl[w][h];
            x += f * wacc[w][h][d];
        }
        const uint32_t head = h0 + h;
        if (fin) {
            float r = L > 0.f ? x / L : 0.f;
            if (it.gate) r *= 1.f / (1.f + expf(-ldg(it.gate + (size_t)head * hd + d)));
            stg(it.out + (size_t)head * hd + d, r);
        } else {
            stg(pbase + head * PSTRIDE + 2u + d, x);
            if (d == 0u) {
                stg(pbase + head * PSTRIDE, M);
                stg(pbase + head * PSTRIDE + 1u, L);
            }
        }
    }
}

/* The kernels above need hd a multiple of 32 and at most 16 query heads per
 * KV head; every other shape runs qsa_any_k. */
static bool any_shape(uint32_t hd, uint32_t gqa) { return (hd % 32u) != 0u || gqa > 16u; }

/* qsa_any_k's split count: about split_target() workgroups, at most one
 * split per 256 list entries, partials within cap floats. */
static uint32_t any_splits(uint32_t n_items, uint32_t max_n, uint32_t gqa, bool have_part,
                           size_t cap) {
    const uint32_t hc = (gqa + ANY_HEADS - 1u) / ANY_HEADS;
    const uint32_t n_iter = max_n ? (max_n + 255u) / 256u : 1u;
    const uint64_t wgs = (uint64_t)n_items * hc;
    uint32_t S = wgs >= split_target() ? 1u : (uint32_t)((split_target() + wgs - 1u) / wgs);
    if (S > n_iter) S = n_iter;
    if (S > COMB_REG) S = COMB_REG; /* the merge's register path */
    const size_t per = (size_t)gqa * PSTRIDE;
    while (S > 1u && (size_t)n_items * S * per > cap) S--;
    return have_part && S >= 1u ? S : 1u;
}

template <int KIND, int MODE>
static bool launch_any(AttnArgs a, uint32_t n_items, uint32_t max_n, uint32_t gqa, PartBuf pb) {
    const uint32_t hc = (gqa + ANY_HEADS - 1u) / ANY_HEADS;
    const uint32_t S = any_splits(n_items, max_n, gqa, pb.ptr != nullptr, pb.cap);
    if (S > 1u && (size_t)n_items * S * gqa * PSTRIDE > pb.cap) {
        Q4KV_ERR("qsa attention: %u splits of %u items exceed the partial buffer", S, n_items);
        return false;
    }
    a.S = S;
    a.cps = 0u;
    a.part = pb.ptr;
    a.band_nb = nullptr;
    a.band_ml = nullptr;
    for (uint32_t i0 = 0; i0 < n_items; i0 += Q4KV_MAX_GRID_Y) {
        const uint32_t ni = n_items - i0 < Q4KV_MAX_GRID_Y ? n_items - i0 : Q4KV_MAX_GRID_Y;
        a.item0 = i0;
        qsa_any_k<KIND, MODE><<<dim3(S, ni, hc), 256, 0, q4kv_stream>>>(a);
        /* natural column order: the f32 instance's column map */
        if (S > 1u) qsa_comb_k<Q4KV_F32, MODE><<<dim3(gqa, ni), 256, 0, q4kv_stream>>>(a);
    }
    return hipGetLastError() == hipSuccess;
}

/* Which kernel runs a launch, and its split division. */
struct Plan {
    bool slab;    /* qsa_slab_k (else qsa_q8d256_k / qsa_attn_k) */
    uint32_t hg;  /* slab kernels: head groups of 8; the chunk kernel: its
                   * grid.z groups of 8 query heads (2 for 9-16 heads) */
    uint32_t S, cps;
    bool h16;     /* qsa_h16_k (f16 cache, hd 256) */
    bool f32w;    /* qsa_f32w_k (f32 cache, hd 256) */
};

/* The slab kernel takes q8_0 / hd 256 shapes with 9 to 16 query heads per KV
 * head (two head groups), and prefill-sized launches of any head count, whose
 * workgroups then stream their passes (each wave's online softmax carried
 * across them): there its lower VALU work per position wins (config 3: 2.82
 * vs 3.67 ms per layer). Decode launches with up to 8 query heads per KV head
 * keep the chunk kernel qsa_q8d256_k, whose shorter per-workgroup chain
 * measures faster there (18.7 vs 19.9 us for the 12-layer step).
 * Q4KV_SLAB=0 turns the slab kernel off, Q4KV_SLAB=2 uses it everywhere
 * (A/B measurement). */
#define SLAB_MAX_WG 16384u
static int slab_mode(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4KV_SLAB");
        v = !e ? 1 : e[0] == '0' ? 0 : e[0] == '2' ? 2 : 1;
    }
    return v;
}
static bool slab_takes(uint32_t gqa, bool prefill_sized) {
    const int m = slab_mode();
    return gqa <= 16u && (m == 2 || (m == 1 && (gqa > 8u || prefill_sized)));
}

/* Launches of up to this many items with 9-16 query heads per KV head take
 * the chunk kernel in two head groups (Q4KV_CHUNK_HG=<n> sets it, 0 off).
 * Measured against the slab kernel at 12 and 16 heads per KV head, 262144-
 * token cache: 9.9 vs 12.0 us at 2 items, 14.6 vs 15.2 at 8, 19.3 vs 19.6
 * at 16. */
static uint32_t chunk_hg_max_items(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4KV_CHUNK_HG");
        v = e ? atoi(e) : 16;
        if (v < 0) v = 0;
    }
    return (uint32_t)v;
}

template <int KIND, int MODE>
static Plan plan_launch(uint32_t hd, uint32_t n_items, uint32_t max_n, uint32_t gqa,
                        bool have_part, size_t cap, bool rows16 = true) {
    /* rows16: the caches are 16-byte aligned (the slab, f16 and f32 kernels
     * fetch 16-byte pieces; the chunk and generic kernels check for
     * themselves) */
    Plan pl = {false, 1u, 1u, 1u, false, false};
    const bool h16 = KIND == Q4KV_F16 && hd == 256u && gqa <= 16u && rows16 && h16_enabled();
    const bool f32w = KIND == Q4KV_F32 && hd == 256u && gqa <= 16u && rows16 && f32w_enabled();
    if (h16 || f32w) {
        /* splits of whole passes, as many as fill the chip's resident
         * workgroup slots once (choose_split, as the chunk kernel); launches
         * beyond that size (prefill) stream their passes through fewer
         * splits */
        const uint32_t hg = h16 && gqa > 8u ? 2u : 1u, ne = 4u / hg * 16u;
        const uint32_t s_full = max_n ? (max_n + ne - 1u) / ne : 1u;
        uint32_t S, cps;
        if ((uint64_t)n_items * s_full <= SLAB_MAX_WG) {
            choose_split(n_items, s_full, gqa, have_part, cap, S, cps);
        } else {
            S = n_items >= SLAB_MAX_WG ? 1u : SLAB_MAX_WG / n_items;
            if (S < 1u) S = 1u;
            if (S > COMB_REG) S = COMB_REG; /* the merge's register path */
            const size_t per = (size_t)gqa * PSTRIDE;
            while (S > 1u && (size_t)n_items * S * per > cap) S--;
            if (!have_part) S = 1u;
        }
        pl.h16 = h16;
        pl.f32w = f32w;
        pl.hg = hg;
        pl.S = S;
        pl.cps = 0u;
        return pl;
    }
    const uint32_t hg = gqa > 8u ? 2u : 1u, ne = 128u / hg;
    const uint32_t s_full = max_n ? (max_n + ne - 1u) / ne : 1u;
    const bool prefill_sized = (uint64_t)n_items * s_full > SLAB_MAX_WG;
    if (KIND == Q4KV_Q8 && hd == 256u && gqa > 8u && gqa <= 16u && !IS_BATCH(MODE) &&
        n_items <= chunk_hg_max_items()) {
        /* a few decode items with 9-16 query heads per KV head: the chunk
         * kernel in two head groups (grid.z) over the same rows; its shorter
         * per-workgroup chain beats the slab kernel where latency, not the
         * doubled gather, bounds the launch. Batch descriptors keep the slab
         * kernel, which splits each item's own length: the chunk kernel's
         * splits follow max_n, and a batch's max_n can far exceed most of
         * its items (four list items under max_n 262144: 91 vs 12.8 us) */
        constexpr uint32_t CP = KCfg<KIND>::CP;
        /* 2 n_items workgroups per split, ceil(gqa / 2) heads' partials each */
        choose_split(2u * n_items, (max_n + CP - 1u) / CP, (gqa + 1u) / 2u, have_part, cap,
                     pl.S, pl.cps);
        pl.hg = 2u;
        return pl;
    }
    bool slab = KIND == Q4KV_Q8 && hd == 256u && rows16 && slab_takes(gqa, prefill_sized);
    if (!slab && KIND == Q4KV_Q8 && hd == 256u && rows16 && gqa <= 8u && slab_mode() == 1) {
        /* many items (batched decode): where the chunk kernel would walk
         * three or more chunks per split, the slab kernel's barrier-free
         * passes measure faster (32 sequences: 30.7 vs 33.6 us per step) */
        uint32_t S0, cps0;
        choose_split(n_items, (max_n + 63u) / 64u, gqa, have_part, cap, S0, cps0);
        slab = cps0 >= db_min_chunks();
    }
    if (slab) {
        /* decode: splits of whole passes filling the resident slots once
         * (choose_split); many items (prefill): fewer splits, each wave
         * streaming its passes */
        uint32_t S, cps;
        if (!prefill_sized) {
            choose_split(n_items, s_full, gqa, have_part, cap, S, cps);
        } else {
            S = n_items >= SLAB_MAX_WG ? 1u : SLAB_MAX_WG / n_items;
            if (S < 1u) S = 1u;
            if (S > COMB_REG) S = COMB_REG; /* the merge's register path */
            const size_t per = (size_t)gqa * PSTRIDE;
            while (S > 1u && (size_t)n_items * S * per > cap) S--; /* waves then loop */
            if (!have_part) S = 1u;
        }
        {
            pl.slab = true;
            pl.hg = hg;
            pl.S = S;
            pl.cps = 0u;
            return pl;
        }
    }
    constexpr uint32_t CP = KCfg<KIND>::CP;
    choose_split(n_items, (max_n + CP - 1u) / CP, gqa, have_part, cap, pl.S, pl.cps);
    return pl;
}

/* The prefill band kernel (Q4KV_BAND=0 turns it off, for measurement). */
static bool band_enabled(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4KV_BAND");
        v = (e && e[0] == '0') ? 0 : 1;
    }
    return v != 0;
}

/* KV-head grouping on one XCD (xcd_slot). Q4KV_XPAIR=0 starts with it off;
 * q4kv_xcd_group switches it (measurement and tests). */
static int g_xpair = -1;
static bool xcd_pair_enabled(void) {
    if (g_xpair < 0) {
        const char *e = getenv("Q4KV_XPAIR");
        g_xpair = (e && e[0] == '0') ? 0 : 1;
    }
    return g_xpair != 0;
}
extern "C" int q4kv_xcd_group(int on) {
    if (on == 0 || on == 1) g_xpair = on;
    return xcd_pair_enabled() ? 1 : 0;
}

/* A fused append + attention launch exists for this shape. */
static bool step_fusable(int kind, uint32_t hd, uint32_t gqa) {
    if (kind == Q4KV_F16) return hd == 256u && gqa <= 16u && h16_enabled();
    if (kind == Q4KV_F32) return hd == 256u && gqa <= 16u && f32w_enabled();
    return kind == Q4KV_Q8 && hd == 256u && (gqa <= 8u || slab_takes(gqa, false));
}

/* The held append this launch can perform (same caches, whole 256-dim q8_0
 * rows of its KV heads). */
static bool held_matches(const AttnArgs &a) {
    const q4kv_held_append &h = q4kv_held;
    return h.on && h.kind == Q4KV_Q8 && h.kc == a.kc && h.vc == a.vc &&
           h.n == a.n_kvh * 256u && h.bpt == a.n_kvh * 272u;
}

template <int KIND, int MODE>
static bool launch_kind(AttnArgs a, uint32_t n_items, uint32_t max_n, uint32_t gqa,
                        const OutProj *op = nullptr, PartBuf pb = lib_part()) {
    if (any_shape(a.hd, gqa)) {
        if (!q4kv_flush()) return false;
        if constexpr (IS_STEP(MODE)) {
            return false;
        } else {
            if (op) return false;
            return launch_any<KIND, MODE>(a, n_items, max_n, gqa, pb);
        }
    }
    /* the kernels resolve items from what the mode names: descriptors, or
     * the direct arguments */
    if (IS_BATCH(MODE) ? !a.seqs : (!a.kc || !a.vc || !a.q || !a.out)) return false;
    const bool fast = KIND == Q4KV_Q8 && a.hd == 256u && gqa <= 8u;
    /* batch modes: the caches are in device descriptors, 16-byte aligned by
     * contract */
    const bool rows16 = IS_BATCH(MODE) || ((((uintptr_t)a.kc) | ((uintptr_t)a.vc)) & 15u) == 0u;
    const Plan pl =
        plan_launch<KIND, MODE>(a.hd, n_items, max_n, gqa, pb.ptr != nullptr, pb.cap, rows16);
    if (IS_STEP(MODE) && !fast && !pl.slab && !pl.h16 && !pl.f32w) return false; /* the fused append needs these */
    const uint32_t S = pl.S, cps = pl.cps;
    /* the chunk kernel: up to 8 query heads per KV head, or 9-16 in two
     * head groups (grid.z) */
    const uint32_t zg = !pl.slab && !pl.h16 && !pl.f32w && pl.hg == 2u ? 2u : 1u;
    const bool chunk = fast || zg == 2u;
    if (S > 1u && (!pb.ptr || (size_t)n_items * S * gqa * PSTRIDE > pb.cap)) {
        Q4KV_ERR("qsa attention: %u splits of %u items exceed the partial buffer", S, n_items);
        return false;
    }
    /* a held append on these caches rides in the chunk kernel's launch (one
     * launch pass: the split kernel then the merge); any other launch runs
     * it first */
    bool app = false;
    if constexpr (KIND == Q4KV_Q8 && (MODE == MODE_INDEXED || MODE == MODE_DENSE)) {
        /* the chunk kernel's single-buffer instance, or the slab kernel on
         * decode-sized launches (prefill-sized ones run the band kernel
         * first, which reads the rows without the substitution) */
        app = a.hd == 256u && n_items <= 64u && held_matches(a) &&
              ((chunk && !pl.slab && cps < db_min_chunks()) ||
               (pl.slab && gqa <= 16u && !(S == 1u && gqa <= 8u)));
        if (app) {
            a.app_k = q4kv_held.k;
            a.app_v = q4kv_held.v;
            a.app_pos = q4kv_pos_d;
            q4kv_held.on = 0;
        }
    }
    if (!app && !q4kv_flush()) return false;
    a.S = S;
    a.cps = cps;
    a.part = pb.ptr;
    for (uint32_t i0 = 0; i0 < n_items; i0 += Q4KV_MAX_GRID_Y) {
        const uint32_t ni = n_items - i0 < Q4KV_MAX_GRID_Y ? n_items - i0 : Q4KV_MAX_GRID_Y;
        a.item0 = i0;
        dim3 grid(S, ni, zg);
        /* the chunk kernel and the batched slab decode over whole tokens: the
         * KV heads of each (token, split) on one XCD (for the slab kernel's
         * prefill and the f16 / f32 kernels it measured 1-2 % slower) */
        a.xgrp = 0u;
        const bool grouped = pl.slab ? IS_BATCH(MODE) : (chunk && !pl.h16 && !pl.f32w);
        if (grouped && xcd_pair_enabled() && a.n_kvh > 1u && ni == n_items &&
            ni % a.n_kvh == 0u) {
            a.xgrp = ni / a.n_kvh * S;
            grid = dim3(8u * a.n_kvh * ((a.xgrp + 7u) / 8u), 1u, zg);
        }
        const bool prof = prof_armed();
        if (prof) (void)hipEventRecord(g_pev[2 * g_prof_n], q4kv_stream);
        /* prefill through the slab kernel (one split): the shared recent
         * window of consecutive tokens goes to the band kernel first */
        a.band_nb = nullptr;
        a.band_ml = nullptr;
        if (MODE == MODE_INDEXED && KIND == Q4KV_Q8 && pl.slab && S == 1u && gqa <= 8u &&
            band_enabled() && pb.ptr && (size_t)ni * (1u + 2u * gqa) <= pb.cap && ni % a.n_kvh == 0u) {
            AttnArgs ab = a;
            ab.band_nb = (int32_t *)pb.ptr;
            ab.band_ml = pb.ptr + ni;
            ab.kv_base = ni / a.n_kvh; /* tokens */
            ab.idx = a.idx + (size_t)(i0 / a.n_kvh) * a.tok_stride;
            ab.q = a.q + (size_t)(i0 / a.n_kvh) * a.n_head * a.hd;
            ab.out = a.out + (size_t)(i0 / a.n_kvh) * a.n_head * a.hd;
            qsa_band_k<<<dim3((ni / a.n_kvh + BAND_TOK - 1u) / BAND_TOK, a.n_kvh), 64u * BAND_WAVES, 0,
                         q4kv_stream>>>(ab);
            a.band_nb = ab.band_nb - i0; /* indexed by the launch's item */
            a.band_ml = ab.band_ml - (size_t)i0 * gqa * 2u;
        }
        /* double-buffered rows pay when a workgroup walks three or more chunks
         * (prefill, batched decode of many sequences); with one or two (the
         * 12-layer step) the extra LDS traffic does not */
        if (pl.f32w)
            qsa_f32w_k<MODE><<<grid, 256, 0, q4kv_stream>>>(a);
        else if (pl.h16 && pl.hg == 1u)
            qsa_h16_k<MODE, 1><<<grid, 256, 0, q4kv_stream>>>(a);
        else if (pl.h16)
            qsa_h16_k<MODE, 2><<<grid, 256, 0, q4kv_stream>>>(a);
        else if (pl.slab && app) {
            if constexpr (MODE == MODE_INDEXED || MODE == MODE_DENSE) {
                if (pl.hg == 1u)
                    qsa_slab_k<MODE, 1, true><<<grid, 256, 0, q4kv_stream>>>(a);
                else
                    qsa_slab_k<MODE, 2, true><<<grid, 256, 0, q4kv_stream>>>(a);
            }
        } else if (pl.slab && pl.hg == 1u) {
            bool piped = false;
            if constexpr (MODE == MODE_INDEXED || MODE == MODE_BATCH || MODE == MODE_STEP) {
                /* two or more passes per wave (a split's entries over 128 per
                 * pass): the pipelined passes */
                const uint32_t per_split = (max_n + S - 1u) / S;
                if (per_split > 128u && (MODE != MODE_INDEXED || a.idx) && slab_pipe_enabled()) {
                    qsa_slab_k<MODE, 1, false, true><<<grid, 256, 0, q4kv_stream>>>(a);
                    piped = true;
                }
            }
            if (!piped) qsa_slab_k<MODE, 1><<<grid, 256, 0, q4kv_stream>>>(a);
        }
        else if (pl.slab)
            qsa_slab_k<MODE, 2><<<grid, 256, 0, q4kv_stream>>>(a);
        else if (chunk && cps >= db_min_chunks())
            qsa_q8d256_k<MODE, true><<<grid, 256, 0, q4kv_stream>>>(a);
        else if (chunk && app) {
            if constexpr (MODE == MODE_INDEXED || MODE == MODE_DENSE)
                qsa_q8d256_k<MODE, false, true><<<grid, 256, 0, q4kv_stream>>>(a);
        } else if (chunk)
            qsa_q8d256_k<MODE, false><<<grid, 256, 0, q4kv_stream>>>(a);
        else if (IS_STEP(MODE))
            return false;
        else if (gqa <= 8u)
            qsa_attn_k<KIND, IS_STEP(MODE) ? MODE_BATCH : MODE, 1><<<grid, 256, 0, q4kv_stream>>>(a);
        else
            qsa_attn_k<KIND, IS_STEP(MODE) ? MODE_BATCH : MODE, 2><<<grid, 256, 0, q4kv_stream>>>(a);
        if (prof) (void)hipEventRecord(g_pev[2 * g_prof_n++ + 1], q4kv_stream);
        /* qsa_h16_k writes the q8_0 kernels' column order */
        if (S > 1u && !op && pl.h16)
            qsa_comb_k<Q4KV_Q8, MODE><<<dim3(gqa, ni), 256, 0, q4kv_stream>>>(a);
        else if (S > 1u && !op)
            qsa_comb_k<KIND, MODE><<<dim3(gqa, ni), 256, 0, q4kv_stream>>>(a);
    }
    if (op) {
        if (!chunk && !pl.slab) return false;
        a.item0 = 0;
        const uint32_t n_rb = (op->n_embd + OUT_RPB - 1u) / OUT_RPB;
        qsa_comb_gemv_k<MODE><<<dim3(a.n_head * n_rb, n_items / a.n_kvh), 256, 0, q4kv_stream>>>(
            a, op->od, op->n_embd, n_rb, op->y_scale);
    }
    return q4kv_launch_ok("qsa attention");
}

template <int MODE>
static bool launch_attn(int kind, const AttnArgs &a, uint32_t n_items, uint32_t max_n,
                        PartBuf pb = lib_part()) {
    const uint32_t gqa = a.n_head / a.n_kvh;
    switch (kind) {
    case Q4KV_Q8: return launch_kind<Q4KV_Q8, MODE>(a, n_items, max_n, gqa, nullptr, pb);
    case Q4KV_F16: return launch_kind<Q4KV_F16, MODE>(a, n_items, max_n, gqa, nullptr, pb);
    case Q4KV_F32: return launch_kind<Q4KV_F32, MODE>(a, n_items, max_n, gqa, nullptr, pb);
    default: return false;
    }
}

/* Shapes the attention entry points take: head_dim up to 256 (a multiple
 * of 32 for q8_0, whose rows are 32-element blocks), n_head a multiple of
 * n_kvh. */
static bool shape_ok(uint32_t n_head, uint32_t n_kvh, uint32_t hd, int kind) {
    if (!n_head || !n_kvh || !hd || hd > 256u || (n_head % n_kvh)) return false;
    if (kind == Q4KV_Q8 && (hd % 32u)) return false;
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
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d_descs || !n_seq || !max_n || !shape_ok(n_head, n_kvh, hd, kv_f16))
        return false;
    (void)hipGetLastError();
    AttnArgs a = base_args(nullptr, nullptr, nullptr, nullptr, nullptr, n_head, n_kvh, hd, 0,
                           scale);
    a.seqs = d_descs;
    a.desc_stride = sizeof(q4kv_seq_desc);
    return launch_attn<MODE_BATCH>(kv_f16, a, n_seq * n_kvh, max_n);
}

/* The split plan q4_hip_qsa_step_batch's launch takes for these arguments
 * (the dispatch of step_batch below, then launch_kind's plan_launch). */
static Plan step_batch_plan(int kind, uint32_t hd, uint32_t n_items, uint32_t max_n,
                            uint32_t gqa, bool have, size_t cap) {
    if (any_shape(hd, gqa)) return Plan{false, 1u, any_splits(n_items, max_n, gqa, have, cap), 0u};
    if (step_fusable(kind, hd, gqa) && kind == Q4KV_F16)
        return plan_launch<Q4KV_F16, MODE_STEP>(hd, n_items, max_n, gqa, have, cap);
    if (step_fusable(kind, hd, gqa) && kind == Q4KV_F32)
        return plan_launch<Q4KV_F32, MODE_STEP>(hd, n_items, max_n, gqa, have, cap);
    if (step_fusable(kind, hd, gqa))
        return plan_launch<Q4KV_Q8, MODE_STEP>(hd, n_items, max_n, gqa, have, cap);
    if (kind == Q4KV_F32) return plan_launch<Q4KV_F32, MODE_BATCH>(hd, n_items, max_n, gqa, have, cap);
    if (kind == Q4KV_F16) return plan_launch<Q4KV_F16, MODE_BATCH>(hd, n_items, max_n, gqa, have, cap);
    return plan_launch<Q4KV_Q8, MODE_BATCH>(hd, n_items, max_n, gqa, have, cap);
}

static bool step_batch(const q4kv_step_desc *d_descs, uint32_t n_seq, uint32_t n_head,
                       uint32_t n_kvh, uint32_t hd, float scale, int kv_f16, uint32_t max_n,
                       PartBuf pb) {
    (void)hipGetLastError();
    AttnArgs a = base_args(nullptr, nullptr, nullptr, nullptr, nullptr, n_head, n_kvh, hd, 0,
                           scale);
    a.seqs = (const q4kv_seq_desc *)d_descs;
    a.desc_stride = sizeof(q4kv_step_desc);
    const uint32_t gqa = n_head / n_kvh;
    if (step_fusable(kv_f16, hd, gqa) && kv_f16 == Q4KV_F16)
        return launch_kind<Q4KV_F16, MODE_STEP>(a, n_seq * n_kvh, max_n, gqa, nullptr, pb);
    if (step_fusable(kv_f16, hd, gqa) && kv_f16 == Q4KV_F32)
        return launch_kind<Q4KV_F32, MODE_STEP>(a, n_seq * n_kvh, max_n, gqa, nullptr, pb);
    if (step_fusable(kv_f16, hd, gqa))
        return launch_kind<Q4KV_Q8, MODE_STEP>(a, n_seq * n_kvh, max_n, gqa, nullptr, pb);
    /* other widths and shapes: the append launch, then the attention */
    const uint32_t row = kv_f16 == Q4KV_Q8 ? hd / 32u * 34u : hd * (kv_f16 == Q4KV_F16 ? 2u : 4u);
    if (!q4kv_append_steps(d_descs, n_seq, n_kvh * hd, n_kvh * row, kv_f16)) return false;
    return launch_attn<MODE_BATCH>(kv_f16, a, n_seq * n_kvh, max_n, pb);
}

extern "C" bool q4_hip_qsa_step_batch(const q4kv_step_desc *d_descs, uint32_t n_seq,
                                      uint32_t n_head, uint32_t n_kvh, uint32_t hd, float scale,
                                      int kv_f16, uint32_t max_n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d_descs || !n_seq || !max_n || !shape_ok(n_head, n_kvh, hd, kv_f16))
        return false;
    return step_batch(d_descs, n_seq, n_head, n_kvh, hd, scale, kv_f16, max_n, lib_part());
}

/* ---- the no-allocation variant of q4_hip_qsa_step_batch ----
 * Its split partials live in this file-scope device array instead of the
 * buffer q4_hip_init allocates. Each device holds its own copy; the host
 * reaches it only through the address hipGetSymbolAddress returns for the
 * current device (the array's name in host code is not a device address).
 * Nothing in it needs clearing: every partial row the merge reads is
 * written by the same launch first. Calls that overlap on one device share
 * the array and race. */
#define Q4KV_SCRATCH_FLOATS (4u << 20) /* 16 MiB */
#define Q4KV_SCRATCH_DEVS 64
static __device__ __align__(256) float scratch[Q4KV_SCRATCH_FLOATS];
static float *g_scratch_ptr[Q4KV_SCRATCH_DEVS];

/* Resolve the scratch address on the current device (once per device; the
 * library's init calls it with its device current). */
extern "C" bool q4kv_scratch_init(void) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= Q4KV_SCRATCH_DEVS) {
        (void)hipGetLastError();
        Q4KV_ERR("scratch init: no current device below %d", Q4KV_SCRATCH_DEVS);
        return false;
    }
    if (g_scratch_ptr[dev]) return true;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        Q4KV_ERR("scratch init: hipGetSymbolAddress: %s", hipGetErrorString(e));
        return false;
    }
    g_scratch_ptr[dev] = (float *)p;
    return true;
}

extern "C" bool q4_hip_qsa_step_batch_noalloc(const q4kv_step_desc *d_descs, uint32_t n_seq,
                                              uint32_t n_head, uint32_t n_kvh, uint32_t hd,
                                              float scale, int kv_f16, uint32_t max_n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d_descs || !n_seq || !max_n || !shape_ok(n_head, n_kvh, hd, kv_f16))
        return false;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= Q4KV_SCRATCH_DEVS ||
        !g_scratch_ptr[dev]) {
        (void)hipGetLastError();
        Q4KV_ERR("qsa_step_batch_noalloc: scratch not resolved on this device (q4_hip_init)");
        return false;
    }
    /* the split division q4_hip_qsa_step_batch takes with the library's
     * buffer (so the same results) must fit the static scratch; planned on
     * the scratch's own capacity it is then the same division (every larger
     * split count misses the larger buffer too) */
    const uint32_t gqa = n_head / n_kvh, n_items = n_seq * n_kvh;
    const Plan pl = step_batch_plan(kv_f16, hd, n_items, max_n, gqa, q4kv_part != nullptr,
                                    q4kv_part_cap);
    const uint32_t S = pl.S;
    const size_t need = S > 1u ? (size_t)n_items * S * gqa * PSTRIDE : 0u;
    if (need > Q4KV_SCRATCH_FLOATS) {
        Q4KV_ERR("qsa_step_batch_noalloc: %u items x %u splits need %zu floats of scratch, "
                 "the maximum is %u",
                 n_items, S, need, Q4KV_SCRATCH_FLOATS);
        return false;
    }
    return step_batch(d_descs, n_seq, n_head, n_kvh, hd, scale, kv_f16, max_n,
                      PartBuf{g_scratch_ptr[dev], Q4KV_SCRATCH_FLOATS});
}

#ifdef Q4KV_TRACE
extern "C" int q4kv_trace_read(uint64_t *host, size_t n) {
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(q4kv_trace_buf), n * sizeof(uint64_t), 0,
                               hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
extern "C" int q4kv_trace_read_band(uint64_t *host, size_t n) {
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(q4kv_trace_band), n * sizeof(uint64_t), 0,
                               hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif

extern "C" bool q4_hip_qsa_topk_alloc(void) {
    Q4KV_FLUSH_OR_FAIL(); return q4kv_ok && q4kv_part != nullptr; }

extern "C" bool q4_hip_qsa_step_prep_batch(const q4kv_prep_step_desc *d_descs, uint32_t n_seq,
                                           uint32_t n_head, uint32_t n_kvh, uint32_t hd,
                                           float scale, int kv_f16, uint32_t max_n,
                                           uint32_t n_rot, float rope_base, float eps) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d_descs || !n_seq || !max_n || !shape_ok(n_head, n_kvh, hd, kv_f16))
        return false;
    const uint32_t gqa = n_head / n_kvh;
    if (kv_f16 != Q4KV_Q8 || hd != 256u || !step_fusable(kv_f16, hd, gqa) || n_rot > hd) {
        Q4KV_ERR("qsa_step_prep_batch: needs a q8_0 cache, hd 256, gqa <= 16, n_rot <= hd");
        return false;
    }
    (void)hipGetLastError();
    AttnArgs a = base_args(nullptr, nullptr, nullptr, nullptr, nullptr, n_head, n_kvh, hd, 0,
                           scale);
    a.seqs = (const q4kv_seq_desc *)d_descs;
    a.desc_stride = sizeof(q4kv_prep_step_desc);
    a.n_rot = n_rot;
    a.rope_base = rope_base;
    a.eps = eps;
    return launch_kind<Q4KV_Q8, MODE_PSTEP>(a, n_seq * n_kvh, max_n, gqa);
}

extern "C" bool q4_hip_qsa_step_out_batch(const q4kv_step_desc *d_descs,
                                          const q4kv_out_desc *d_outs, uint32_t n_seq,
                                          uint32_t n_head, uint32_t n_kvh, uint32_t hd,
                                          float scale, int kv_f16, uint32_t max_n,
                                          uint32_t n_embd, float y_scale) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d_descs || !d_outs || !n_seq || !max_n || !n_embd ||
        !shape_ok(n_head, n_kvh, hd, kv_f16))
        return false;
    const uint32_t gqa = n_head / n_kvh;
    if (kv_f16 != Q4KV_Q8 || hd != 256u || !step_fusable(kv_f16, hd, gqa) || n_seq > 65535u) {
        Q4KV_ERR("qsa_step_out_batch: needs a q8_0 cache, hd 256, gqa <= 16");
        return false;
    }
    (void)hipGetLastError();
    AttnArgs a = base_args(nullptr, nullptr, nullptr, nullptr, nullptr, n_head, n_kvh, hd, 0,
                           scale);
    a.seqs = (const q4kv_seq_desc *)d_descs;
    a.desc_stride = sizeof(q4kv_step_desc);
    const OutProj op = {d_outs, n_embd, y_scale};
    return launch_kind<Q4KV_Q8, MODE_STEP>(a, n_seq * n_kvh, max_n, gqa, &op);
}
