/*
 * q4kv_internal.h -- state shared by the library's HIP translation units.
 * Not part of the public ABI (that is include/q4kv.h).
 */
#ifndef Q4KV_INTERNAL_H
#define Q4KV_INTERNAL_H
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>

/* The single compute stream every q4_hip_* launch is enqueued on. It is a
 * non-blocking stream at the default priority so it can be captured into a
 * hipGraph. */
extern hipStream_t q4kv_stream;
extern int q4kv_ok;
extern int q4kv_capturing;
/* Device-side decode position (one int32) read by the *_d entry points. */
extern int32_t *q4kv_pos_d;
/* Library-owned split-KV partial buffer (floats) and its capacity. */
extern float *q4kv_part;
extern size_t q4kv_part_cap;

/* A held q4_hip_kv_append_d: the append of one token's K/V rows at the
 * device position, recorded instead of launched. A one-token decode on the
 * same caches performs it inside its own launch; any other library call
 * first launches it (q4kv_flush), so every caller of the library sees the
 * same stream order as if it had been launched at once. */
struct q4kv_held_append {
    int on;
    uint8_t *kc, *vc;
    const float *k, *v;
    uint32_t n, bpt;
    int kind;
};
extern q4kv_held_append q4kv_held;
/* Launch the held append, if any. False if that launch failed. */
bool q4kv_flush(void);
#define Q4KV_FLUSH_OR_FAIL()                                                   \
    do {                                                                       \
        if (!q4kv_flush()) return false;                                       \
    } while (0)

/* Resolves the no-allocation entry point's static scratch on the current
 * device (q4kv_attn.hip); q4_hip_init calls it once. */
extern "C" bool q4kv_scratch_init(void);


/* The append half of q4_hip_qsa_step_batch for widths the fused kernel
 * does not cover: d_step_descs is a device array of q4kv_step_desc. */
bool q4kv_append_steps(const void *d_step_descs, uint32_t n_desc, uint32_t n, uint32_t bpt,
                       int kind);

#define GLOBAL __attribute__((address_space(1)))
#define LOCAL __attribute__((address_space(3)))
/* Loads/stores through the global address space: pointers taken from
 * argument structs and descriptors would otherwise compile to flat
 * accesses, whose waits also cover LDS traffic. */
template <class T> __device__ static inline T ldg(const T *p) { return *(const GLOBAL T *)p; }
template <class T> __device__ static inline void stg(T *p, T v) { *(GLOBAL T *)p = v; }
/* A pointer read from device memory (a descriptor field) is a generic
 * pointer: accesses through it compile to flat memory instructions, which
 * also count against lgkmcnt. Built from the field's integer value as a
 * global-address-space pointer instead, it lets the compiler use global
 * instructions for every access through it. */
template <class T> __device__ static inline T *q4kv_gptr(uintptr_t v) { return (T *)(GLOBAL T *)v; }
template <class T> __device__ static inline T *q4kv_gptr_at(T *const *field) {
    return q4kv_gptr<T>(ldg((const uintptr_t *)field));
}

/* One lane's share of a q8_0 block (src/q4_rocm.cu:7221-7238): lanes 8k ..
 * 8k+7 of a wave hold the block's 32 values, four each (lane part p holds
 * values 4p .. 4p+3). Returns the block scale d = amax / 127 and this lane's
 * four int8 q = clamp(rint(x / d), -127, 127), in IEEE binary32 with
 * round-to-nearest-even (explicitly rounded divide and multiply). */
__device__ static inline float q8_lane_quant(float x0, float x1, float x2, float x3,
                                             int (&q)[4]) {
    float a = fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(x2), fabsf(x3)));
    a = fmaxf(a, __shfl_xor(a, 1, 8));
    a = fmaxf(a, __shfl_xor(a, 2, 8));
    a = fmaxf(a, __shfl_xor(a, 4, 8));
    const float d = __fdiv_rn(a, 127.f);
    const float id = d > 0.f ? __fdiv_rn(1.f, d) : 0.f;
    const float xs[4] = {x0, x1, x2, x3};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int v = (int)__builtin_rintf(__fmul_rn(xs[i], id));
        v = v > 127 ? 127 : v;
        v = v < -127 ? -127 : v;
        q[i] = v;
    }
    return d;
}
/* Store a lane's share into its 34-byte block (fp16 scale, then 32 int8);
 * the payload starts 2 bytes in, so 16-bit stores. */
__device__ static inline void q8_lane_store(uint8_t *blk, uint32_t part, float d,
                                            const int (&q)[4]) {
    *(uint16_t *)(blk + 2u + part * 4u) = (uint16_t)((q[0] & 0xff) | ((q[1] & 0xff) << 8));
    *(uint16_t *)(blk + 4u + part * 4u) = (uint16_t)((q[2] & 0xff) | ((q[3] & 0xff) << 8));
    if (part == 0) *(uint16_t *)blk = __half_as_ushort(__float2half_rn(d));
}

typedef float q4kv_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t q4kv_u4 __attribute__((ext_vector_type(4)));
#define QBLK_PER_WG 32u /* 256 threads / 8 lanes per block */

/* Quantise q8_0 blocks [blk0, blk0 + 32) of src into dst (block-indexed) with
 * one 256-thread workgroup; the 1088 output bytes are assembled in LDS and
 * written as 16-byte stores where dst allows. */
__device__ static inline void q8_quant_wg(const float *__restrict__ src,
                                          uint8_t *__restrict__ dst, uint64_t nblocks,
                                          uint64_t blk0, bool src_al16, bool dst_al16) {
    __shared__ __attribute__((aligned(16))) uint8_t ob[QBLK_PER_WG * 34u];
    const uint32_t t = threadIdx.x, lb = t >> 3, part = t & 7u;
    const uint64_t b = blk0 + lb;
    const bool live = b < nblocks;
    float x0 = 0.f, x1 = 0.f, x2 = 0.f, x3 = 0.f;
    if (live) {
        const float *p = src + b * 32u + part * 4u;
        if (src_al16) {
            const q4kv_f4 v = ldg((const q4kv_f4 *)p);
            x0 = v[0]; x1 = v[1]; x2 = v[2]; x3 = v[3];
        } else {
            x0 = ldg(p); x1 = ldg(p + 1); x2 = ldg(p + 2); x3 = ldg(p + 3);
        }
    }
    int q[4];
    const float d = q8_lane_quant(x0, x1, x2, x3, q);
    q8_lane_store(ob + lb * 34u, part, d, q);
    __syncthreads();
    const uint64_t nb = nblocks - blk0 < QBLK_PER_WG ? nblocks - blk0 : QBLK_PER_WG;
    uint8_t *out = dst + blk0 * 34u;
    if (dst_al16 && nb == QBLK_PER_WG) {
        if (t < QBLK_PER_WG * 34u / 16u) stg((q4kv_u4 *)out + t, ((const q4kv_u4 *)ob)[t]);
    } else {
        for (uint32_t i = t; i < nb * 34u; i += blockDim.x) stg(out + i, ob[i]);
    }
}

/* A held append carried by another launch: workgroups w < wgs of the
 * carrying range write the K rows, wgs <= w < 2 wgs the V rows, q8_0 at the
 * device position (n values per cache, 32 blocks per workgroup), as the
 * append kernel itself would. */
struct q4kv_app_args {
    const float *k, *v;
    uint8_t *kc, *vc;
    const int32_t *pp;
    uint32_t n, bpt, wgs;
};
__device__ static inline void q4kv_app_wg(const q4kv_app_args &a, uint32_t w) {
    const bool isv = w >= a.wgs;
    const float *src = isv ? a.v : a.k;
    uint8_t *dst = (isv ? a.vc : a.kc) + (size_t)(uint32_t)ldg(a.pp) * a.bpt;
    q8_quant_wg(src, dst, a.n / 32u, (uint64_t)(isv ? w - a.wgs : w) * QBLK_PER_WG,
                ((uintptr_t)src & 15u) == 0, ((uintptr_t)dst & 15u) == 0);
}
/* Hands the held append (if any) to a launch that carries it and clears the
 * hold: returns the number of extra workgroups it needs (0: none held). */
uint32_t q4kv_take_held(q4kv_app_args *a);

/* ---- shared wave-level arithmetic of the Q/K preparation ---- */
template <int CTRL> __device__ static inline float q4kv_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
/* Sum over the 8-lane group containing this lane, broadcast to all 8. */
__device__ static inline float q4kv_sum8(float v) {
    v += q4kv_dpp<0xB1>(v);  /* quad_perm [1,0,3,2] */
    v += q4kv_dpp<0x4E>(v);  /* quad_perm [2,3,0,1] */
    v += q4kv_dpp<0x141>(v); /* row_half_mirror: lane i <-> 7-i */
    return v;
}
__device__ static inline float q4kv_wave_sum(float v) {
    v = q4kv_sum8(v);
    v += q4kv_dpp<0x140>(v); /* row_mirror: the other half of the 16-lane row */
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}
/* fp32 RoPE frequency base^(-(p/np)) with the exponent an fp32 quotient
 * (src/q4_rocm.cu:6255, 7391), correctly rounded: pow in double, rounded once.
 * At positions near 2^18 one ulp of freq moves the angle by ~0.016 rad, so the
 * frequency is not left to an approximate powf. */
__device__ static inline float q4kv_rope_freq(float base, uint32_t p, uint32_t np) {
    const float e = -__fdiv_rn((float)p, (float)np);
    return (float)pow((double)base, (double)e);
}
/* Rotate (x0, x1) by the fp32 angle pos * freq (one fp32 rounding, as the
 * reference forms it). */
__device__ static inline void q4kv_rope_rotate(float &x0, float &x1, float pos_f, float freq) {
    const float ang = __fmul_rn(pos_f, freq);
    float s, c;
    sincosf(ang, &s, &c);
    const float a = x0, b = x1;
    x0 = a * c - b * s;
    x1 = a * s + b * c;
}
constexpr uint32_t Q4KV_PREP_MAXP = 8; /* pairs per lane: hd <= 1024 */
/* One (token, head) row by one wave (src/q4_rocm.cu:6229-6289): RMSNorm
 * times wn (NULL = 1), then RoPE of pairs p < n_rot/2 at position pos.
 * Lane l owns pairs p = l + 64m; in and out may alias (every lane reads its
 * pairs before the reduction). Every kernel that prepares rows calls this,
 * so their results agree bit for bit. */
__device__ static inline __attribute__((always_inline)) void q4kv_prep_row(const float *in, float *out, const float *wn,
                                            uint32_t hd, uint32_t n_rot, int32_t pos,
                                            float base, float eps, uint32_t lane) {
    const uint32_t np = hd / 2;
    float2 x[Q4KV_PREP_MAXP];
    float ss = 0.f;
#pragma unroll
    for (uint32_t m = 0; m < Q4KV_PREP_MAXP; m++) {
        const uint32_t p = lane + 64u * m;
        x[m] = p < np ? make_float2(in[2 * p], in[2 * p + 1]) : make_float2(0.f, 0.f);
        ss = fmaf(x[m].x, x[m].x, ss);
        ss = fmaf(x[m].y, x[m].y, ss);
    }
    ss = q4kv_wave_sum(ss);
    const float scale = __fdiv_rn(1.f, __fsqrt_rn(__fdiv_rn(ss, (float)hd) + eps));
    const uint32_t nrp = n_rot / 2;
#pragma unroll
    for (uint32_t m = 0; m < Q4KV_PREP_MAXP; m++) {
        const uint32_t p = lane + 64u * m;
        if (p >= np) continue;
        const float w0 = wn ? wn[2 * p] : 1.f, w1 = wn ? wn[2 * p + 1] : 1.f;
        float y0 = x[m].x * scale * w0, y1 = x[m].y * scale * w1;
        if (p < nrp) q4kv_rope_rotate(y0, y1, (float)pos, q4kv_rope_freq(base, p, nrp));
        out[2 * p] = y0;
        out[2 * p + 1] = y1;
    }
}

/* byte k of w as a float (one v_cvt_f32_ubyte<k>) */
__device__ static inline float q4kv_ubyte_f(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xffu); }

/* sum over the 4 biased bytes of w times x[0..3] */
__device__ static inline float q4kv_dot4(uint32_t w, const float4 &x, float acc) {
    w ^= 0x80808080u;
    acc = fmaf(q4kv_ubyte_f(w, 0), x.x, acc);
    acc = fmaf(q4kv_ubyte_f(w, 1), x.y, acc);
    acc = fmaf(q4kv_ubyte_f(w, 2), x.z, acc);
    acc = fmaf(q4kv_ubyte_f(w, 3), x.w, acc);
    return acc;
}

/* One pair of q8_0 blocks (68 bytes as 17 dwords: blocks 2p, 2p+1 of a
 * row) against x columns 64p .. 64p+63 (in LDS), given the two blocks'
 * column sums xa, xb of x: d_a * sum(q x) + d_b * sum(q x). Each int8 is
 * converted with v_cvt_f32_ubyte after flipping the sign bit (q + 128), and
 * the block result is d * (S - 128 X). */
__device__ static inline float q4kv_q8_pair_dot(const uint32_t (&dw)[17], const float *xs, uint32_t p,
                                 float xa, float xb) {
    const float4 *x4 = (const float4 *)(xs + 64u * p);
    /* block A: fp16 d in bytes 0-1, quants in bytes 2..33 */
    const float da = __half2float(__ushort_as_half((unsigned short)(dw[0] & 0xffffu)));
    float sa = 0.f;
    /* quants 0,1 are the high half of dw0; 2..29 in dw1..dw7; 30,31 low half of dw8 */
    {
        const uint32_t w0 = __builtin_amdgcn_perm(dw[1], dw[0], 0x05040302u); /* q0 q1 q2 q3 */
        sa = q4kv_dot4(w0, x4[0], sa);
#pragma unroll
        for (int k = 1; k < 8; k++) {
            const uint32_t wk = __builtin_amdgcn_perm(dw[k + 1], dw[k], 0x05040302u);
            sa = q4kv_dot4(wk, x4[k], sa);
        }
    }
    const float db = __half2float(__ushort_as_half((unsigned short)(dw[8] >> 16)));
    float sb = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) sb = q4kv_dot4(dw[9 + k], x4[8 + k], sb);
    return da * (sa - 128.f * xa) + db * (sb - 128.f * xb);
}

#define Q4KV_ERR(...)                                                          \
    do {                                                                       \
        fprintf(stderr, "q4 hip: " __VA_ARGS__);                               \
        fputc('\n', stderr);                                                   \
    } while (0)

/* Drain and report a launch error. Returns true when the last launch was ok. */
static inline bool q4kv_launch_ok(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        Q4KV_ERR("%s launch: %s", what, hipGetErrorString(e));
        return false;
    }
    return true;
}
#endif
