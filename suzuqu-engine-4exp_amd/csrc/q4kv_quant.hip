/*
 * q4kv_quant.hip -- KV-cache write kernels: fp32 -> q8_0 / fp16 / fp32 rows.
 *
 * q8_0 block format (src/q4_rocm.cu:7221-7238): 32 values per block, 34 bytes:
 * a little-endian fp16 scale d = fp16(amax / 127) followed by 32 int8
 * q = clamp(rint(x * (1/d)), -127, 127). The arithmetic here is IEEE
 * binary32 with round-to-nearest-even everywhere (explicitly rounded divide,
 * no contraction), so the bytes equal the source semantics of the reference
 * kernel bit for bit.
 *
 * Layout on gfx950: 8 lanes cooperate on one block (one float4 each, so a
 * wave reads 1 KiB of contiguous input), the block's absolute max is reduced
 * across the 8 lanes, and a workgroup's 32 output blocks (1088 bytes) are
 * assembled in LDS and written back as 68 coalesced 16-byte stores.
 */
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdlib.h>

#include "q4kv_internal.h"

extern "C" {
#include "q4kv.h"
}


__global__ __launch_bounds__(256) static void f32_to_q8_k(const float *__restrict__ src,
                                                          uint8_t *__restrict__ dst,
                                                          uint64_t nblocks, int src_al16,
                                                          int dst_al16) {
    q8_quant_wg(src, dst, nblocks, (uint64_t)blockIdx.x * QBLK_PER_WG, src_al16 != 0,
                dst_al16 != 0);
}

/* fp16 width: RNE per element (src/q4_rocm.cu:7208-7211), 4 per thread. */
__global__ __launch_bounds__(256) static void f32_to_f16_k(const float *__restrict__ src,
                                                           __half *__restrict__ dst,
                                                           uint64_t n, int vec) {
    const uint64_t i4 = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4u;
    if (i4 >= n) return;
    if (vec && i4 + 4u <= n) {
        float4 v = *(const float4 *)(src + i4);
        uint2 o;
        o.x = (uint32_t)__half_as_ushort(__float2half_rn(v.x)) |
              ((uint32_t)__half_as_ushort(__float2half_rn(v.y)) << 16);
        o.y = (uint32_t)__half_as_ushort(__float2half_rn(v.z)) |
              ((uint32_t)__half_as_ushort(__float2half_rn(v.w)) << 16);
        *(uint2 *)(dst + i4) = o;
    } else {
        for (uint64_t i = i4; i < n && i < i4 + 4u; i++) dst[i] = __float2half_rn(src[i]);
    }
}

/* Device-position append of one token's K and V rows (n floats each) into
 * caches with bpt bytes per token (src/q4_rocm.cu:7962-8012). grid.y = 0
 * writes K, 1 writes V. The position is read from device memory so the
 * launch can sit in a captured graph and replay for every token. */
__global__ __launch_bounds__(256) static void kv_append_k(const float *__restrict__ k,
                                                          const float *__restrict__ v,
                                                          uint8_t *kc, uint8_t *vc, uint32_t n,
                                                          uint32_t bpt, int kind,
                                                          const int32_t *__restrict__ pp) {
    const size_t off = (size_t)(uint32_t)*pp * bpt;
    const float *src = blockIdx.y ? v : k;
    uint8_t *dst = (blockIdx.y ? vc : kc) + off;
    if (kind == Q4KV_Q8) {
        const bool s_al = ((uintptr_t)src & 15u) == 0;
        const bool d_al = ((uintptr_t)dst & 15u) == 0;
        q8_quant_wg(src, dst, n / 32u, (uint64_t)blockIdx.x * QBLK_PER_WG, s_al, d_al);
    } else {
        for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n;
             i += gridDim.x * blockDim.x) {
            if (kind == Q4KV_F16)
                ((__half *)dst)[i] = __float2half_rn(src[i]);
            else
                ((float *)dst)[i] = src[i];
        }
    }
}

/* One launch appending a token's rows into several caches (layers or
 * sequences): grid.z selects the descriptor. Each descriptor carries its own
 * caches, fp32 rows and token position, so no device position is needed.
 * STEP: the descriptors are q4kv_step_desc (the append half of a decode
 * step), otherwise q4kv_append_desc. */
template <bool STEP>
__global__ __launch_bounds__(256) static void kv_append_batch_k(const void *__restrict__ dsv,
                                                                uint32_t n, uint32_t bpt, int kind) {
    const float *kf, *vf;
    uint8_t *kc, *vc;
    uint32_t pos;
    if (STEP) {
        const q4kv_step_desc *d = (const q4kv_step_desc *)dsv + blockIdx.z;
        kf = ldg(&d->k);
        vf = ldg(&d->v);
        kc = (uint8_t *)ldg(&d->seq.kcache);
        vc = (uint8_t *)ldg(&d->seq.vcache);
        pos = ldg(&d->pos);
    } else {
        const q4kv_append_desc *d = (const q4kv_append_desc *)dsv + blockIdx.z;
        kf = ldg(&d->k);
        vf = ldg(&d->v);
        kc = (uint8_t *)ldg(&d->kcache);
        vc = (uint8_t *)ldg(&d->vcache);
        pos = ldg(&d->pos);
    }
    const size_t off = (size_t)pos * bpt;
    const float *src = blockIdx.y ? vf : kf;
    uint8_t *dst = (blockIdx.y ? vc : kc) + off;
    if (kind == Q4KV_Q8) {
        const bool s_al = ((uintptr_t)src & 15u) == 0;
        const bool d_al = ((uintptr_t)dst & 15u) == 0;
        q8_quant_wg(src, dst, n / 32u, (uint64_t)blockIdx.x * QBLK_PER_WG, s_al, d_al);
    } else {
        for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n;
             i += gridDim.x * blockDim.x) {
            if (kind == Q4KV_F16)
                stg((uint16_t *)dst + i, __half_as_ushort(__float2half_rn(ldg(src + i))));
            else
                stg((float *)dst + i, ldg(src + i));
        }
    }
}

static bool append_batch(const void *d_descs, bool step, uint32_t n_desc, uint32_t n,
                         uint32_t bpt, int kind) {
    if (!q4kv_ok || !d_descs || !n_desc || !n || !bpt || n_desc > 65535u) return false;
    if (kind < Q4KV_F32 || kind > Q4KV_Q8) return false;
    if (kind == Q4KV_Q8 && (n % 32u)) return false;
    (void)hipGetLastError();
    const uint32_t gx = kind == Q4KV_Q8 ? (n / 32u + QBLK_PER_WG - 1) / QBLK_PER_WG
                                        : (n + 255u) / 256u;
    if (step)
        kv_append_batch_k<true><<<dim3(gx, 2, n_desc), 256, 0, q4kv_stream>>>(d_descs, n, bpt, kind);
    else
        kv_append_batch_k<false><<<dim3(gx, 2, n_desc), 256, 0, q4kv_stream>>>(d_descs, n, bpt, kind);
    return q4kv_launch_ok("kv_append_batch");
}

bool q4kv_append_steps(const void *d_step_descs, uint32_t n_desc, uint32_t n, uint32_t bpt,
                       int kind) {
    return append_batch(d_step_descs, true, n_desc, n, bpt, kind);
}

extern "C" bool q4_hip_kv_append_batch(const q4kv_append_desc *d_descs, uint32_t n_desc,
                                       uint32_t n, uint32_t bpt, int kind) {
    Q4KV_FLUSH_OR_FAIL();
    return append_batch(d_descs, false, n_desc, n, bpt, kind);
}

extern "C" bool q4_hip_f32_to_q8(void *dst_q8, const float *src, uint64_t n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !dst_q8 || !src || n == 0 || (n % 32u) != 0) return false;
    (void)hipGetLastError();
    const uint64_t nb = n / 32u;
    const uint64_t grid = (nb + QBLK_PER_WG - 1) / QBLK_PER_WG;
    if (grid > 0x7fffffffull) return false;
    f32_to_q8_k<<<(uint32_t)grid, 256, 0, q4kv_stream>>>(
        src, (uint8_t *)dst_q8, nb, ((uintptr_t)src & 15u) == 0,
        ((uintptr_t)dst_q8 & 15u) == 0);
    return q4kv_launch_ok("f32_to_q8");
}

extern "C" bool q4_hip_f32_to_f16(void *dst_f16, const float *src, uint64_t n) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !dst_f16 || !src || !n) return false;
    (void)hipGetLastError();
    const uint64_t threads = (n + 3u) / 4u;
    const uint64_t grid = (threads + 255u) / 256u;
    if (grid > 0x7fffffffull) return false;
    const int vec = ((uintptr_t)src & 15u) == 0 && ((uintptr_t)dst_f16 & 7u) == 0;
    f32_to_f16_k<<<(uint32_t)grid, 256, 0, q4kv_stream>>>(src, (__half *)dst_f16, n, vec);
    return q4kv_launch_ok("f32_to_f16");
}

static bool append_launch(uint8_t *kc, uint8_t *vc, const float *k, const float *v, uint32_t n,
                          uint32_t bpt, int kind) {
    (void)hipGetLastError();
    uint32_t gx;
    if (kind == Q4KV_Q8)
        gx = (n / 32u + QBLK_PER_WG - 1) / QBLK_PER_WG;
    else
        gx = (n + 255u) / 256u;
    dim3 grid(gx, 2);
    kv_append_k<<<grid, 256, 0, q4kv_stream>>>(k, v, kc, vc, n, bpt, kind, q4kv_pos_d);
    return q4kv_launch_ok("kv_append");
}

q4kv_held_append q4kv_held = {};

bool q4kv_flush(void) {
    if (!q4kv_held.on) return true;
    q4kv_held.on = 0;
    return append_launch(q4kv_held.kc, q4kv_held.vc, q4kv_held.k, q4kv_held.v, q4kv_held.n,
                         q4kv_held.bpt, q4kv_held.kind);
}

uint32_t q4kv_take_held(q4kv_app_args *a) {
    if (!q4kv_held.on) return 0;
    q4kv_held.on = 0;
    const uint32_t wgs = (q4kv_held.n / 32u + QBLK_PER_WG - 1) / QBLK_PER_WG;
    *a = q4kv_app_args{q4kv_held.k,  q4kv_held.v, q4kv_held.kc,  q4kv_held.vc,
                       q4kv_pos_d,   q4kv_held.n, q4kv_held.bpt, wgs};
    return 2u * wgs;
}

/* Q4KV_HOLD_APPEND=0 launches every append at once (no held append). */
static bool hold_enabled(void) {
    static int v = -1;
    if (v < 0) {
        const char *e = getenv("Q4KV_HOLD_APPEND");
        v = (e && e[0] == '0') ? 0 : 1;
    }
    return v != 0;
}

/* src/q4_rocm.cu:7962-8012. A q8_0 append of whole 256-dim head rows is held
 * (q4kv_held) for the next library call: a one-token decode over the same
 * caches performs it in its own launch, any other call launches it first. */
extern "C" bool q4_hip_kv_append_d(void *kcache, void *vcache, const float *k,
                                   const float *v, uint32_t n, uint32_t bpt, int kind) {
    if (!q4kv_ok || !q4kv_pos_d || !kcache || !vcache || !k || !v || !n || !bpt)
        return false;
    if (kind < Q4KV_F32 || kind > Q4KV_Q8) return false;
    if (kind == Q4KV_Q8 && (n % 32u)) return false;
    Q4KV_FLUSH_OR_FAIL();
    if (kind == Q4KV_Q8 && n % 256u == 0u && bpt == n / 256u * 272u && hold_enabled()) {
        q4kv_held = q4kv_held_append{1, (uint8_t *)kcache, (uint8_t *)vcache, k, v, n, bpt, kind};
        return true;
    }
    return append_launch((uint8_t *)kcache, (uint8_t *)vcache, k, v, n, bpt, kind);
}
