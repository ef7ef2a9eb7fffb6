/*
 * q4kv_out.hip -- the attention output projection: the q8_0 GEMV
 * y = scale * W x of src/q4_fwd.c:925 (q4_hip_gemv_dd, src/q4_rocm.cu:
 * 4962-5005, 5536-5541, 1262-1285).
 *
 * Design: one wave per output row at a time, four rows per wave in flight.
 * Lane l owns 64-column pairs of q8_0 blocks p = l, l + 64, ... (68 bytes,
 * dword aligned, 17 dword loads). x is staged once per workgroup in LDS.
 * Each int8 is converted with v_cvt_f32_ubyte after flipping the sign bit
 * (q + 128 in 0..255), so a block's sum is S = sum (q + 128) x and the
 * result d * (S - 128 * X) uses the block's column sum X of x, computed
 * once per workgroup. The row sum is a wave reduction.
 */
#include "q4kv_internal.h"
#include "q4kv.h"

namespace {

constexpr uint32_t GV_RPW = 4;       /* rows per wave in flight */
constexpr uint32_t GV_MAXCOLS = 8192; /* x staged in LDS (32 KiB) */

__global__ __launch_bounds__(256) void gemv_q8_k(const uint8_t *w, const float *x, float *y,
                                                 uint32_t nrows, uint32_t ncols, float scale) {
    __shared__ __attribute__((aligned(16))) float xs[GV_MAXCOLS];
    __shared__ float xsum[GV_MAXCOLS / 32];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t nb = ncols / 32u;
    const uint32_t npair = ncols / 64u;
    const size_t rowb = (size_t)nb * 34u;
    const uint32_t r0 = (blockIdx.x * 4u + wave) * GV_RPW;
    /* 17 dwords (a block pair) of each of the wave's rows at pair p */
    uint32_t dw[GV_RPW][17];
    auto load_pair = [&](uint32_t p) {
#pragma unroll
        for (uint32_t j = 0; j < GV_RPW; j++) {
            const uint32_t r = min(r0 + j, nrows - 1u);
            const uint32_t *src = (const uint32_t *)(w + (size_t)r * rowb + 68u * p);
#pragma unroll
            for (int k = 0; k < 17; k++) dw[j][k] = ldg(src + k);
        }
    };
    /* x is loaded first, then the first pair's weights: x reaches LDS (its
     * wait does not cover the weights, issued later) and the block sums are
     * formed while the weights are in flight */
    constexpr uint32_t XPT = GV_MAXCOLS / 4u / 256u; /* four-float groups of x per thread */
    typedef float xf4 __attribute__((ext_vector_type(4)));
    xf4 xv[XPT];
#pragma unroll
    for (uint32_t k = 0; k < XPT; k++) {
        const uint32_t i = tid + 256u * k;
        xv[k] = ldg((const xf4 *)x + (i < ncols / 4u ? i : 0u));
    }
    __builtin_amdgcn_sched_barrier(0); /* keep the x loads ahead of the weights */
    load_pair(lane < npair ? lane : 0u);
    /* every index is inside xs (XPT x 256 float4 = GV_MAXCOLS floats); the
     * entries past ncols are not read */
#pragma unroll
    for (uint32_t k = 0; k < XPT; k++) ((xf4 *)xs)[tid + 256u * k] = xv[k];
    __syncthreads();
    for (uint32_t b = tid; b < nb; b += 256u) {
        float s = 0.f;
        for (int i = 0; i < 32; i++) s += xs[32u * b + i];
        xsum[b] = s;
    }
    __syncthreads();
    float acc[GV_RPW];
#pragma unroll
    for (uint32_t j = 0; j < GV_RPW; j++) acc[j] = 0.f;
    for (uint32_t p = lane; p < npair; p += 64u) {
        if (p != lane) load_pair(p);
        const float xa = xsum[2u * p], xb = xsum[2u * p + 1u];
#pragma unroll
        for (uint32_t j = 0; j < GV_RPW; j++) acc[j] += q4kv_q8_pair_dot(dw[j], xs, p, xa, xb);
    }
#pragma unroll
    for (uint32_t j = 0; j < GV_RPW; j++) {
        const float s = q4kv_wave_sum(acc[j]);
        if (lane == 0 && r0 + j < nrows) y[r0 + j] = s * scale;
    }
}

/* Rows whose length is an odd number of blocks: one block per lane, bytes
 * through 16-bit loads (the row stride is only 2-byte aligned). */
__global__ __launch_bounds__(256) void gemv_q8_any_k(const uint8_t *w, const float *x, float *y,
                                                     uint32_t nrows, uint32_t ncols,
                                                     float scale) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t r = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (r >= nrows) return;
    const uint32_t nb = ncols / 32u;
    const uint8_t *row = w + (size_t)r * nb * 34u;
    float acc = 0.f;
    for (uint32_t b = lane; b < nb; b += 64u) {
        const uint16_t *blk = (const uint16_t *)(row + 34u * b);
        const float d = __half2float(__ushort_as_half(ldg(blk)));
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint16_t v = ldg(blk + 1 + i);
            s = fmaf((float)(int8_t)(v & 0xffu), ldg(x + 32u * b + 2 * i), s);
            s = fmaf((float)(int8_t)(v >> 8), ldg(x + 32u * b + 2 * i + 1), s);
        }
        acc = fmaf(d, s, acc);
    }
    acc = q4kv_wave_sum(acc);
    if (lane == 0) y[r] = acc * scale;
}

} // namespace

/* q8_0 only (ggml type 8); other types return false. */
extern "C" bool q4_hip_gemv_dd(uint32_t ggml_type, const uint8_t *d_w, uint64_t nrows,
                               uint64_t ncols, const float *d_x, float *d_y, float scale) {
    Q4KV_FLUSH_OR_FAIL();
    if (!q4kv_ok || !d_w || !d_x || !d_y || nrows == 0 || ncols == 0) return false;
    if (ggml_type != 8u || ncols % 32u || nrows > 0xffffffffull || ncols > 0xffffffffull) {
        Q4KV_ERR("gemv_dd: only q8_0 rows of whole blocks are supported");
        return false;
    }
    (void)hipGetLastError();
    const bool fast = ncols % 64u == 0 && ncols <= GV_MAXCOLS && ((uintptr_t)d_w & 3u) == 0 &&
                      ((uintptr_t)d_x & 15u) == 0;
    if (fast) {
        const uint32_t rows_wg = 4u * GV_RPW;
        const uint64_t grid = (nrows + rows_wg - 1) / rows_wg;
        gemv_q8_k<<<(uint32_t)grid, 256, 0, q4kv_stream>>>(d_w, d_x, d_y, (uint32_t)nrows,
                                                           (uint32_t)ncols, scale);
    } else {
        if ((uintptr_t)d_w & 1u) return false;
        const uint64_t grid = (nrows + 3u) / 4u;
        gemv_q8_any_k<<<(uint32_t)grid, 256, 0, q4kv_stream>>>(d_w, d_x, d_y, (uint32_t)nrows,
                                                               (uint32_t)ncols, scale);
    }
    return q4kv_launch_ok("gemv_dd");
}
