/*
 * q4kv_synth.hip -- synthetic benchmark inputs generated on the device
 * (libq4kv_synth.so, used by bench.py only; not part of the KV-cache ABI).
 *
 * Rows of hd fp32 values ~N(0,1) (counter-based splitmix64 + Box-Muller, so
 * any element is reproducible from (seed, index)), with up to 4 outlier
 * channels per row scaled by 8.
 */
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

__device__ static inline uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void synth_heads_k(float *dst, uint64_t n, uint32_t hd, uint64_t seed, int o0,
                              int o1, int o2, int o3) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t h = mix64(seed ^ (i * 0xD1B54A32D192ED03ull));
        const float u1 = ((float)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);
        const float u2 = (float)((h >> 8) & 0xFFFFFFu) * (1.0f / 16777216.0f);
        float x = sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
        const int c = (int)(i % hd);
        if (c == o0 || c == o1 || c == o2 || c == o3) x *= 8.0f;
        dst[i] = x;
    }
}

extern "C" int q4kv_synth_heads(float *dst, uint64_t n, uint32_t hd, uint64_t seed, int o0,
                                int o1, int o2, int o3) {
    if (!dst || !n || !hd) return -1;
    synth_heads_k<<<4096, 256>>>(dst, n, hd, seed, o0, o1, o2, o3);
    if (hipGetLastError() != hipSuccess) return -1;
    return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}

/* Gather-ceiling probe: the row traffic of a q8_0 hd-256 decode batch with no
 * compute at all. Each workgroup DMAs the K and V rows of 64 list entries of
 * one (item, kv head) into LDS (16-byte global_load_lds, like the attention
 * kernel) and exits; items are described by q4kv_seq_desc-compatible
 * (kcache, vcache, idx, n_sel, idx_kvh_stride) fields passed as arrays. */
#define GLOBAL __attribute__((address_space(1)))
#define LOCAL __attribute__((address_space(3)))
__global__ __launch_bounds__(256) void gather_probe_k(const uint8_t *const *kc,
                                                      const uint8_t *const *vc,
                                                      const int32_t *const *idx, uint32_t width,
                                                      uint32_t n_kvh, float *sink) {
    constexpr uint32_t CP = 64, ROWB = 272, NCH = 17, TOT = CP * NCH;
    __shared__ __attribute__((aligned(16))) uint8_t kr[CP * ROWB], vr[CP * ROWB];
    const uint32_t item = blockIdx.y, seq = item / n_kvh, kh = item % n_kvh;
    const uint8_t *kb = kc[seq] + kh * ROWB, *vb = vc[seq] + kh * ROWB;
    const int32_t *ix = idx[seq] + kh * width;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, base = blockIdx.x * CP;
    for (uint32_t e0 = wave * 64u; e0 < TOT; e0 += 256u) {
        const uint32_t e = e0 + lane;
        if (e < TOT) {
            const uint32_t r = e / NCH, q = e - r * NCH;
            const uint32_t j = base + r < width ? base + r : width - 1u;
            const size_t off = (size_t)ix[j] * n_kvh * ROWB + q * 16u;
            __builtin_amdgcn_global_load_lds((const GLOBAL void *)(kb + off),
                                             (LOCAL void *)(kr + e0 * 16u), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const GLOBAL void *)(vb + off),
                                             (LOCAL void *)(vr + e0 * 16u), 16, 0, 0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.y * gridDim.x + blockIdx.x] = kr[lane] + vr[lane];
}

/* Runs iters launches, rotating over n_sets (kc, vc, idx) pointer tables of
 * n_seq entries each (device arrays laid out [set][seq]); returns the mean
 * microseconds per launch (event-timed), or -1. */
extern "C" double q4kv_gather_probe_us(const void *const *d_kc, const void *const *d_vc,
                                       const int32_t *const *d_idx, uint32_t n_seq,
                                       uint32_t n_sets, uint32_t n_kvh, uint32_t width,
                                       int iters) {
    float *sink = nullptr;
    hipEvent_t e0, e1;
    if (hipMalloc(&sink, 1u << 20) != hipSuccess) return -1.0;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0;
    dim3 grid((width + 63u) / 64u, n_seq * n_kvh);
    for (int w = 0; w < 3; w++)
        gather_probe_k<<<grid, 256>>>((const uint8_t *const *)d_kc, (const uint8_t *const *)d_vc,
                                      d_idx, width, n_kvh, sink);
    (void)hipEventRecord(e0, 0);
    for (int i = 0; i < iters; i++) {
        const size_t o = (size_t)(i % n_sets) * n_seq;
        gather_probe_k<<<grid, 256>>>((const uint8_t *const *)d_kc + o,
                                      (const uint8_t *const *)d_vc + o, d_idx + o, width, n_kvh,
                                      sink);
    }
    (void)hipEventRecord(e1, 0);
    (void)hipEventSynchronize(e1);
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipFree(sink);
    return hipGetLastError() == hipSuccess ? 1000.0 * ms / iters : -1.0;
}
