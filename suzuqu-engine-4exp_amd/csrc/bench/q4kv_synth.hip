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
