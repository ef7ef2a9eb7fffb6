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
