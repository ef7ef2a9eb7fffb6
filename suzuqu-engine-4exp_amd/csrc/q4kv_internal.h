/*
 * q4kv_internal.h -- state shared by the library's HIP translation units.
 * Not part of the public ABI (that is include/q4kv.h).
 */
#ifndef Q4KV_INTERNAL_H
#define Q4KV_INTERNAL_H
#include <hip/hip_runtime.h>
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

#define GLOBAL __attribute__((address_space(1)))
#define LOCAL __attribute__((address_space(3)))
/* Loads/stores through the global address space: pointers taken from
 * argument structs and descriptors would otherwise compile to flat
 * accesses, whose waits also cover LDS traffic. */
template <class T> __device__ static inline T ldg(const T *p) { return *(const GLOBAL T *)p; }
template <class T> __device__ static inline void stg(T *p, T v) { *(GLOBAL T *)p = v; }

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
