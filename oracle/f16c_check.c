/*
 * f16c_check.c -- TEST INFRASTRUCTURE ONLY. Cross-checks the oracle's
 * binary16 encoder against the x86 F16C instruction (vcvtps2ph, RNE), an
 * independent hardware implementation of IEEE-754 float->half conversion.
 */
#include <immintrin.h>
#include <stdint.h>
#include <string.h>

uint16_t orc_f16_from_f32(float x);

/* Number of non-NaN float bit patterns u = start + i*step (i < count) whose
 * oracle encoding differs from F16C's. */
uint64_t orc_check_f16c(uint64_t start, uint64_t count, uint64_t step) {
    uint64_t bad = 0;
    for (uint64_t i = 0; i < count; i++) {
        uint32_t u = (uint32_t)(start + i * step);
        if ((u & 0x7fffffffu) > 0x7f800000u) continue;
        float x;
        memcpy(&x, &u, 4);
        uint16_t hw = (uint16_t)_cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT);
        if (hw != orc_f16_from_f32(x)) bad++;
    }
    return bad;
}
