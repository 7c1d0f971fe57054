/* f16c_check.c -- pins or_f32_to_f16 / or_f16_to_f32 against the x86 F16C instructions.
 *
 * TEST INFRASTRUCTURE ONLY.  VCVTPS2PH with imm8 = 0 rounds to nearest even regardless of MXCSR;
 * VCVTPH2PS is exact.  F16C is an implementation independent of quant_ref.c, so agreement over every
 * 32-bit pattern is a known-answer test of the restated conversion.  Compiled with -mf16c.
 */
#include "oracle.h"

#include <immintrin.h>
#include <string.h>

uint64_t or_check_f16c_range(uint64_t lo, uint64_t hi, uint32_t *first) {
    uint64_t bad = 0;
    uint64_t first_bad = UINT64_MAX;
    long long i;
#pragma omp parallel for schedule(static) reduction(+ : bad) reduction(min : first_bad)
    for (i = (long long)lo; i < (long long)hi; i += 8) {
        uint32_t pat[8];
        float f[8];
        for (int j = 0; j < 8; ++j) pat[j] = (uint32_t)(i + j);
        memcpy(f, pat, sizeof f);
        const __m128i hw = _mm256_cvtps_ph(_mm256_loadu_ps(f), 0);
        uint16_t h[8];
        _mm_storeu_si128((__m128i *)h, hw);
        for (int j = 0; j < 8 && (uint64_t)(i + j) < hi; ++j) {
            if (or_f32_to_f16(f[j]) != h[j]) {
                ++bad;
                if ((uint64_t)(i + j) < first_bad) first_bad = (uint64_t)(i + j);
            }
        }
    }
    if (first) *first = (uint32_t)(first_bad == UINT64_MAX ? 0 : first_bad);
    return bad;
}

uint64_t or_check_f16c_back(void) {
    uint64_t bad = 0;
    for (uint32_t i = 0; i < 65536; ++i) {
        const float hw = _cvtsh_ss((unsigned short)i);
        const float sw = or_f16_to_f32((uint16_t)i);
        uint32_t a, b;
        memcpy(&a, &hw, 4);
        memcpy(&b, &sw, 4);
        if (a != b) ++bad;
    }
    return bad;
}
