/* quant_ref.c -- fp32<->fp16 conversion and the INT8 weight scheme, restated on the CPU.
 *
 * TEST INFRASTRUCTURE ONLY.
 *
 * fp16: IEEE binary16 with round-to-nearest-even, which is what the reference's upload
 * (__float2half, cuda/forward_cuda.cu:36) and its quantizer's fp16 view
 * (astype(float16).astype(float32), tools/quantize.py:108-109) both do.  Written from the IEEE 754
 * definition with integer arithmetic; pinned exhaustively against F16C in f16c_check.c.
 *
 * INT8 (tools/quantize.py:58-73), per output row n of W[N,K] (already fp16-rounded):
 *     absmax = max_k |w[n,k]|
 *     s[n]   = absmax == 0 ? 1.0f : fl32(absmax / 127)         (float32 division)
 *     q[n,k] = clamp(rint_half_even(fl32(w[n,k] / s[n])), -127, 127)
 * Dequantized value (tools/quantize.py:65, tools/dequant_check.py:65): fl32((float)q * s).
 * Build without -ffast-math: the division must be the correctly rounded float division, never a
 * multiply by a reciprocal, and rintf must round half to even.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t or_f32_to_f16(float f) {
    const uint32_t u = f32_bits(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t mag = u & 0x7fffffffu;
    if (mag >= 0x7f800000u) {
        if (mag == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);   /* infinity */
        /* NaN: keep the top 10 payload bits and force the quiet bit. */
        return (uint16_t)(sign | 0x7e00u | ((mag >> 13) & 0x03ffu));
    }
    const int bexp = (int)(mag >> 23);              /* biased float exponent */
    const uint32_t frac = mag & 0x007fffffu;
    if (bexp >= 113) {
        /* Normal half range (or overflow after rounding). 13 fraction bits are dropped. */
        uint32_t h = ((uint32_t)(bexp - 112) << 10) | (frac >> 13);
        const uint32_t rest = frac & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
        if (h >= 0x7c00u) h = 0x7c00u;              /* rounds to or past 65520 -> inf */
        return (uint16_t)(sign | h);
    }
    /* Result is subnormal or zero: value = sig * 2^(bexp-150), counted in units of 2^-24. */
    if (bexp < 102) return sign;                    /* below 2^-25: rounds to zero */
    const uint32_t sig = frac | 0x00800000u;
    const int shift = 126 - bexp;                   /* 14 .. 24 */
    uint32_t h = sig >> shift;
    const uint32_t rest = sig & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rest > halfway || (rest == halfway && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t m = (uint32_t)h & 0x03ffu;
    if (e == 0x1fu) {
        if (m == 0) return bits_f32(sign | 0x7f800000u);
        return bits_f32(sign | 0x7fc00000u | (m << 13));   /* NaN comes back quiet */
    }
    if (e != 0) return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return bits_f32(sign);
    /* subnormal: m * 2^-24, exact in float */
    const float v = (float)m * 5.9604644775390625e-08f;
    return sign ? -v : v;
}

void or_f32_to_f16_array(uint16_t *dst, const float *src, size_t n) {
    long i;
#pragma omp parallel for schedule(static)
    for (i = 0; i < (long)n; ++i) dst[i] = or_f32_to_f16(src[i]);
}

void or_f16_to_f32_array(float *dst, const uint16_t *src, size_t n) {
    long i;
#pragma omp parallel for schedule(static)
    for (i = 0; i < (long)n; ++i) dst[i] = or_f16_to_f32(src[i]);
}

/* tools/quantize.py:58-73 */
int or_quantize_rows(int8_t *q, float *s, const float *w16, int N, int K) {
    int dead = 0;
    int n;
#pragma omp parallel for schedule(static) reduction(+ : dead)
    for (n = 0; n < N; ++n) {
        const float *row = w16 + (size_t)n * K;
        float peak = 0.0f;
        for (int k = 0; k < K; ++k) {
            const float a = fabsf(row[k]);
            if (a > peak) peak = a;
        }
        const int is_dead = (peak == 0.0f);
        const float scale = is_dead ? 1.0f : peak / 127.0f;
        dead += is_dead;
        s[n] = scale;
        int8_t *qr = q + (size_t)n * K;
        for (int k = 0; k < K; ++k) {
            float r = rintf(row[k] / scale);
            if (r > 127.0f) r = 127.0f;
            if (r < -127.0f) r = -127.0f;
            qr[k] = (int8_t)r;
        }
    }
    return dead;
}

int or_quantize_fp16_view(int8_t *q, float *s, const float *w32, int N, int K) {
    /* tools/quantize.py:108-109: the fp16 values the engine runs, back in float32 */
    const size_t n = (size_t)N * (size_t)K;
    float *w16 = (float *)malloc(n * sizeof(float));
    long i;
#pragma omp parallel for schedule(static)
    for (i = 0; i < (long)n; ++i) w16[i] = or_f16_to_f32(or_f32_to_f16(w32[i]));
    const int dead = or_quantize_rows(q, s, w16, N, K);
    free(w16);
    return dead;
}

void or_dequantize(float *w, const int8_t *q, const float *s, int N, int K) {
    long n;
#pragma omp parallel for schedule(static)
    for (n = 0; n < N; ++n)
        for (int k = 0; k < K; ++k)
            w[(size_t)n * K + k] = (float)q[(size_t)n * K + k] * s[n];
}

/* Second implementation used only to cross-check or_quantize_rows: the quotient is formed in long
 * double and rounded to float afterwards (64-bit significand >= 2*24+2, so the double rounding is
 * exact for a quotient), and the half-even rounding is done by hand on the long double value. */
int or_quantize_rows_ld(int8_t *q, float *s, const float *w16, int N, int K) {
    int dead = 0;
    for (int n = 0; n < N; ++n) {
        const float *row = w16 + (size_t)n * K;
        long double peak = 0.0L;
        for (int k = 0; k < K; ++k) {
            long double a = row[k] < 0 ? -(long double)row[k] : (long double)row[k];
            if (a > peak) peak = a;
        }
        float scale;
        if (peak == 0.0L) {
            scale = 1.0f;
            ++dead;
        } else {
            scale = (float)(peak / 127.0L);
        }
        s[n] = scale;
        for (int k = 0; k < K; ++k) {
            const long double quot = (long double)(float)((long double)row[k] / (long double)scale);
            long double fl = floorl(quot);
            const long double frac = quot - fl;
            long double r;
            if (frac > 0.5L) r = fl + 1.0L;
            else if (frac < 0.5L) r = fl;
            else r = (fmodl(fl, 2.0L) == 0.0L) ? fl : fl + 1.0L;
            if (r > 127.0L) r = 127.0L;
            if (r < -127.0L) r = -127.0L;
            q[(size_t)n * K + k] = (int8_t)(int)r;
        }
    }
    return dead;
}
