/* bf16.c -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * float <-> bf16 as include/utils/bfloat16.hpp:18-45 defines it:
 *   - exponent all-ones: sign | 0x7F80 | (mantissa != 0 ? 1 : 0)
 *     (so every NaN becomes the single pattern 0x7F81 / 0xFF81),
 *   - exponent zero (zero or subnormal float): signed zero,
 *   - otherwise round to nearest, ties to even, on the 16 dropped bits, with the
 *     carry into the exponent, and overflow to signed infinity.
 * bf16 -> float is a 16-bit left shift (bfloat16.hpp:42-45).
 */
#include <string.h>

#include "oracle.h"

static uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

static float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

uint16_t or_f32_to_bf16(float f) {
    uint32_t bits = f2u(f);
    uint32_t sign = bits >> 31;
    uint32_t exponent = (bits >> 23) & 0xFFu;
    uint32_t mantissa = bits & 0x7FFFFFu;
    if (exponent == 0xFFu) /* inf / NaN: bfloat16.hpp:23-25 */
        return (uint16_t)((sign << 15) | 0x7F80u | (mantissa != 0 ? 1u : 0u));
    if (exponent == 0u) /* zero and subnormals flush to signed zero: :26-28 */
        return (uint16_t)(sign << 15);
    /* ties-to-even on the dropped half-word: :29-31 */
    uint32_t low = bits & 0xFFFFu;
    uint32_t up = (low > 0x8000u) || (low == 0x8000u && (mantissa & 0x10000u));
    uint32_t m7 = (mantissa >> 16) + up;
    uint32_t e8 = exponent;
    if (m7 >= 0x80u) { /* mantissa carry: :33-39 */
        e8 += 1;
        m7 = 0;
        if (e8 >= 0xFFu) return (uint16_t)((sign << 15) | 0x7F80u);
    }
    return (uint16_t)((sign << 15) | (e8 << 7) | m7);
}

float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

void or_f32_to_bf16_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = or_f32_to_bf16(src[i]);
}

void or_bf16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = or_bf16_to_f32(src[i]);
}
