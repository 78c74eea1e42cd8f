/* f16.c -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * float16_t's conversions, restated from include/utils/float16.hpp:
 *   float_to_f16_bits (:16-51): exponent re-biased by 15-127; exponent >= 31
 *     (overflow, infinity and NaN alike) -> +-infinity; exponent <= 0 ->
 *     subnormal or zero: the mantissa with its hidden bit (none for an fp32
 *     subnormal) shifted right by 13 + (1 - exponent), rounded to nearest even
 *     on the shifted-out bits, zero when the shift passes 24; else the
 *     mantissa rounded to nearest even at bit 13, a carry into bit 10 moving
 *     to the next exponent (infinity past 30).
 *   f16_bits_to_float (:54-77): zero; subnormal normalised with clz; exponent
 *     31 -> +-infinity, or a NaN with only the quiet bit (0x400000) set;
 *     normal re-biased.
 */
#include <string.h>

#include "oracle.h"

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t or_f32_to_f16(float f) {
    uint32_t bits = f2u(f);
    uint32_t sign = (bits >> 31) & 1u, exp = (bits >> 23) & 0xFFu, mant = bits & 0x7FFFFFu;
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)((sign << 15) | 0x7C00u);
    if (e <= 0) {
        uint32_t m = exp != 0 ? (mant | 0x800000u) : mant;
        int32_t shift = 1 - e;
        if (shift > 24) return (uint16_t)(sign << 15);
        uint32_t kept = m >> (shift + 13);
        uint32_t round_bit = (m >> (shift + 12)) & 1u;
        uint32_t sticky = m & ((1u << (shift + 12)) - 1u);
        uint32_t up = (round_bit && (sticky || (kept & 1u))) ? 1u : 0u;
        return (uint16_t)((sign << 15) | (kept + up));
    }
    uint32_t kept = mant >> 13;
    uint32_t round_bit = (mant >> 12) & 1u;
    uint32_t sticky = mant & 0xFFFu;
    uint32_t up = (round_bit && (sticky || (kept & 1u))) ? 1u : 0u;
    uint32_t m = kept + up;
    if (m >= 0x400u) {
        m = 0;
        ++e;
        if (e >= 31) return (uint16_t)((sign << 15) | 0x7C00u);
    }
    return (uint16_t)((sign << 15) | ((uint32_t)e << 10) | m);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    uint32_t out;
    if (exp == 0) {
        if (mant == 0) {
            out = sign << 31;
        } else {
            int shift = __builtin_clz(mant) - 21;
            mant <<= shift;
            int32_t e = 1 - shift;
            out = (sign << 31) | ((uint32_t)(e + 127 - 15) << 23) | ((mant & 0x3FFu) << 13);
        }
    } else if (exp == 31) {
        out = (sign << 31) | 0x7F800000u | (mant ? 0x400000u : 0u);
    } else {
        out = (sign << 31) | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    return u2f(out);
}
