/* rms_norm.c -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * rms_norm of src/backend/cpu/normalization.cpp:44-107 (called by
 * RmsNormImpl<CPU>, :138-153), restated lane by lane so the fp32 summation
 * order is the reference's exactly:
 *
 *   sum of squares: 32 running sums A[0..31] (four 8-wide AVX accumulators,
 *     :59-73); block j of 32 elements adds x[j+a]^2 into A[a] with one fused
 *     multiply-add per element (_mm256_fmadd_ps).  Then the four accumulators
 *     are combined per lane as (A0+A1)+(A2+A3) (:75-77), remaining 8-blocks are
 *     fused into that sum (:79-82), the 8 lanes are reduced as
 *     lo+hi then two horizontal adds, i.e. ((u0+u1)+(u2+u3)) with
 *     u[i] = T[i]+T[i+4] (hsum_ps :34-41), and any scalar tail is added with a
 *     fused multiply-add (GCC contracts "sum_sq += val*val" under -mfma).
 *   scale: r = 1 / sqrt(ss / hidden + eps)                          (:90)
 *   output: (x * r) * w[j]; the 8-wide part is stored by TRUNCATING to bf16
 *     (store_f32_bf16 :25-31), the scalar tail by round-to-nearest-even
 *     through the bfloat16_t constructor (:102-105).
 */
#include <math.h>

#include "oracle.h"

void or_rms_norm(uint16_t *out, const uint16_t *x, const float *w, size_t rows, size_t hidden, float eps) {
    for (size_t i = 0; i < rows; ++i) {
        const uint16_t *xr = x + i * hidden;
        uint16_t *orow = out + i * hidden;
        float A[32];
        for (int a = 0; a < 32; ++a) A[a] = 0.0f;
        size_t j = 0;
        for (; j + 32 <= hidden; j += 32)
            for (int a = 0; a < 32; ++a) {
                float v = or_bf16_to_f32(xr[j + a]);
                A[a] = fmaf(v, v, A[a]);
            }
        float T[8];
        for (int l = 0; l < 8; ++l) T[l] = (A[l] + A[8 + l]) + (A[16 + l] + A[24 + l]);
        for (; j + 8 <= hidden; j += 8)
            for (int l = 0; l < 8; ++l) {
                float v = or_bf16_to_f32(xr[j + l]);
                T[l] = fmaf(v, v, T[l]);
            }
        float u0 = T[0] + T[4], u1 = T[1] + T[5], u2 = T[2] + T[6], u3 = T[3] + T[7];
        float ss = (u0 + u1) + (u2 + u3);
        for (; j < hidden; ++j) {
            float v = or_bf16_to_f32(xr[j]);
            ss = fmaf(v, v, ss);
        }
        float r = 1.0f / sqrtf(ss / (float)hidden + eps);
        size_t vec_end = (hidden / 8) * 8;
        for (j = 0; j < vec_end; ++j) {
            float y = (or_bf16_to_f32(xr[j]) * r) * w[j];
            uint32_t u;
            __builtin_memcpy(&u, &y, sizeof u);
            orow[j] = (uint16_t)(u >> 16); /* truncation */
        }
        for (j = vec_end; j < hidden; ++j) {
            float y = (or_bf16_to_f32(xr[j]) * r) * w[j];
            orow[j] = or_f32_to_bf16(y); /* RNE tail */
        }
    }
}
