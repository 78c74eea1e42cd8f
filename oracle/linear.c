/* linear.c -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * linear<bfloat16_t> of src/backend/cpu/linear.cpp:46-122 (called by
 * LinearImpl<CPU>::execute, :325-345, transpose_w = 1, batch 1), restated lane
 * by lane so the fp32 summation order is the reference's exactly.  For output
 * (r, c), with x [rows][common] and w [cols][common] row-major:
 *
 *   acc = 0; for each K-block of 256 elements (KR, :57; :66-114):
 *     local = acc
 *     if the block holds >= 16 elements (:76-89): two 8-lane accumulators,
 *       step i covers elements 16i..16i+15 of the block: lane l of sum0 takes
 *       element 16i+l, lane l of sum1 element 16i+8+l, each one fused
 *       multiply-add (_mm256_fmadd_ps); then v = sum0 + sum1 lane-wise and
 *       local += hsum(v), hsum(v) = (t0+t1)+(t2+t3) with t[i] = v[i]+v[i+4]
 *       (hsum_ps :24-31)
 *     each remaining 8-element group (:91-96): s[l] = x*w rounded (fmadd with
 *       a zero addend), local += hsum(s)
 *     each remaining element (:98-101): local += x*w, contracted to a fused
 *       multiply-add by GCC under -mfma (-ffp-contract=fast)
 *     acc = local
 *   out = bfloat16_t(acc + bias[c]) (:104-114): the bias (bf16 -> fp32) is
 *   added in fp32 and the sum rounded once, RNE with the constructor's
 *   special cases (or_f32_to_bf16).
 *
 * The row blocking (MR = NR = 16) and the OpenMP split over row blocks do not
 * change any output's summation order.
 */
#include <math.h>

#include "oracle.h"

static float hsum8(const float v[8]) {
    const float t0 = v[0] + v[4], t1 = v[1] + v[5], t2 = v[2] + v[6], t3 = v[3] + v[7];
    return (t0 + t1) + (t2 + t3);
}

void or_linear_bf16(uint16_t *out, const uint16_t *x, const uint16_t *w, int64_t rows, int64_t common, int64_t cols,
                    const uint16_t *bias) {
    const int64_t KR = 256;
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t *xr = x + r * common;
        for (int64_t c = 0; c < cols; ++c) {
            const uint16_t *wc = w + c * common;
            float acc = 0.0f;
            for (int64_t k0 = 0; k0 < common; k0 += KR) {
                const int64_t k_len = common - k0 < KR ? common - k0 : KR;
                const uint16_t *xp = xr + k0, *wp = wc + k0;
                float local = acc;
                int64_t k = 0;
                if (k_len >= 16) {
                    float s0[8] = {0}, s1[8] = {0}, v[8];
                    for (; k + 16 <= k_len; k += 16)
                        for (int l = 0; l < 8; ++l) {
                            s0[l] = fmaf(or_bf16_to_f32(xp[k + l]), or_bf16_to_f32(wp[k + l]), s0[l]);
                            s1[l] = fmaf(or_bf16_to_f32(xp[k + 8 + l]), or_bf16_to_f32(wp[k + 8 + l]), s1[l]);
                        }
                    for (int l = 0; l < 8; ++l) v[l] = s0[l] + s1[l];
                    local += hsum8(v);
                }
                for (; k + 8 <= k_len; k += 8) {
                    float s[8];
                    for (int l = 0; l < 8; ++l) s[l] = or_bf16_to_f32(xp[k + l]) * or_bf16_to_f32(wp[k + l]);
                    local += hsum8(s);
                }
                for (; k < k_len; ++k) local = fmaf(or_bf16_to_f32(xp[k]), or_bf16_to_f32(wp[k]), local);
                acc = local;
            }
            float val = acc;
            if (bias) val += or_bf16_to_f32(bias[c]);
            out[r * cols + c] = or_f32_to_bf16(val);
        }
    }
}
