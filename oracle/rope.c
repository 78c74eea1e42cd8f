/* rope.c -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * RopeCacheImpl<CPU> (src/backend/cpu/rope.cpp:121-148): inverse frequencies
 * and angles in double, each table row [max_seq][head_dim] holds the value for
 * pair i twice, at i and at i + head_dim/2.
 *
 * ApplyRopeImpl<CPU> (rope.cpp:76-119), bf16, B == 1: NeoX half rotation on
 * rows of a head-major [H][S][D] tensor at position start_pos + s:
 *   y[i]        = x0*c - x1*s
 *   y[i + D/2]  = x0*s + x1*c        x0 = x[i], x1 = x[i+D/2], c,s = tab[pos][i]
 * Outputs are rounded to bf16 by the bfloat16_t constructor (RNE, subnormal
 * flush).  The expressions are written as in the reference and compiled with
 * the same GCC contraction (-ffp-contract=fast, -mfma), which turns them into
 *   fmaf(x0, c, -(x1*s))   and   fmaf(x0, s, x1*c)
 * (checked in the object code of this file; the HIP kernels use these forms).
 */
#include <math.h>

#include "oracle.h"

void or_rope_cache(float *dst, float theta, int head_dim, int max_seq, int is_cos) {
    int half = head_dim / 2;
    double inv_f[1024];
    for (int i = 0; i < half && i < 1024; ++i) {
        double e = (2.0 * (double)i) / (double)head_dim;
        inv_f[i] = 1.0 / pow((double)theta, e);
    }
    for (int s = 0; s < max_seq; ++s) {
        double pos = (double)s;
        int base = s * head_dim;
        for (int i = 0; i < half; ++i) {
            double ang = pos * inv_f[i];
            float v = is_cos ? (float)cos(ang) : (float)sin(ang);
            dst[base + i] = v;
            dst[base + i + half] = v;
        }
    }
}

void or_apply_rope(uint16_t *out, const uint16_t *x, const float *cos_tab, const float *sin_tab,
                   int64_t n_heads, int64_t seq_len, int64_t head_dim, int64_t start_pos) {
    int64_t half = head_dim / 2;
    size_t head_stride = (size_t)(seq_len * head_dim);
    for (int64_t h = 0; h < n_heads; ++h) {
        for (int64_t s = 0; s < seq_len; ++s) {
            int64_t pos = start_pos + s;
            const float *c = cos_tab + pos * head_dim;
            const float *sn = sin_tab + pos * head_dim;
            uint16_t *ro = out + (size_t)h * head_stride + (size_t)(s * head_dim);
            const uint16_t *ri = x + (size_t)h * head_stride + (size_t)(s * head_dim);
            for (int64_t i = 0; i < half; ++i) {
                float x0 = or_bf16_to_f32(ri[i]);
                float x1 = or_bf16_to_f32(ri[i + half]);
                float ci = c[i], si = sn[i];
                float xr = x0 * ci - x1 * si;
                float xi = x0 * si + x1 * ci;
                ro[i] = or_f32_to_bf16(xr);
                ro[i + half] = or_f32_to_bf16(xi);
            }
        }
    }
}

/* Partial rotation (Qwen3.5: rope_dimension_count 64 of head_dim 256,
 * Qwen35.hpp:14-16, tables built by rope_cache(max_seq, 64, theta),
 * Qwen35.cpp:95-100, so rows of rope_dim floats).  The reference's
 * ApplyRopeImpl reads op_params[0] only (rope.cpp:80-82) and indexes the
 * rope_dim-wide table with stride head_dim -- outside the table for this shape
 * -- so there is no reference behaviour to restate; the op's contract
 * (op_params[1] = rope_dim = the table width, op_factory.hpp:504-529) and the
 * Qwen3.5 convention define it: the first rope_dim dims rotate exactly as
 * or_apply_rope does with head_dim = rope_dim (same expressions, same
 * contraction), the remaining dims are copied unchanged.  With rope_dim ==
 * head_dim this is or_apply_rope. */
void or_apply_rope_partial(uint16_t *out, const uint16_t *x, const float *cos_tab, const float *sin_tab,
                           int64_t n_heads, int64_t seq_len, int64_t head_dim, int64_t rope_dim, int64_t start_pos) {
    int64_t half = rope_dim / 2;
    size_t head_stride = (size_t)(seq_len * head_dim);
    for (int64_t h = 0; h < n_heads; ++h) {
        for (int64_t s = 0; s < seq_len; ++s) {
            int64_t pos = start_pos + s;
            const float *c = cos_tab + pos * rope_dim;
            const float *sn = sin_tab + pos * rope_dim;
            uint16_t *ro = out + (size_t)h * head_stride + (size_t)(s * head_dim);
            const uint16_t *ri = x + (size_t)h * head_stride + (size_t)(s * head_dim);
            for (int64_t i = 0; i < half; ++i) {
                float x0 = or_bf16_to_f32(ri[i]);
                float x1 = or_bf16_to_f32(ri[i + half]);
                float ci = c[i], si = sn[i];
                float xr = x0 * ci - x1 * si;
                float xi = x0 * si + x1 * ci;
                ro[i] = or_f32_to_bf16(xr);
                ro[i + half] = or_f32_to_bf16(xi);
            }
            for (int64_t i = rope_dim; i < head_dim; ++i) ro[i] = ri[i];
        }
    }
}

/* PermuteImpl<CPU> fast path (shape.cpp:69-100): the innermost dim is kept, so
 * rows of D elements are copied; here the two permutations the Qwen3 layer uses
 * between [1,S,H,D] and [1,H,S,D] (Qwen3.cpp:137-141, :169). */
void or_permute_tok_to_head(uint16_t *dst, const uint16_t *src, int64_t S, int64_t H, int64_t D) {
    for (int64_t h = 0; h < H; ++h)
        for (int64_t s = 0; s < S; ++s)
            for (int64_t d = 0; d < D; ++d) dst[(h * S + s) * D + d] = src[(s * H + h) * D + d];
}

void or_permute_head_to_tok(uint16_t *dst, const uint16_t *src, int64_t S, int64_t H, int64_t D) {
    for (int64_t s = 0; s < S; ++s)
        for (int64_t h = 0; h < H; ++h)
            for (int64_t d = 0; d < D; ++d) dst[(s * H + h) * D + d] = src[(h * S + s) * D + d];
}
