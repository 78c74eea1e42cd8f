/* attention.c -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * PagedAttentionImpl<CPU>::execute (src/backend/cpu/attention.cpp:123-216) and
 * FlashAttentionImpl<CPU>::execute (:39-121) for bf16 (and, for the paged op,
 * fp16) tensors, single thread,
 * per-token online softmax in fp32 exactly as written there:
 *   score = (sum_d q[d]*k[d]) * scale               (:184-192, fma chain)
 *   m' = fmax(m, score); e_s = exp(score-m'); e_p = exp(m-m')   (:194-197)
 *   o[d] = o[d]*e_p + e_s*v[d];  l = l*e_p + e_s                (:199-203)
 *   out = bf16(o[d] * (1/l))                                    (:207-212)
 * with kv_h = h / n_kv_groups (:158) and q_abs = total_cached - S + sq (:164).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

int or__layer_view(or_manager *m, int32_t layer, int32_t *active, int32_t *num_cached, int32_t *n_pages,
                   const int32_t **k_ids, const int32_t **v_ids, or_block_pool **kp, or_block_pool **vp);

/* to_f32_rt / from_f32_rt for the two 16-bit types (dtype_traits.hpp:52-69) */
static inline float elem_to_f32(int32_t dtype, uint16_t x) {
    return dtype == OR_DTYPE_F16 ? or_f16_to_f32(x) : or_bf16_to_f32(x);
}
static inline uint16_t elem_from_f32(int32_t dtype, float f) {
    return dtype == OR_DTYPE_F16 ? or_f32_to_f16(f) : or_f32_to_bf16(f);
}

int or_paged_attend_dt(or_manager *m, int32_t layer, const uint16_t *Q, uint16_t *out, int32_t batch,
                       int32_t n_q_heads, int32_t seq_len, int32_t head_dim, int32_t n_kv_heads,
                       int32_t n_kv_groups, float scale, int causal, int32_t dtype) {
    int32_t active, total_cached, num_blocks;
    const int32_t *k_ids, *v_ids;
    or_block_pool *kp, *vp;
    or__layer_view(m, layer, &active, &total_cached, &num_blocks, &k_ids, &v_ids, &kp, &vp);
    if (!active || num_blocks == 0) return 1; /* :148 */
    float *o = (float *)malloc((size_t)head_dim * sizeof(float));
    for (int32_t b = 0; b < batch; ++b) {
        for (int32_t h = 0; h < n_q_heads; ++h) {
            int32_t kv_h = h / n_kv_groups;
            for (int32_t sq = 0; sq < seq_len; ++sq) {
                const uint16_t *qrow = Q + (((size_t)b * n_q_heads + h) * seq_len + sq) * head_dim;
                float mx = -INFINITY, l = 0.0f;
                for (int32_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
                int32_t q_abs = total_cached - seq_len + sq;
                int32_t limit = causal ? q_abs : (total_cached - 1);
                for (int32_t blk = 0; blk < num_blocks; ++blk) {
                    int32_t bs = blk * OR_PAGE_BLOCK_SIZE;
                    int32_t be = bs + OR_PAGE_BLOCK_SIZE < total_cached ? bs + OR_PAGE_BLOCK_SIZE : total_cached;
                    if (bs > limit) break;
                    const uint16_t *kb = (const uint16_t *)or_pool_block_data(kp, k_ids[blk]);
                    const uint16_t *vb = (const uint16_t *)or_pool_block_data(vp, v_ids[blk]);
                    if (!kb || !vb) continue; /* :177 */
                    for (int32_t t = 0; t < be - bs; ++t) {
                        int32_t kv_pos = bs + t;
                        if (causal && kv_pos > q_abs) break;
                        size_t off = ((size_t)t * n_kv_heads + kv_h) * head_dim;
                        float score = 0.0f;
                        for (int32_t d = 0; d < head_dim; ++d)
                            score += elem_to_f32(dtype, qrow[d]) * elem_to_f32(dtype, kb[off + d]);
                        score *= scale;
                        float m_prev = mx;
                        mx = fmaxf(mx, score);
                        float e_s = expf(score - mx);
                        float e_p = expf(m_prev - mx);
                        for (int32_t d = 0; d < head_dim; ++d)
                            o[d] = o[d] * e_p + e_s * elem_to_f32(dtype, vb[off + d]);
                        l = l * e_p + e_s;
                    }
                }
                float inv_l = 1.0f / l;
                uint16_t *orow = out + (((size_t)b * n_q_heads + h) * seq_len + sq) * head_dim;
                for (int32_t d = 0; d < head_dim; ++d) orow[d] = elem_from_f32(dtype, o[d] * inv_l);
            }
        }
    }
    free(o);
    return 0;
}

int or_paged_attend(or_manager *m, int32_t layer, const uint16_t *Q, uint16_t *out, int32_t batch,
                    int32_t n_q_heads, int32_t seq_len, int32_t head_dim, int32_t n_kv_heads,
                    int32_t n_kv_groups, float scale, int causal) {
    return or_paged_attend_dt(m, layer, Q, out, batch, n_q_heads, seq_len, head_dim, n_kv_heads, n_kv_groups,
                              scale, causal, OR_DTYPE_BF16);
}

int or_paged_attention_dt(or_manager *m, int32_t layer, const uint16_t *Q, const uint16_t *K,
                          const uint16_t *V, uint16_t *out, int32_t batch, int32_t n_q_heads,
                          int32_t seq_len, int32_t head_dim, int32_t n_kv_heads, int32_t n_kv_groups,
                          float scale, int causal, int32_t dtype) {
    if (!m || !or_mgr_is_active(m, layer)) return 1; /* :124-127 */
    or_mgr_append_kv_from_tensor(m, layer, K, V, n_kv_heads, seq_len, head_dim, dtype); /* :146 */
    return or_paged_attend_dt(m, layer, Q, out, batch, n_q_heads, seq_len, head_dim, n_kv_heads, n_kv_groups,
                              scale, causal, dtype);
}

int or_paged_attention(or_manager *m, int32_t layer, const uint16_t *Q, const uint16_t *K,
                       const uint16_t *V, uint16_t *out, int32_t batch, int32_t n_q_heads,
                       int32_t seq_len, int32_t head_dim, int32_t n_kv_heads, int32_t n_kv_groups,
                       float scale, int causal) {
    return or_paged_attention_dt(m, layer, Q, K, V, out, batch, n_q_heads, seq_len, head_dim, n_kv_heads,
                                 n_kv_groups, scale, causal, OR_DTYPE_BF16);
}

/* FlashAttentionImpl<CPU> -- attention.cpp:39-121.  Scores for all keys, causal
 * mask skv > sq to -inf, max, exp/sum, normalise by division, then P.V. */
void or_flash_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *out,
                        int32_t batch, int32_t n_q_heads, int32_t seq_len, int32_t n_kv_heads,
                        int32_t head_dim, int32_t n_kv_groups, float scale, int causal) {
    float *scores = (float *)malloc((size_t)(seq_len > 0 ? seq_len : 1) * sizeof(float));
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < n_q_heads; ++h) {
            int64_t kv_h = h / n_kv_groups;
            for (int64_t sq = 0; sq < seq_len; ++sq) {
                size_t q_off = (size_t)((b * n_q_heads * seq_len + h * seq_len + sq) * head_dim);
                for (int64_t skv = 0; skv < seq_len; ++skv) {
                    size_t k_off = (size_t)((b * n_kv_heads * seq_len + kv_h * seq_len + skv) * head_dim);
                    float dot = 0.0f;
                    for (int32_t d = 0; d < head_dim; ++d)
                        dot += or_bf16_to_f32(Q[q_off + d]) * or_bf16_to_f32(K[k_off + d]);
                    scores[skv] = dot * scale;
                }
                if (causal)
                    for (int64_t skv = sq + 1; skv < seq_len; ++skv) scores[skv] = -INFINITY;
                float mx = -INFINITY;
                for (int64_t skv = 0; skv < seq_len; ++skv)
                    if (scores[skv] > mx) mx = scores[skv];
                float sum = 0.0f;
                for (int64_t skv = 0; skv < seq_len; ++skv) {
                    scores[skv] = expf(scores[skv] - mx);
                    sum += scores[skv];
                }
                for (int64_t skv = 0; skv < seq_len; ++skv) scores[skv] /= sum;
                size_t o_off = q_off;
                for (int32_t d = 0; d < head_dim; ++d) {
                    float val = 0.0f;
                    for (int64_t skv = 0; skv < seq_len; ++skv) {
                        size_t v_off = (size_t)((b * n_kv_heads * seq_len + kv_h * seq_len + skv) * head_dim + d);
                        val += scores[skv] * or_bf16_to_f32(V[v_off]);
                    }
                    out[o_off + d] = or_f32_to_bf16(val);
                }
            }
        }
    free(scores);
}

/* The Qwen3 attention block's K/V side, Qwen3.cpp:137-166: permute token-major
 * k/v to head-major (shape.cpp:69-100), per-head rms_norm of k (and q), RoPE at
 * start_pos (rope.cpp:76-119), then append_kv_from_tensor (page_attention.cpp:104-140). */
void or_qk_norm_rope_append(or_manager *m, int32_t layer, const uint16_t *q_tok, int32_t n_q_heads,
                            const float *gamma_q, uint16_t *q_out, const uint16_t *k_tok,
                            const uint16_t *v_tok, int32_t n_kv_heads, int32_t seq_len, int32_t head_dim,
                            const float *gamma_k, float eps, const float *cos_tab, const float *sin_tab,
                            int32_t rope_dim, int64_t start_pos) {
    size_t nk = (size_t)n_kv_heads * seq_len * head_dim;
    uint16_t *k4 = (uint16_t *)malloc(nk * 2), *kn = (uint16_t *)malloc(nk * 2);
    uint16_t *kr = (uint16_t *)malloc(nk * 2), *v4 = (uint16_t *)malloc(nk * 2);
    or_permute_tok_to_head(k4, k_tok, seq_len, n_kv_heads, head_dim);
    or_permute_tok_to_head(v4, v_tok, seq_len, n_kv_heads, head_dim);
    or_rms_norm(kn, k4, gamma_k, (size_t)n_kv_heads * seq_len, (size_t)head_dim, eps);
    or_apply_rope_partial(kr, kn, cos_tab, sin_tab, n_kv_heads, seq_len, head_dim, rope_dim, start_pos);
    if (q_tok && q_out) {
        size_t nq = (size_t)n_q_heads * seq_len * head_dim;
        uint16_t *q4 = (uint16_t *)malloc(nq * 2), *qn = (uint16_t *)malloc(nq * 2);
        or_permute_tok_to_head(q4, q_tok, seq_len, n_q_heads, head_dim);
        or_rms_norm(qn, q4, gamma_q, (size_t)n_q_heads * seq_len, (size_t)head_dim, eps);
        or_apply_rope_partial(q_out, qn, cos_tab, sin_tab, n_q_heads, seq_len, head_dim, rope_dim, start_pos);
        free(q4);
        free(qn);
    }
    or_mgr_append_kv_from_tensor(m, layer, kr, v4, n_kv_heads, seq_len, head_dim, OR_DTYPE_BF16);
    free(k4);
    free(kn);
    free(kr);
    free(v4);
}
