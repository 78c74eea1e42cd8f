/*
 * oracle.h -- CPU restatement of Genllm's paged KV-cache attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The MI355X product path (genllm_amd/, libgenllm_hip.so) never
 * links, loads or calls anything in this directory.
 *
 * Every function restates one reference function; the citation in front of
 * each declaration names the file:line of /root/reference it follows.  It is
 * compiled like the reference (gcc -O3 -mavx2 -mfma -mf16c, GNU default
 * -ffp-contract=fast, see oracle/Makefile), single-threaded.
 *
 * Pinning (each function is checked by tests/test_oracle.py against the
 * reference's own unit-test values, closed forms and brute force):
 *   bf16 conversion   test_dtype.cpp values + independent textbook RNE
 *   block pool / mgr  test_page_attention.cpp (all 5 tests) + LIFO/overflow
 *   rms_norm          test_ops_cpu.cpp:118-148 values + fp64 closed form
 *   rope_cache        fp64 closed form (numpy), bit-exact
 *   apply_rope        pos-0 identity, fp64 closed form, rotation composition;
 *                     the partial form: equal to apply_rope at rope_dim ==
 *                     head_dim, copied dims bit-exact, fp64 closed form
 *   linear            integer closed form on every summation path, hand-derived
 *                     block/tree order cases, fp64 bound
 *   append (scatter)  closed-form page address, bit-exact
 *   paged attention   fp64 brute force, N=1 identity, equal-keys mean,
 *                     dominant-score selection, GQA head map
 *   flash attention   fp64 brute force
 * libm boundary (expf/sqrtf/cos/sin/pow): the same glibc as the reference
 * would use; no reference test pins values there ("parity unpinned" at the
 * libm ulp level only -- the functions above are pinned to tolerance).
 */
#ifndef GENLLM_ORACLE_H
#define GENLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* PAGE_BLOCK_SIZE -- include/core/page_attention.h:9 */
#define OR_PAGE_BLOCK_SIZE 16

/* DataType ids used on this path -- include/utils/utils.hpp:30-59 */
#define OR_DTYPE_F32 0
#define OR_DTYPE_F16 1
#define OR_DTYPE_BF16 30

/* ---- fp16 scalar conversion: include/utils/float16.hpp:16-77 (float16_t) ---- */
uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);

/* ---- bf16 scalar conversion: include/utils/bfloat16.hpp:18-45 ---- */
uint16_t or_f32_to_bf16(float f);
float or_bf16_to_f32(uint16_t b);
void or_f32_to_bf16_array(const float *src, uint16_t *dst, size_t n);
void or_bf16_to_f32_array(const uint16_t *src, float *dst, size_t n);

/* ---- BlockPool: page_attention.h:11-45, page_attention.cpp:25-64 ---- */
typedef struct or_block_pool or_block_pool;
or_block_pool *or_pool_create(void *buffer, size_t buffer_bytes, int32_t block_capacity,
                              int32_t n_kv_heads, int32_t head_dim, size_t elem_size);
void or_pool_destroy(or_block_pool *p);
int32_t or_pool_alloc(or_block_pool *p);
void or_pool_free(or_block_pool *p, int32_t id);
void or_pool_reset(or_block_pool *p);
void *or_pool_block_data(const or_block_pool *p, int32_t id);
int32_t or_pool_num_blocks(const or_block_pool *p);
int32_t or_pool_num_free(const or_block_pool *p);

/* ---- PagedAttentionManager: page_attention.h:52-90, page_attention.cpp:66-216 ----
 * with_pool == 0 mirrors a manager built with no MemoryPool (pool_ == nullptr,
 * the fake of test_page_attention.cpp:50); reserve_layer is then a no-op.
 * With a pool, K/V pools are zeroed host buffers (resource_cpu.cpp:43). */
typedef struct or_manager or_manager;
or_manager *or_mgr_create(int with_pool);
void or_mgr_destroy(or_manager *m);
void or_mgr_init_layer(or_manager *m, int32_t layer, int32_t n_kv_heads, int32_t head_dim, int32_t dtype);
void or_mgr_reserve_layer(or_manager *m, int32_t layer, int32_t max_blocks);
void or_mgr_append_kv_pages(or_manager *m, int32_t layer, int32_t count);
void or_mgr_append_kv_from_tensor(or_manager *m, int32_t layer, const void *K, const void *V,
                                  int32_t n_kv_heads, int32_t seq_len, int32_t head_dim, int32_t dtype);
void or_mgr_append_kv_from_pos(or_manager *m, int32_t layer, const void *K, const void *V, int32_t n_kv_heads,
                               int32_t head_dim, int32_t dtype, int32_t global_pos, int32_t count);
void or_mgr_reset(or_manager *m);
int or_mgr_is_active(const or_manager *m, int32_t layer);
int32_t or_mgr_num_cached(or_manager *m, int32_t layer);
int32_t or_mgr_num_pages(or_manager *m, int32_t layer);
/* copies up to cap entries of the page table; returns the table length */
int32_t or_mgr_get_page_table(or_manager *m, int32_t layer, int32_t *k_ids, int32_t *v_ids, int32_t cap);
/* direct mutation of the layer state (get_layer returns a mutable reference,
 * page_attention.cpp:204-206): replace the table and num_cached */
void or_mgr_set_page_table(or_manager *m, int32_t layer, const int32_t *k_ids, const int32_t *v_ids,
                           int32_t n, int32_t num_cached);
void *or_mgr_k_pool(or_manager *m, int32_t layer);
void *or_mgr_v_pool(or_manager *m, int32_t layer);
or_block_pool *or_mgr_pool(or_manager *m, int32_t layer, int which /*0 K, 1 V*/);

/* ---- rms_norm: src/backend/cpu/normalization.cpp:44-107 (bf16 in/out, fp32 gamma) ---- */
void or_rms_norm(uint16_t *out, const uint16_t *x, const float *w, size_t rows, size_t hidden, float eps);

/* ---- RopeCacheImpl<CPU>: src/backend/cpu/rope.cpp:121-148 ---- */
void or_rope_cache(float *dst, float theta, int head_dim, int max_seq, int is_cos);
/* ---- ApplyRopeImpl<CPU> (bf16): src/backend/cpu/rope.cpp:76-119, B == 1 ---- */
void or_apply_rope(uint16_t *out, const uint16_t *x, const float *cos_tab, const float *sin_tab,
                   int64_t n_heads, int64_t seq_len, int64_t head_dim, int64_t start_pos);
/* Partial rotation over the first rope_dim dims with [max_seq][rope_dim]
 * tables (Qwen3.5, Qwen35.hpp:14-16); the other dims are copied.  No reference
 * behaviour exists for rope_dim < head_dim (see rope.c); rope_dim == head_dim
 * is or_apply_rope. */
void or_apply_rope_partial(uint16_t *out, const uint16_t *x, const float *cos_tab, const float *sin_tab,
                           int64_t n_heads, int64_t seq_len, int64_t head_dim, int64_t rope_dim, int64_t start_pos);

/* ---- PermuteImpl<CPU> fast path for [1,S,H,D] -> [1,H,S,D]: shape.cpp:69-117 ---- */
void or_permute_tok_to_head(uint16_t *dst, const uint16_t *src, int64_t S, int64_t H, int64_t D);
void or_permute_head_to_tok(uint16_t *dst, const uint16_t *src, int64_t S, int64_t H, int64_t D);

/* ---- PagedAttentionImpl<CPU>::execute: src/backend/cpu/attention.cpp:123-216 (bf16) ----
 * Q,K,V head-major [1,H,S,D]; appends K/V then attends; returns 0, or 1 when the
 * op returned early (inactive layer / empty table). */
int or_paged_attention(or_manager *m, int32_t layer, const uint16_t *Q, const uint16_t *K,
                       const uint16_t *V, uint16_t *out, int32_t batch, int32_t n_q_heads,
                       int32_t seq_len, int32_t head_dim, int32_t n_kv_heads, int32_t n_kv_groups,
                       float scale, int causal);
/* the attention half alone (attention.cpp:148-215), for attention-only configs */
int or_paged_attend(or_manager *m, int32_t layer, const uint16_t *Q, uint16_t *out, int32_t batch,
                    int32_t n_q_heads, int32_t seq_len, int32_t head_dim, int32_t n_kv_heads,
                    int32_t n_kv_groups, float scale, int causal);
/* the same two with the element type of Q, the pools and out (the reference
 * reads K/V as Q->dtype through to_f32_rt and stores out through from_f32_rt,
 * dtype_traits.hpp:52-69): OR_DTYPE_BF16 or OR_DTYPE_F16 */
int or_paged_attention_dt(or_manager *m, int32_t layer, const uint16_t *Q, const uint16_t *K,
                          const uint16_t *V, uint16_t *out, int32_t batch, int32_t n_q_heads,
                          int32_t seq_len, int32_t head_dim, int32_t n_kv_heads, int32_t n_kv_groups,
                          float scale, int causal, int32_t dtype);
int or_paged_attend_dt(or_manager *m, int32_t layer, const uint16_t *Q, uint16_t *out, int32_t batch,
                       int32_t n_q_heads, int32_t seq_len, int32_t head_dim, int32_t n_kv_heads,
                       int32_t n_kv_groups, float scale, int causal, int32_t dtype);

/* ---- FlashAttentionImpl<CPU>::execute: attention.cpp:39-121 (bf16 Q/K/V/out) ---- */
void or_flash_attention(const uint16_t *Q, const uint16_t *K, const uint16_t *V, uint16_t *out,
                        int32_t batch, int32_t n_q_heads, int32_t seq_len, int32_t n_kv_heads,
                        int32_t head_dim, int32_t n_kv_groups, float scale, int causal);

/* ---- Composition used by the Qwen3 layer (Qwen3.cpp:137-166) for the K/V side:
 * token-major k,v [S][Hkv][D] -> permute -> rms_norm(k) -> apply_rope(k) ->
 * append_kv_from_tensor.  Also q (optional, q_out head-major [Hq][S][D]).
 * start_pos is the RoPE op_params[2] (executor.cpp:208-247); rope_dim the
 * rotated dims (head_dim for Qwen3; 64 of 256 for Qwen3.5's layer,
 * Qwen35.cpp:191-226). */
void or_qk_norm_rope_append(or_manager *m, int32_t layer, const uint16_t *q_tok, int32_t n_q_heads,
                            const float *gamma_q, uint16_t *q_out, const uint16_t *k_tok,
                            const uint16_t *v_tok, int32_t n_kv_heads, int32_t seq_len, int32_t head_dim,
                            const float *gamma_k, float eps, const float *cos_tab, const float *sin_tab,
                            int32_t rope_dim, int64_t start_pos);

/* ---- linear<bfloat16_t>: src/backend/cpu/linear.cpp:46-122 (LinearImpl<CPU>, :325-345) ----
 * x [rows][common], w [cols][common] (transpose_w = 1), bias [cols] or NULL,
 * out [rows][cols]; the reference's fp32 summation order, one rounding. */
void or_linear_bf16(uint16_t *out, const uint16_t *x, const uint16_t *w, int64_t rows, int64_t common, int64_t cols,
                    const uint16_t *bias);

#ifdef __cplusplus
}
#endif
#endif
