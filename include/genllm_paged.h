/*
 * genllm_paged.h -- C ABI of the MI355X (gfx950) paged KV-cache attention path.
 *
 * This is the drop-in boundary for Genllm's paged attention: a
 * PagedAttentionImpl<Device::HIP> specialisation (same shape as
 * include/backend/cpu/attention.h:15-18 in the reference) calls these
 * functions with raw device pointers.  Plain C types only: pointers, sizes,
 * int32/int64/float; `stream` is a hipStream_t passed as void* (NULL = the
 * default stream).  Every function returns GENLLM_OK (0) or an error code, and
 * genllm_last_error() describes the last failure of the calling thread.
 *
 * Not thread-safe per genllm_kv object (the reference's PagedAttentionManager
 * is not either).  No call synchronises the stream; work is stream-ordered.
 * Tensors are bf16 (GGML_TYPE_BF16 = 30) unless stated; gammas and RoPE tables
 * are fp32, as in the reference.
 */
#ifndef GENLLM_PAGED_H
#define GENLLM_PAGED_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
#define GENLLM_OK 0
#define GENLLM_ERR_INVALID 1     /* bad argument: null pointer, shape, layer state */
#define GENLLM_ERR_UNSUPPORTED 2 /* head_dim / dtype the kernels do not cover
                                    (reference throws, src/backend/cuda/attention.cu:511) */
#define GENLLM_ERR_NO_MEMORY 3   /* kv_cache MemoryPool exhausted (reference throws,
                                    src/core/pools.cpp:26-31) */
#define GENLLM_ERR_POOL_FULL 4   /* BlockPool has no free page; the reference silently
                                    truncates (src/core/page_attention.cpp:155,161) */
#define GENLLM_ERR_HIP 5         /* HIP runtime error (allocation, copy, launch) */

#define GENLLM_PAGE_BLOCK_SIZE 16 /* include/core/page_attention.h:9 */
#define GENLLM_DTYPE_BF16 30      /* DataType::GGML_TYPE_BF16, include/utils/utils.hpp:59 */
#define GENLLM_DTYPE_F16 1        /* DataType::GGML_TYPE_F16 */

/* Message for the last failing call on this thread ("" if none). */
const char *genllm_last_error(void);

/* ------------------------------------------------------------- KV cache
 * One genllm_kv = the device's kv_cache MemoryPool (include/core/pools.h:11-48,
 * one hipMalloc of kv_pool_bytes, bump-allocated) plus the
 * PagedAttentionManager living on it (include/core/page_attention.h:52-90):
 * per layer a K and a V BlockPool of 16-token pages laid out [16][Hkv][D], a
 * host page table of {k_block_id, v_block_id} and its device-resident copy.
 */
typedef struct genllm_kv genllm_kv;

/* MemoryPool(kv_cache) + MemoryManager::create_attention_manager
 * (src/core/pools.cpp:3-15, src/core/manager.cpp:102-116). */
int genllm_kv_create(int32_t device, size_t kv_pool_bytes, genllm_kv **out);
int genllm_kv_destroy(genllm_kv *kv);

/* PagedAttentionManager::init_layer, src/core/page_attention.cpp:72-79 */
int genllm_kv_init_layer(genllm_kv *kv, int32_t layer, int32_t n_kv_heads, int32_t head_dim, int32_t dtype);
/* PagedAttentionManager::reserve_layer, page_attention.cpp:81-101: carves the
 * K pool and the V pool (max_blocks pages each, 256-byte aligned) from the
 * kv_cache pool -- exactly the 2 * max_blocks * block_bytes per layer the
 * reference scheduler sizes it for (scheduler.cpp:62-79, 371).  The device
 * page table (max_blocks entries), its pinned host staging and the manager's
 * decode workspace are allocated separately, here, once: the op itself never
 * allocates, frees or synchronises. */
int genllm_kv_reserve_layer(genllm_kv *kv, int32_t layer, int32_t max_blocks);
/* PagedAttentionManager::is_active, page_attention.h:82-85; *active = 0/1 */
int genllm_kv_is_active(genllm_kv *kv, int32_t layer, int32_t *active);
/* PagedAttentionManager::append_kv_pages, page_attention.cpp:141-162, plus the
 * upload of the new table entries on `stream`.  Unlike the reference, a pool
 * without enough free pages returns GENLLM_ERR_POOL_FULL and leaves the layer
 * unchanged. */
int genllm_kv_append_pages(genllm_kv *kv, int32_t layer, int32_t count, void *stream);
/* PagedAttentionManager::append_kv_from_pos, page_attention.cpp:164-203: write
 * count tokens at positions global_pos.. (k, v: device, head-major
 * [n_kv_heads][count][head_dim], dtype the layer's 2-byte type), opening pages
 * by the rule of append_kv_pages (a K and a V block at every position that is
 * a multiple of 16, entered into the table only past its end), then
 * num_cached = max(num_cached, global_pos + count).  Every head reads its own
 * rows: the reference copies head 0's row p to every head (:195, :198).
 * Errors leave the layer unchanged: GENLLM_ERR_INVALID when a position's page
 * is neither in the table nor opened by this call (the reference indexes the
 * table unchecked there), GENLLM_ERR_POOL_FULL when a pool cannot supply the
 * pages (the reference stops part-way).  count <= 0 does nothing. */
int genllm_kv_append_from_pos(genllm_kv *kv, int32_t layer, const void *k, const void *v, int32_t n_kv_heads,
                              int32_t head_dim, int32_t dtype, int32_t global_pos, int32_t count, void *stream);
/* PagedAttentionManager::reset (page_attention.cpp:208-216), reached through
 * MemoryManager::reset_kv_cache (manager.cpp:97-101). Host-only. */
int genllm_kv_reset(genllm_kv *kv);

/* LayerState (page_attention.h:57-66) as plain fields. */
typedef struct genllm_layer_info {
    int32_t active;
    int32_t num_cached;
    int32_t num_pages;  /* page_table.size() */
    int32_t n_kv_heads;
    int32_t head_dim;
    int32_t dtype;
    int32_t max_blocks; /* BlockPool capacity */
    int32_t k_num_blocks, k_num_free, v_num_blocks, v_num_free;
    void *k_pool;       /* device: K pool base (block 0) */
    void *v_pool;       /* device: V pool base */
    int32_t *k_ids;     /* device: page table, K block ids [max_blocks] */
    int32_t *v_ids;     /* device: page table, V block ids [max_blocks] */
    size_t block_bytes; /* 16 * n_kv_heads * head_dim * elem */
} genllm_layer_info;
int genllm_kv_layer_info(genllm_kv *kv, int32_t layer, genllm_layer_info *out);

/* Copy of the host page table (LayerState::page_table); *n = its length. */
int genllm_kv_page_table(genllm_kv *kv, int32_t layer, int32_t *k_ids, int32_t *v_ids, int32_t cap,
                         int32_t *n);
/* Direct mutation of the layer state (get_layer returns a mutable reference,
 * page_attention.cpp:204-206): replaces the table and num_cached, uploads the
 * table on `stream`.  Every id must be a block its pool has handed out. */
int genllm_kv_set_page_table(genllm_kv *kv, int32_t layer, const int32_t *k_ids, const int32_t *v_ids,
                             int32_t n, int32_t num_cached, void *stream);
/* BlockPool::alloc / free / num_blocks / num_free (page_attention.cpp:37-57);
 * which = 0 for the K pool, 1 for the V pool.  alloc writes -1 when full. */
int genllm_kv_block_alloc(genllm_kv *kv, int32_t layer, int32_t which, int32_t *id);
int genllm_kv_block_free(genllm_kv *kv, int32_t layer, int32_t which, int32_t id);

/* ---------------------------------------------------------------- the op
 * PagedAttentionImpl<D>::execute (src/backend/cpu/attention.cpp:123-216,
 * src/backend/cuda/attention.cu:491-580): append this step's K/V to the layer's
 * pages, then attend.  q, out: head-major [batch][n_q_heads][seq_len][head_dim];
 * k, v: [batch][n_kv_heads][seq_len][head_dim] (op_factory.hpp:413-476), of
 * the layer's element type (genllm_kv_init_layer: GENLLM_DTYPE_BF16 or
 * GENLLM_DTYPE_F16; the reference reads K/V as Q's dtype, attention.cpp:
 * 186-200).  As in the reference, every batch entry attends over the layer's
 * one cache and only the first entry's k/v rows are appended (attention.cpp:
 * 146, 156; append_kv_from_tensor reads n_kv_heads x seq_len rows).  scale,
 * causal and n_kv_groups are op_params[1..3].  An inactive layer returns
 * GENLLM_OK without touching out (attention.cpp:127).  head_dim 128 (Qwen3)
 * and 256 (Qwen3.5, Qwen35.hpp:14-16) are served; any other returns
 * GENLLM_ERR_UNSUPPORTED (the CUDA op throws for head_dim != 128,
 * attention.cu:511).  Chunks of up to 16 (query, q-head) rows per kv head run
 * the split-K decode kernel, longer chunks the MFMA prefill kernel.  Every
 * argument check and the split plan run before the layer changes: a call that
 * returns an error leaves num_cached, the page tables and the block pools as
 * they were. */
int genllm_paged_attention(genllm_kv *kv, int32_t layer, const void *q, const void *k, const void *v, void *out,
                           int32_t batch, int32_t n_q_heads, int32_t seq_len, int32_t head_dim,
                           int32_t n_kv_heads, int32_t n_kv_groups, float scale, int32_t causal, void *stream);

/* ------------------------------------------ device-position decode steps
 * The reference's decode loop advances the cache position every step
 * (src/core/executor.cpp:227-236) and each step's append opens a page when the
 * position reaches a multiple of 16 (append_kv_pages, page_attention.cpp:
 * 141-162).  These calls move both to the device so that a decode step can be
 * captured once into a HIP graph and replayed for successive tokens:
 *
 *   genllm_kv_stage_decode(kv, l, n, s)   host: open the pages positions
 *       [end, end + n) need, in the order per-step appends would (same block
 *       ids), and upload them; the first call also hands the position to the
 *       device.  Later calls extend the window.  Not capturable (async copies
 *       from pinned staging on s); run it before capture or between replays.
 *   genllm_apply_rope_step / genllm_paged_attention_step   capturable: kernel
 *       launches only, reading the position from the layer's device control
 *       block; the attention step appends this step's K/V, attends, and its
 *       last workgroup advances the position by seq_len.
 *   genllm_kv_sync_decode(kv, l, s, &n)   host: waits for s, reads the
 *       position back into num_cached and returns the staged blocks no step
 *       reached, in reverse order, so that the layer (tables, pools, free
 *       lists) is exactly what the same per-step appends would have left.
 *
 * While staged, num_cached / the page tables report the end of the window,
 * and the host-driven calls (paged_attention, append_pages, set_page_table,
 * block_alloc/free, qk_norm_rope_append) are refused with GENLLM_ERR_INVALID.
 * A step whose tokens would pass the window (or, for the attention step, the
 * window the step was planned for when it was captured) does nothing and
 * raises the layer's error flag, which genllm_kv_sync_decode reports as
 * GENLLM_ERR_POOL_FULL; later steps then do nothing either.  Steps of one layer
 * must run in stream order (one stream, or a graph replayed on it). */
int genllm_kv_stage_decode(genllm_kv *kv, int32_t layer, int32_t n_tokens, void *stream);
int genllm_kv_sync_decode(genllm_kv *kv, int32_t layer, void *stream, int32_t *num_cached);
/* PagedAttentionImpl::execute (attention.cpp:123-216) at the device position:
 * arguments as genllm_paged_attention; seq_len * n_kv_groups <= 16. */
int genllm_paged_attention_step(genllm_kv *kv, int32_t layer, const void *q, const void *k, const void *v,
                                void *out, int32_t batch, int32_t n_q_heads, int32_t seq_len, int32_t head_dim,
                                int32_t n_kv_heads, int32_t n_kv_groups, float scale, int32_t causal,
                                void *stream);
/* ApplyRopeImpl::execute (rope.cpp:76-119) with start_pos = the staged layer's
 * device position; arguments as genllm_apply_rope, and max_seq = the rows of
 * the cos/sin tables (a step past them raises the layer's error flag). */
int genllm_apply_rope_step(genllm_kv *kv, int32_t layer, void *out, const void *x, const float *cos_tab,
                           const float *sin_tab, int32_t n_heads, int32_t seq_len, int32_t head_dim,
                           int32_t rope_dim, int32_t max_seq, void *stream);

/* The Qwen3 layer's q/k per-head RMSNorm -> RoPE -> page scatter, fused
 * (src/model/Qwen3.cpp:137-166 = RmsNormImpl normalization.cpp:138-153, then
 * ApplyRopeImpl rope.cpp:76-119, then append_kv_from_tensor
 * page_attention.cpp:104-140), as one kernel.  Appends seq_len tokens at the
 * layer's num_cached; RoPE position of token t is rope_pos0 + t (op_params[2]).
 * k, v: token-major [seq_len][n_kv_heads][head_dim] (pre-permute), strides in
 * elements.  q (optional, NULL to skip) has its own strides and is written,
 * normed and rotated, to q_out.  gamma_k/gamma_q may be NULL (no norm);
 * cos_tab/sin_tab may be NULL (no RoPE); tables are [max_seq][rope_dim] fp32
 * as RopeCacheImpl builds them for rope_dim (the op's op_params[1],
 * op_factory.hpp:504-529): the first rope_dim dims rotate in pairs
 * (i, i + rope_dim/2), the others pass through.  rope_dim = head_dim is the
 * Qwen3 layer; Qwen3.5 rotates 64 of 256 (Qwen35.hpp:14-16).  rope_dim must
 * be a multiple of 64.  (The reference's ApplyRopeImpl ignores op_params[1]
 * and indexes the table with stride head_dim, rope.cpp:80-101, so its
 * partial form reads outside the table; that is not reproduced.) */
int genllm_qk_norm_rope_append(genllm_kv *kv, int32_t layer, int32_t seq_len,
                               const void *k, int64_t k_tok_stride, int64_t k_head_stride,
                               const void *v, int64_t v_tok_stride, int64_t v_head_stride,
                               const float *gamma_k, const void *q, int64_t q_tok_stride, int64_t q_head_stride,
                               int32_t n_q_heads, const float *gamma_q, void *q_out, int64_t qo_tok_stride,
                               int64_t qo_head_stride, float eps, const float *cos_tab, const float *sin_tab,
                               int32_t rope_dim, int64_t rope_pos0, void *stream);

/* --------------------------------------------------- stateless kernels */

/* RmsNormImpl<D>::execute (normalization.cpp:138-153 / rms_norm :44-107):
 * rows x hidden bf16, fp32 gamma; same fp32 summation order and stores
 * (truncation for whole 8-blocks, RNE for the tail) as the CPU op. */
int genllm_rms_norm(void *out, const void *x, const float *w, int64_t rows, int32_t hidden, float eps,
                    void *stream);
/* ApplyRopeImpl<D>::execute (rope.cpp:76-119): head-major [n_heads][seq_len][head_dim]
 * bf16, positions start_pos + s, op_params = {head_dim, rope_dim, start_pos}.
 * Tables [max_seq][rope_dim]; the first rope_dim dims rotate, the others are
 * copied (rope_dim = head_dim: the reference op; rope_dim even, <= head_dim). */
int genllm_apply_rope(void *out, const void *x, const float *cos_tab, const float *sin_tab, int32_t n_heads,
                      int32_t seq_len, int32_t head_dim, int32_t rope_dim, int64_t start_pos, void *stream);
/* RopeCacheImpl<CPU>::execute (rope.cpp:121-148) into host memory, in double
 * precision like the reference; the caller copies it to the device once. */
int genllm_rope_cache(float *host_dst, float theta, int32_t head_dim, int32_t max_seq, int32_t is_cos);

/* Page scatter of append_kv_from_tensor (page_attention.cpp:104-140) without
 * norm/RoPE: rows of token t (global position pos0 + t) go to page
 * k_ids[(pos0+t)/16], slot (pos0+t)%16.  Strides in elements. */
int genllm_kv_scatter(const void *k, int64_t k_tok_stride, int64_t k_head_stride, const void *v,
                      int64_t v_tok_stride, int64_t v_head_stride, void *k_pool, void *v_pool,
                      const int32_t *k_ids, const int32_t *v_ids, int32_t pos0, int32_t seq_len,
                      int32_t n_kv_heads, int32_t head_dim, void *stream);

/* Workspace for genllm_paged_decode: 1 KiB of per-kv-head arrival counters,
 * then fp32 partial (m, l, o) per split (at most 256 splits).  Zero-fill it
 * once before its first use (the counters must start at zero; every launch
 * leaves them at zero again).  Two launches sharing a workspace must be
 * ordered (same stream). */
size_t genllm_paged_decode_workspace_bytes(int32_t n_q_heads, int32_t n_kv_heads, int32_t seq_len,
                                           int32_t head_dim, int32_t max_pages);

/* The attention loop of PagedAttentionImpl (attention.cpp:148-215) for short
 * query chunks (seq_len * n_q_heads / n_kv_heads <= 16 rows per kv head):
 * split-K over pages, GQA rows packed per kv head, then a log-sum-exp merge of
 * the splits by a second kernel on the same stream (genllm_decode_tuning
 * selects a single-launch form).  q/out rows addressed as base + h*head_stride + s*tok_stride
 * (elements).  n_cached = total_cached; query s sits at n_cached - seq_len + s. */
int genllm_paged_decode(const void *q, int64_t q_head_stride, int64_t q_tok_stride, void *out,
                        int64_t o_head_stride, int64_t o_tok_stride, const void *k_pool, const void *v_pool,
                        const int32_t *k_ids, const int32_t *v_ids, int32_t n_pages, int32_t n_cached,
                        int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                        int32_t causal, void *workspace, size_t workspace_bytes, void *stream);

/* No counterpart in the reference: a tuning and test hook for the decode
 * kernels of this library (genllm_paged_decode, _noalloc, the op and its
 * device-position steps), process-wide, for later calls.  pages_per_split > 0
 * forces the split size (0: automatic, about one workgroup per CU).  merge:
 * 0 = a merge kernel after the split kernel (default), 1 = the last split
 * workgroup of each kv head to finish merges it in the same launch.
 * heads_per_workgroup: kv heads one split workgroup reads; 0 = automatic (4
 * for long page ranges, else 1), 1, or 4 (taken where head_dim is 128, the kv
 * heads come in groups of 4 and the merge runs in a kernel; else 1).  The
 * initial values come from GENLLM_DECODE_PPS, GENLLM_DECODE_MERGE (kernel |
 * fused) and GENLLM_DECODE_HEADS, read once.  Returns GENLLM_ERR_INVALID for
 * another merge or heads value. */
int genllm_decode_tuning(int32_t pages_per_split, int32_t merge, int32_t heads_per_workgroup);

/* No counterpart in the reference: genllm_paged_decode for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and kernels, no
 * workspace: the split partials and arrival counters live in a static device
 * scratch of GENLLM_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends.  The call allocates nothing; its first call on a device resolves that
 * device's scratch and clears its counters with a small kernel on `stream`.
 * A launch whose split plan needs more scratch (kv heads x splits x rows x
 * (head_dim + 2) x 4 bytes + 1 KiB; the Qwen3-4B decode needs about 0.5
 * MiB at 8K keys and 2.1 MiB from 32K keys on, where its plan takes 4 kv
 * heads per split workgroup and 128 splits) returns GENLLM_ERR_INVALID and
 * launches nothing.
 * Every call on a GPU shares that GPU's scratch: calls that overlap on one
 * GPU (different streams, threads) race; calls ordered on one stream do not. */
#define GENLLM_NOALLOC_SCRATCH_BYTES (4u << 20)
int genllm_paged_decode_noalloc(const void *q, int64_t q_head_stride, int64_t q_tok_stride, void *out,
                                int64_t o_head_stride, int64_t o_tok_stride, const void *k_pool, const void *v_pool,
                                const int32_t *k_ids, const int32_t *v_ids, int32_t n_pages, int32_t n_cached,
                                int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
                                float scale, int32_t causal, void *stream);

/* The same attention loop for long query chunks (prefill): bf16 MFMA
 * FlashAttention over page-gathered K/V tiles, causal with query s at
 * n_cached - seq_len + s. */
int genllm_paged_prefill(const void *q, int64_t q_head_stride, int64_t q_tok_stride, void *out,
                         int64_t o_head_stride, int64_t o_tok_stride, const void *k_pool, const void *v_pool,
                         const int32_t *k_ids, const int32_t *v_ids, int32_t n_pages, int32_t n_cached,
                         int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                         int32_t causal, void *stream);

/* FlashAttentionImpl<D>::execute (src/backend/cpu/attention.cpp:39-121,
 * src/backend/cuda/attention.cu:226-399): attention over the node's own K/V,
 * no cache (the op type of kv_cache_per_layer = 0, README.md:97).  q, out:
 * [batch][n_q_heads][seq_len][head_dim]; k, v: [batch][n_kv_heads][seq_len][head_dim],
 * contiguous bf16.  kv head = q head / n_kv_groups; causal masks key s_kv > s_q.
 * head_dim 128 or 256; any other returns GENLLM_ERR_UNSUPPORTED. */
int genllm_flash_attention(const void *q, const void *k, const void *v, void *out, int32_t batch,
                           int32_t n_q_heads, int32_t seq_len, int32_t n_kv_heads, int32_t head_dim,
                           int32_t n_kv_groups, float scale, int32_t causal, void *stream);

/* ---------------------------------------------------------------- linear
 * LinearImpl<D>::execute (src/backend/cpu/linear.cpp:46-122 and :325-345,
 * src/backend/cuda/linear.cu:72-126), the Q/K/V projections in front of the
 * attention op (Qwen3.cpp:130-134): out[r][c] = bf16(sum_k x[r][k] w[c][k] +
 * bias[c]) with x [rows][common], w [cols][common] (the reference's
 * transpose_w = 1 layout, one weight row per output), bias [cols] or NULL,
 * out [rows][cols], all bf16 on the device; fp32 accumulation, the bias added
 * in fp32, one rounding.  rows <= 4 with common % 8 == 0: the reference CPU
 * summation order exactly (bit-identical results) and no workspace.  Other
 * shapes: rocBLAS GEMM (fp32 accumulation in rocBLAS's order).  With a bias
 * it writes into an fp32 workspace of genllm_linear_workspace_bytes(rows,
 * common, cols) bytes (0 when none is needed; GENLLM_ERR_INVALID if it is
 * missing or smaller) and a second kernel adds the bias and rounds; without a
 * bias it rounds straight into out (round to nearest even; an fp32 subnormal
 * result stays a bf16 subnormal) and the workspace is not used. */
size_t genllm_linear_workspace_bytes(int64_t rows, int64_t common, int64_t cols);
int genllm_linear(const void *x, const void *w, const void *bias, void *out, int64_t rows, int64_t common,
                  int64_t cols, void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------ utilities
 * No counterpart in the reference: synthetic seeded inputs for tests and the
 * benchmark (counter-based hash -> Box-Muller -> RNE bf16, or RNE fp16 with
 * gradual underflow). */
int genllm_fill_normal_bf16(void *dst, size_t n, uint64_t seed, uint64_t offset, void *stream);
int genllm_fill_normal_f16(void *dst, size_t n, uint64_t seed, uint64_t offset, void *stream);

/* No counterpart in the reference: runs one bf16 MFMA, k = 32
 * (v_mfma_f32_16x16x32_bf16) or k = 16 (v_mfma_f32_16x16x16_bf16), on
 * a[16][k], b[k][16] (bf16, device) into c[16][16] (fp32, device) through the
 * operand layouts the kernels assume; the tests compare it with a host matrix
 * product. */
int genllm_selftest_mfma(int32_t k, const void *a, const void *b, float *c, void *stream);

#ifdef __cplusplus
}
#endif
#endif
