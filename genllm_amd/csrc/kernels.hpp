// kernels.hpp -- launch parameter blocks and launchers of the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace genllm {

// Device page-table entries opened by this call, passed by value in the launch
// arguments so that no copy precedes the kernel; the kernel writes them into
// the device table.
template <int N>
struct TableUpdateN {
    int32_t first = 0;
    int32_t count = 0;
    int32_t k[N] = {};
    int32_t v[N] = {};
};
using TableUpdate = TableUpdateN<4>;  // decode step: at most 16 queries open at most 2 pages
constexpr int kAppendUpdMax = 256;    // append chunk: up to 4096 tokens (2 KiB of ids)
using AppendTableUpdate = TableUpdateN<kAppendUpdMax>;

struct AppendParams {
    const uint16_t* k = nullptr;
    int64_t k_tok_stride = 0, k_head_stride = 0;
    const uint16_t* v = nullptr;
    int64_t v_tok_stride = 0, v_head_stride = 0;
    const uint16_t* q = nullptr;
    int64_t q_tok_stride = 0, q_head_stride = 0;
    uint16_t* q_out = nullptr;
    int64_t qo_tok_stride = 0, qo_head_stride = 0;
    const float* gamma_k = nullptr;
    const float* gamma_q = nullptr;
    float eps = 0.0f;
    const float* cos_tab = nullptr;
    const float* sin_tab = nullptr;
    int64_t rope_stride = 0;  // elements per table row (= the rotated dims)
    int64_t rope_pos0 = 0;
    int32_t rope_dim = 0;     // leading dims rotated (pairs i, i + rope_dim/2); the rest pass through
    int32_t S = 0, Hkv = 0, Hq = 0;
    int32_t pos0 = 0;         // cache position of token 0
    int32_t nq_tasks = 0, nkv_tasks = 0;
    uint16_t* k_pool = nullptr;
    uint16_t* v_pool = nullptr;
    int64_t page_elems = 0;   // 16 * Hkv * D
    int32_t* k_ids = nullptr;
    int32_t* v_ids = nullptr;
    int32_t max_blocks = INT32_MAX;  // ids outside [0, max_blocks) are never written through
    AppendTableUpdate upd;
};
int launch_kv_append(const AppendParams& p, int head_dim, hipStream_t stream);

struct AttnParams {
    const uint16_t* q = nullptr;
    int64_t q_head_stride = 0, q_tok_stride = 0;
    uint16_t* out = nullptr;
    int64_t o_head_stride = 0, o_tok_stride = 0;
    const uint16_t* k_pool = nullptr;
    const uint16_t* v_pool = nullptr;
    const int32_t* k_ids = nullptr;
    const int32_t* v_ids = nullptr;
    int32_t n_pages = 0;      // pages holding tokens < n_cached
    int32_t n_cached = 0;
    int32_t S = 0, Hq = 0, Hkv = 0, G = 0;
    float scale_log2 = 0.0f;  // scale * log2(e)
    // causal and the element type share one 32-bit word: a larger argument
    // block (296 instead of 288 bytes, the fields after it moved) measured 0.16
    // us slower per config-3 decode
    int16_t causal = 1;
    int16_t f16 = 0;          // element type of q, the pools and out: 0 bf16, 1 fp16
    int64_t page_elems = 0;
    int64_t kv_row = 0;       // elements between consecutive tokens in a page (Hkv * D)
    // Elements between kv heads (0 = head_dim, the page layout [16][Hkv][D]).
    // With k_ids == v_ids == nullptr page i is block i: a contiguous head-major
    // [Hkv][S][D] tensor is then kv_head_stride = S*D, kv_row = D,
    // page_elems = 16*D (non-paged attention; prefill kernel only).
    int64_t kv_head_stride = 0;
    // split-K decode: per-split partials [unit][split][row][D] then {m, l} per (unit, split, row)
    float* partial = nullptr;
    int32_t pages_per_split = 0, n_splits = 1;
    int32_t heads_per_wg = 1;  // kv heads per split workgroup (1, or 4 for long page ranges)
    // Single-launch merge: per-kv-head arrival counters (zero between
    // launches); the last split workgroup of a head to arrive merges them.
    // nullptr = merge in a second kernel.
    int32_t* counters = nullptr;
    // Device-position step (graph-capturable decode): control block
    // {pos, limit, arrivals, error} (kStep* indices).  When set, the kernel
    // reads the cache position from it -- n_cached = pos + S, new_from = pos,
    // pages = ceil(n_cached / 16) -- instead of n_cached / new_from / n_pages,
    // which then only size the plan (n_pages = the most pages a step may
    // span).  A step past `limit` (or past n_pages) sets `error` and does
    // nothing; otherwise the merge kernel advances pos by S (without one, the
    // last split workgroup to finish does).
    int32_t* step = nullptr;
    // fused append (decode of the op): tokens at positions >= new_from are read
    // from k_new / v_new ([Hkv][S][D], strides in elements) instead of the
    // pools and written into the pools by the wave that reads their page; page
    // ids opened by this call come in `upd` and are written to the tables.
    const uint16_t* k_new = nullptr;
    const uint16_t* v_new = nullptr;
    int64_t new_head_stride = 0, new_tok_stride = 0;
    int32_t new_from = INT32_MAX;
    uint16_t* k_pool_w = nullptr;  // writable aliases of k_pool / v_pool
    uint16_t* v_pool_w = nullptr;
    int32_t* k_ids_w = nullptr;
    int32_t* v_ids_w = nullptr;
    TableUpdate upd;
};

// Workspace layout of the split-K decode: kDecodeCounterBytes of per-kv-head
// arrival counters (must be zero before the first launch; every launch leaves
// them at zero), then the per-split partials.
constexpr size_t kDecodeCounterBytes = 1024;
constexpr int kDecodeMaxKvHeads = int(kDecodeCounterBytes / sizeof(int32_t));
// Device-position step control block (int32 indices); arrivals and error
// must be zero before the first step.
constexpr int kStepPos = 0, kStepLimit = 1, kStepArrivals = 2, kStepError = 3, kStepInts = 4;
size_t decode_workspace_bytes(int Hq, int Hkv, int S, int D, int n_pages);
// Decode merge forms (genllm_decode_tuning)
constexpr int kDecodeMergeKernel = 0, kDecodeMergeFused = 1;
int set_decode_tuning(int pages_per_split, int merge, int heads_per_wg);
int decode_plan(AttnParams& p, int D, size_t ws_bytes, void* ws);
int launch_paged_decode(const AttnParams& p, int head_dim, hipStream_t stream);
int launch_paged_prefill(const AttnParams& p, int head_dim, hipStream_t stream);

int launch_rms_norm(uint16_t* out, const uint16_t* x, const float* w, int64_t rows, int hidden, float eps,
                    hipStream_t stream);
// ctl != nullptr: start position from a device-position step control block
// (start_pos ignored), checked against the table's max_seq rows.
int launch_apply_rope(uint16_t* out, const uint16_t* x, const float* cos_tab, const float* sin_tab, int n_heads,
                      int seq_len, int head_dim, int rope_dim, int64_t start_pos, hipStream_t stream,
                      int32_t* ctl = nullptr, int64_t max_seq = 0);

}  // namespace genllm
