// page_attention.hpp -- PagedAttentionManager for HIP devices: the reference's
// interface (include/core/page_attention.h:9-90) over the native manager of
// libgenllm_hip.so (genllm_kv, include/genllm_paged.h).
//
// The K/V pools and a device-resident copy of each layer's page table live in
// one HBM allocation per device (the kv_cache MemoryPool).  Host bookkeeping
// (BlockPool free lists, PageEntry tables, num_cached) follows the reference
// rule for rule; the differences are explicit errors where the reference
// silently truncates (a full pool) or dereferences a missing layer.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <set>
#include <vector>

#include "genllm/tensor.hpp"

struct genllm_kv;

constexpr int32_t PAGE_BLOCK_SIZE = 16;  // include/core/page_attention.h:9

struct PageEntry {  // include/core/page_attention.h:47-50
    int32_t k_block_id;
    int32_t v_block_id;
};

// One of a layer's two BlockPools (page_attention.h:11-45) seen from the host:
// alloc/free/num_blocks/num_free act on the native pool.
class BlockPool {
public:
    BlockPool() = default;
    BlockPool(genllm_kv* kv, int32_t layer, int32_t which) : kv_(kv), layer_(layer), which_(which) {}

    [[nodiscard]] int32_t alloc();         // -1 when full, as page_attention.cpp:37-44
    void free(int32_t block_id);           // ids >= num_blocks are ignored, :46-50
    [[nodiscard]] void* block_data(int32_t block_id) const;  // device address; nullptr past num_blocks
    int32_t num_blocks() const;
    int32_t num_free() const;
    bool empty() const { return num_blocks() == 0; }

private:
    genllm_kv* kv_ = nullptr;
    int32_t layer_ = -1;
    int32_t which_ = 0;  // 0 = K pool, 1 = V pool
};

class PagedAttentionManager {
public:
    // One native manager on `device` whose kv_cache pool holds kv_pool_bytes
    // (pools + page tables of every layer it will reserve).
    PagedAttentionManager(int32_t device, size_t kv_pool_bytes);
    ~PagedAttentionManager();
    PagedAttentionManager(const PagedAttentionManager&) = delete;
    PagedAttentionManager& operator=(const PagedAttentionManager&) = delete;

    // page_attention.h:57-66
    struct LayerState {
        bool active = false;
        int32_t num_cached = 0;
        int32_t n_kv_heads = 0;
        int32_t head_dim = 0;
        DataType dtype = DataType::GGML_TYPE_F32;
        BlockPool k_pool;
        BlockPool v_pool;
        std::vector<PageEntry> page_table;
    };

    // page_attention.h:68.  The reference hands out a mutable reference into
    // its layer map: later calls show through it (test_page_attention.cpp:53-61
    // reads num_cached and page_table after append_kv_pages), and a caller may
    // set page_table / num_cached in place.  The state lives in the native
    // manager here, so get_layer returns a view that this manager keeps in step
    // both ways: an edit of the view's page_table or num_cached is committed
    // (genllm_kv_set_page_table, with its checks) before the next call of this
    // manager or PAGED_ATTN node on that layer, and the view is re-read after
    // each of them.  The other fields are read-only in effect.  A native call
    // made around this manager (genllm_kv_* on handle()) shows in the view at
    // its next refresh_layer or get_layer.
    [[nodiscard]] LayerState& get_layer(int32_t layer_id);
    // Commits edits of layer_id's view, then re-reads it; both are no-ops
    // unless get_layer has handed out a view of that layer, so the decode path
    // pays nothing while nobody holds one.
    void commit_layer(int32_t layer_id);
    void refresh_layer(int32_t layer_id);
    void set_page_table(int32_t layer_id, const std::vector<PageEntry>& table, int32_t num_cached);

    void reserve_layer(int32_t layer_id, int32_t max_blocks);                                      // :81-101
    void init_layer(int32_t layer_id, int32_t n_kv_heads, int32_t head_dim, DataType dtype);         // :72-79
    // :104-140 -- K_data/V_data are device pointers, head-major [n_kv_heads][seq_len][head_dim]
    void append_kv_from_tensor(int32_t layer_id, const void* K_data, const void* V_data, int32_t n_kv_heads,
                               int32_t seq_len, int32_t head_dim, DataType dtype);
    // :164-203 -- K_data/V_data device pointers, head-major [n_kv_heads][count][head_dim] (every head
    // reads its own rows; the reference reads head 0's for all); errors leave the layer unchanged
    void append_kv_from_pos(int32_t layer_id, const void* K_data, const void* V_data, int32_t n_kv_heads,
                            int32_t head_dim, DataType dtype, int32_t global_pos, int32_t count);
    void append_kv_pages(int32_t layer_id, int32_t count);                                          // :141-162
    void reset();                                                                                   // :208-216
    // Device-position decode for a HIP-graph-captured decode loop (no counterpart
    // in the reference, whose executor advances the position on the host,
    // executor.cpp:227-236): stage_decode opens the pages of the next n_tokens
    // positions and hands the layer's position to the device; while a layer is
    // staged, its PagedAttentionImpl / ApplyRopeImpl nodes take the position from
    // the device (capturable); sync_decode reads it back and returns num_cached.
    void stage_decode(int32_t layer_id, int32_t n_tokens);
    int32_t sync_decode(int32_t layer_id);
    bool is_staged(int32_t layer_id) const { return staged_.count(layer_id) != 0; }
    bool is_active(int32_t layer_id) const;                                                         // .h:82-85

    genllm_kv* handle() const { return kv_; }
    int32_t device() const { return device_; }
    // Stream every call of this manager (and the ops using it) is ordered on;
    // nullptr = the device's null stream.
    void* stream() const { return stream_; }
    void set_stream(void* stream) { stream_ = stream; }

private:
    genllm_kv* kv_ = nullptr;
    int32_t device_ = 0;
    void* stream_ = nullptr;
    std::set<int32_t> staged_;
    std::map<int32_t, LayerState> views_;  // node-stable: get_layer's references stay valid
    struct Synced {                        // the native state a view last matched
        int32_t num_cached = 0;
        std::vector<PageEntry> page_table;
    };
    std::map<int32_t, Synced> synced_;
    void read_layer(int32_t layer_id, LayerState& s) const;
    void refresh_views();
    void set_table_native(int32_t layer_id, const std::vector<PageEntry>& table, int32_t num_cached);
};

// Throws std::runtime_error carrying genllm_last_error() when status != 0.
void genllm_check(int status, const char* what);
