// page_attention.cpp -- PagedAttentionManager / BlockPool of the HIP backend
// over the native manager (include/genllm_paged.h).  Method-by-method the
// reference is src/core/page_attention.cpp:25-216.
#include "genllm/page_attention.hpp"

#include <stdexcept>
#include <string>

#include "genllm_paged.h"

void genllm_check(int status, const char* what) {
    if (status != GENLLM_OK) throw std::runtime_error(std::string(what) + ": " + genllm_last_error());
}

namespace {
// A manager call on one layer: edits of the layer's get_layer view are
// committed first, and the view is re-read when the call ends, also when it
// throws after a partial change (a scatter failing after its pages opened).
struct ViewRefresh {
    PagedAttentionManager& mgr;
    int32_t layer;
    ViewRefresh(PagedAttentionManager& m, int32_t l) : mgr(m), layer(l) { mgr.commit_layer(layer); }
    ~ViewRefresh() {
        try {
            mgr.refresh_layer(layer);
        } catch (...) {  // the call's own error is the one that propagates
        }
    }
};

bool same_table(const std::vector<PageEntry>& a, const std::vector<PageEntry>& b) {
    if (a.size() != b.size()) return false;
    for (size_t i = 0; i < a.size(); ++i)
        if (a[i].k_block_id != b[i].k_block_id || a[i].v_block_id != b[i].v_block_id) return false;
    return true;
}
}  // namespace

// ------------------------------------------------------------- BlockPool
int32_t BlockPool::alloc() {
    int32_t id = -1;
    genllm_check(genllm_kv_block_alloc(kv_, layer_, which_, &id), "BlockPool::alloc");
    return id;
}

void BlockPool::free(int32_t block_id) {
    genllm_check(genllm_kv_block_free(kv_, layer_, which_, block_id), "BlockPool::free");
}

void* BlockPool::block_data(int32_t block_id) const {
    genllm_layer_info info;
    genllm_check(genllm_kv_layer_info(kv_, layer_, &info), "BlockPool::block_data");
    const int32_t n = which_ ? info.v_num_blocks : info.k_num_blocks;
    void* base = which_ ? info.v_pool : info.k_pool;
    if (block_id < 0 || block_id >= n || !base) return nullptr;  // page_attention.cpp:59-63
    return static_cast<char*>(base) + size_t(block_id) * info.block_bytes;
}

int32_t BlockPool::num_blocks() const {
    genllm_layer_info info;
    genllm_check(genllm_kv_layer_info(kv_, layer_, &info), "BlockPool::num_blocks");
    return which_ ? info.v_num_blocks : info.k_num_blocks;
}

int32_t BlockPool::num_free() const {
    genllm_layer_info info;
    genllm_check(genllm_kv_layer_info(kv_, layer_, &info), "BlockPool::num_free");
    return which_ ? info.v_num_free : info.k_num_free;
}

// ------------------------------------------------- PagedAttentionManager
PagedAttentionManager::PagedAttentionManager(int32_t device, size_t kv_pool_bytes) : device_(device) {
    genllm_check(genllm_kv_create(device, kv_pool_bytes, &kv_), "PagedAttentionManager");
}

PagedAttentionManager::~PagedAttentionManager() {
    if (kv_) genllm_kv_destroy(kv_);
}

void PagedAttentionManager::read_layer(int32_t layer_id, LayerState& s) const {
    genllm_layer_info info;
    genllm_check(genllm_kv_layer_info(kv_, layer_id, &info), "get_layer");
    s.active = info.active != 0;
    s.num_cached = info.num_cached;
    s.n_kv_heads = info.n_kv_heads;
    s.head_dim = info.head_dim;
    s.dtype = static_cast<DataType>(info.dtype);
    s.k_pool = BlockPool(kv_, layer_id, 0);
    s.v_pool = BlockPool(kv_, layer_id, 1);
    std::vector<int32_t> k(size_t(info.num_pages)), v(size_t(info.num_pages));
    int32_t n = 0;
    genllm_check(genllm_kv_page_table(kv_, layer_id, k.data(), v.data(), info.num_pages, &n), "get_layer");
    s.page_table.resize(size_t(n));
    for (int32_t i = 0; i < n; ++i) s.page_table[size_t(i)] = PageEntry{k[size_t(i)], v[size_t(i)]};
}

PagedAttentionManager::LayerState& PagedAttentionManager::get_layer(int32_t layer_id) {
    commit_layer(layer_id);
    LayerState s;
    read_layer(layer_id, s);  // throws for an unknown layer before a view exists
    LayerState& view = views_[layer_id];
    view = std::move(s);
    synced_[layer_id] = Synced{view.num_cached, view.page_table};
    return view;
}

void PagedAttentionManager::commit_layer(int32_t layer_id) {
    auto it = views_.find(layer_id);
    if (it == views_.end()) return;
    const LayerState& v = it->second;
    Synced& was = synced_[layer_id];
    if (v.num_cached == was.num_cached && same_table(v.page_table, was.page_table)) return;
    set_table_native(layer_id, v.page_table, v.num_cached);
    was = Synced{v.num_cached, v.page_table};
}

void PagedAttentionManager::refresh_layer(int32_t layer_id) {
    auto it = views_.find(layer_id);
    if (it == views_.end()) return;
    read_layer(layer_id, it->second);
    synced_[layer_id] = Synced{it->second.num_cached, it->second.page_table};
}

void PagedAttentionManager::refresh_views() {
    for (auto& [id, view] : views_) refresh_layer(id);
}

void PagedAttentionManager::set_page_table(int32_t layer_id, const std::vector<PageEntry>& table,
                                           int32_t num_cached) {
    ViewRefresh refresh{*this, layer_id};
    set_table_native(layer_id, table, num_cached);
}

void PagedAttentionManager::set_table_native(int32_t layer_id, const std::vector<PageEntry>& table,
                                             int32_t num_cached) {
    std::vector<int32_t> k(table.size()), v(table.size());
    for (size_t i = 0; i < table.size(); ++i) {
        k[i] = table[i].k_block_id;
        v[i] = table[i].v_block_id;
    }
    genllm_check(genllm_kv_set_page_table(kv_, layer_id, k.data(), v.data(), int32_t(table.size()), num_cached,
                                          stream_),
                 "set_page_table");
}

void PagedAttentionManager::reserve_layer(int32_t layer_id, int32_t max_blocks) {
    ViewRefresh refresh{*this, layer_id};
    genllm_check(genllm_kv_reserve_layer(kv_, layer_id, max_blocks), "reserve_layer");
}

void PagedAttentionManager::init_layer(int32_t layer_id, int32_t n_kv_heads, int32_t head_dim, DataType dtype) {
    ViewRefresh refresh{*this, layer_id};
    genllm_check(genllm_kv_init_layer(kv_, layer_id, n_kv_heads, head_dim, int32_t(dtype)), "init_layer");
}

void PagedAttentionManager::append_kv_from_tensor(int32_t layer_id, const void* K_data, const void* V_data,
                                                  int32_t n_kv_heads, int32_t seq_len, int32_t head_dim,
                                                  DataType dtype) {
    ViewRefresh refresh{*this, layer_id};
    genllm_layer_info info;
    genllm_check(genllm_kv_layer_info(kv_, layer_id, &info), "append_kv_from_tensor");
    if (!info.active || seq_len <= 0) return;  // page_attention.cpp:106-107
    if (dtype != static_cast<DataType>(info.dtype) || n_kv_heads != info.n_kv_heads || head_dim != info.head_dim)
        throw std::runtime_error("append_kv_from_tensor: tensor shape/dtype differs from the layer's pools");
    const int32_t pos0 = info.num_cached;
    genllm_check(genllm_kv_append_pages(kv_, layer_id, seq_len, stream_), "append_kv_from_tensor");
    genllm_check(genllm_kv_layer_info(kv_, layer_id, &info), "append_kv_from_tensor");
    // source layout [n_kv_heads][seq_len][head_dim] (page_attention.cpp:118-129)
    genllm_check(genllm_kv_scatter(K_data, head_dim, int64_t(seq_len) * head_dim, V_data, head_dim,
                                   int64_t(seq_len) * head_dim, info.k_pool, info.v_pool, info.k_ids, info.v_ids,
                                   pos0, seq_len, n_kv_heads, head_dim, stream_),
                 "append_kv_from_tensor");
}

void PagedAttentionManager::append_kv_from_pos(int32_t layer_id, const void* K_data, const void* V_data,
                                               int32_t n_kv_heads, int32_t head_dim, DataType dtype,
                                               int32_t global_pos, int32_t count) {
    ViewRefresh refresh{*this, layer_id};
    genllm_check(genllm_kv_append_from_pos(kv_, layer_id, K_data, V_data, n_kv_heads, head_dim, int32_t(dtype),
                                           global_pos, count, stream_),
                 "append_kv_from_pos");
}

void PagedAttentionManager::append_kv_pages(int32_t layer_id, int32_t count) {
    ViewRefresh refresh{*this, layer_id};
    genllm_check(genllm_kv_append_pages(kv_, layer_id, count, stream_), "append_kv_pages");
}

void PagedAttentionManager::reset() {
    // pending view edits are dropped with the rest of the state (page_attention.cpp:208-216)
    genllm_check(genllm_kv_reset(kv_), "reset");
    staged_.clear();  // the native reset leaves every layer host-driven
    refresh_views();
}

void PagedAttentionManager::stage_decode(int32_t layer_id, int32_t n_tokens) {
    ViewRefresh refresh{*this, layer_id};
    genllm_check(genllm_kv_stage_decode(kv_, layer_id, n_tokens, stream_), "stage_decode");
    staged_.insert(layer_id);
}

int32_t PagedAttentionManager::sync_decode(int32_t layer_id) {
    ViewRefresh refresh{*this, layer_id};
    int32_t n = 0;
    const int rc = genllm_kv_sync_decode(kv_, layer_id, stream_, &n);
    staged_.erase(layer_id);  // synced even when it reports a refused step
    genllm_check(rc, "sync_decode");
    return n;
}

bool PagedAttentionManager::is_active(int32_t layer_id) const {
    int32_t a = 0;
    genllm_check(genllm_kv_is_active(kv_, layer_id, &a), "is_active");
    return a != 0;
}
