// manager.hpp -- the slice of MemoryManager the attention ops reach through
// g_mem_manager (include/core/manager.h:30-60, src/core/manager.cpp:16-20,
// 97-116): one PagedAttentionManager per (device, dev_id), a kv-cache reset,
// and the HIP stream the device's ops are ordered on.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <utility>
#include <vector>

#include "genllm/page_attention.hpp"
#include "genllm/tensor.hpp"

class MemoryManager {
public:
    MemoryManager();   // registers itself as g_mem_manager (manager.cpp:20)
    ~MemoryManager();  // unregisters
    MemoryManager(const MemoryManager&) = delete;
    MemoryManager& operator=(const MemoryManager&) = delete;

    // manager.h:56-57.  kv_pool_bytes sizes the device's kv_cache pool (the
    // reference takes it from DevicePools::kv_cache, created beforehand).
    [[nodiscard]] PagedAttentionManager* get_attention_manager(Device dev, size_t dev_id);
    PagedAttentionManager& create_attention_manager(Device dev, size_t dev_id, size_t kv_pool_bytes);

    void reset_kv_cache();  // manager.cpp:97-101

    // HIP stream of a device (nullptr = null stream); attention managers of
    // that device follow it.
    void set_stream(Device dev, size_t dev_id, void* stream);
    void* stream(Device dev, size_t dev_id) const;

    // Device scratch of the ops that need one (the GEMM path of LinearImpl
    // with a bias), reserved before execution -- size it with
    // op_workspace_bytes -- so that no op allocates, frees or synchronises.
    // Growing it waits for the device and replaces the buffer.
    void reserve_op_workspace(Device dev, size_t dev_id, size_t bytes);
    void* op_workspace(Device dev, size_t dev_id, size_t* bytes) const;

private:
    using DevKey = std::pair<Device, size_t>;
    std::map<DevKey, std::unique_ptr<PagedAttentionManager>> attention_managers_;
    std::map<DevKey, void*> streams_;
    std::map<DevKey, std::pair<void*, size_t>> workspaces_;
};

extern MemoryManager* g_mem_manager;

// GraphScheduler's KV rules (src/core/scheduler.cpp:62-79, 363-372, 404-430):
// every OP_TYPE_PAGED_ATTN node with a K source owns a layer of
// ceil(max_seq_len / 16) pages; n_kv_heads = src[1]->dims[1], head_dim =
// dims[3], dtype = the node's dtype.  Nodes of OP_TYPE_FLASH_ATTN (the
// kv_cache_per_layer = 0 configuration) own no pages.
size_t kv_cache_bytes(const std::vector<Tensor*>& nodes, Device dev, int32_t max_seq_len, float pool_factor = 1.0f);
void initialize_kv_cache(PagedAttentionManager& pam, const std::vector<Tensor*>& nodes, int32_t max_seq_len);

// Op workspace the nodes of `dev` need with up to max_rows rows (tokens) per
// call: the largest genllm_linear_workspace_bytes over its LINEAR nodes.
size_t op_workspace_bytes(const std::vector<Tensor*>& nodes, Device dev, int64_t max_rows);

// README.md:97 -- kv_cache_per_layer: 0 = standard attention, >= 1 = paged
// attention; the op type an attention node is built with.
inline OperationType attention_op_type(int32_t kv_cache_per_layer) {
    return kv_cache_per_layer >= 1 ? OperationType::OP_TYPE_PAGED_ATTN : OperationType::OP_TYPE_FLASH_ATTN;
}
