// manager.cpp -- MemoryManager slice and the scheduler's KV sizing rules
// (src/core/manager.cpp:16-20, 97-116; src/core/scheduler.cpp:62-79, 363-372,
// 404-430).
#include "genllm/manager.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <stdexcept>
#include <string>

#include "genllm_paged.h"

MemoryManager* g_mem_manager = nullptr;

MemoryManager::MemoryManager() { g_mem_manager = this; }

MemoryManager::~MemoryManager() {
    attention_managers_.clear();
    for (auto& [key, ws] : workspaces_)
        if (ws.first && hipSetDevice(int(key.second)) == hipSuccess) {
            (void)hipDeviceSynchronize();
            (void)hipFree(ws.first);
        }
    if (g_mem_manager == this) g_mem_manager = nullptr;
}

PagedAttentionManager* MemoryManager::get_attention_manager(Device dev, size_t dev_id) {
    auto it = attention_managers_.find({dev, dev_id});
    return it == attention_managers_.end() ? nullptr : it->second.get();
}

PagedAttentionManager& MemoryManager::create_attention_manager(Device dev, size_t dev_id, size_t kv_pool_bytes) {
    if (dev != Device::HIP) throw std::runtime_error("create_attention_manager: this library manages HIP devices only");
    auto& slot = attention_managers_[{dev, dev_id}];
    if (!slot) {
        slot = std::make_unique<PagedAttentionManager>(int32_t(dev_id), kv_pool_bytes);
        slot->set_stream(stream(dev, dev_id));
    }
    return *slot;
}

void MemoryManager::reset_kv_cache() {
    for (auto& [key, pam] : attention_managers_) pam->reset();
}

void MemoryManager::set_stream(Device dev, size_t dev_id, void* s) {
    streams_[{dev, dev_id}] = s;
    if (auto* pam = get_attention_manager(dev, dev_id)) pam->set_stream(s);
}

void* MemoryManager::stream(Device dev, size_t dev_id) const {
    auto it = streams_.find({dev, dev_id});
    return it == streams_.end() ? nullptr : it->second;
}

void MemoryManager::reserve_op_workspace(Device dev, size_t dev_id, size_t bytes) {
    if (dev != Device::HIP) throw std::runtime_error("reserve_op_workspace: this library manages HIP devices only");
    auto& ws = workspaces_[{dev, dev_id}];
    if (bytes <= ws.second) return;
    if (hipSetDevice(int(dev_id)) != hipSuccess) throw std::runtime_error("reserve_op_workspace: hipSetDevice failed");
    if (ws.first) {
        if (hipDeviceSynchronize() != hipSuccess || hipFree(ws.first) != hipSuccess)
            throw std::runtime_error("reserve_op_workspace: releasing the old workspace failed");
        ws = {nullptr, 0};
    }
    if (hipMalloc(&ws.first, bytes) != hipSuccess)
        throw std::runtime_error("reserve_op_workspace: allocation of " + std::to_string(bytes) + " bytes failed");
    ws.second = bytes;
}

void* MemoryManager::op_workspace(Device dev, size_t dev_id, size_t* bytes) const {
    auto it = workspaces_.find({dev, dev_id});
    const bool have = it != workspaces_.end();
    if (bytes) *bytes = have ? it->second.second : 0;
    return have ? it->second.first : nullptr;
}

// ------------------------------------------------------------- scheduler
namespace {
int32_t max_blocks_for(int32_t max_seq_len) { return (max_seq_len + PAGE_BLOCK_SIZE - 1) / PAGE_BLOCK_SIZE; }
bool owns_pages(const Tensor* t) { return t->op_type == OperationType::OP_TYPE_PAGED_ATTN && t->src[1]; }
}  // namespace

size_t kv_cache_bytes(const std::vector<Tensor*>& nodes, Device dev, int32_t max_seq_len, float pool_factor) {
    const size_t max_blocks = size_t(max_blocks_for(max_seq_len));
    size_t total = 0;
    for (const Tensor* t : nodes) {
        if (!owns_pages(t) || t->device != dev) continue;
        const size_t block_bytes =
            size_t(PAGE_BLOCK_SIZE) * size_t(t->src[1]->dims[1]) * size_t(t->dims[3]) * data_type_size(t->dtype);
        total += size_t(double(2 * max_blocks * block_bytes) * pool_factor);
    }
    return total;
}

void initialize_kv_cache(PagedAttentionManager& pam, const std::vector<Tensor*>& nodes, int32_t max_seq_len) {
    const int32_t max_blocks = max_blocks_for(max_seq_len);
    for (const Tensor* t : nodes) {
        if (!owns_pages(t)) continue;
        pam.init_layer(t->layer_id, int32_t(t->src[1]->dims[1]), int32_t(t->dims[3]), t->dtype);
        pam.reserve_layer(t->layer_id, max_blocks);
    }
}

size_t op_workspace_bytes(const std::vector<Tensor*>& nodes, Device dev, int64_t max_rows) {
    size_t need = 0;
    for (const Tensor* t : nodes) {
        if (t->op_type != OperationType::OP_TYPE_LINEAR || t->device != dev || !t->src[0] || !t->src[1]) continue;
        const bool bias = t->src[2] && t->src[2]->data;
        if (!bias) continue;  // without a bias the GEMM rounds straight into the output
        const int64_t common = t->src[0]->dims[2], cols = t->src[1]->dims[0];
        need = std::max(need, genllm_linear_workspace_bytes(max_rows, common, cols));
    }
    return need;
}
