// manager.cpp -- MemoryManager slice and the scheduler's KV sizing rules
// (src/core/manager.cpp:16-20, 97-116; src/core/scheduler.cpp:62-79, 363-372,
// 404-430).
#include "genllm/manager.hpp"

#include <stdexcept>

MemoryManager* g_mem_manager = nullptr;

MemoryManager::MemoryManager() { g_mem_manager = this; }

MemoryManager::~MemoryManager() {
    attention_managers_.clear();
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
