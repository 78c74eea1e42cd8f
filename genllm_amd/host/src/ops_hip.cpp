// ops_hip.cpp -- ops::*Impl<Device::HIP>::execute and the kernel:: entry
// points.  Each execute() reads the node as the CPU op does (file:line at
// each function) and calls the C ABI of libgenllm_hip.so on the device's
// stream; no host synchronisation (stream order replaces the reference's
// per-op cudaDeviceSynchronize, src/core/executor.cpp:169-173).
#include "genllm/backend/hip/ops.hpp"

#include <hip/hip_runtime_api.h>

#include <map>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "genllm/kernels.hpp"
#include "genllm/manager.hpp"
#include "genllm_paged.h"

namespace {

void* device_stream(const Tensor* out, int32_t dev_id) {
    return g_mem_manager ? g_mem_manager->stream(out->device, size_t(dev_id)) : nullptr;
}

void require_bf16(const Tensor* t, const char* op) {
    if (!t || t->dtype != DataType::GGML_TYPE_BF16)
        throw std::runtime_error(std::string(op) + ": HIP kernels take bf16 tensors");
}

}  // namespace

namespace ops {

// src/backend/cpu/attention.cpp:123-216, src/backend/cuda/attention.cu:491-580
void PagedAttentionImpl<Device::HIP>::execute(Tensor* out, int32_t dev_id) {
    auto* mgr = g_mem_manager ? g_mem_manager->get_attention_manager(out->device, size_t(dev_id)) : nullptr;
    const int32_t layer_id = out->layer_id;
    if (!mgr || !mgr->is_active(layer_id)) return;

    const Tensor* Q = out->src[0];
    const Tensor* K = out->src[1];
    const Tensor* V = out->src[2];
    // q, k, v and out are of the layer's element type, bf16 or fp16 (the
    // reference reads K/V as Q's dtype, attention.cpp:186-200)
    genllm_layer_info info{};
    genllm_check(genllm_kv_layer_info(mgr->handle(), layer_id, &info), "paged_attention");
    const DataType dt = static_cast<DataType>(info.dtype);
    if (dt != DataType::GGML_TYPE_BF16 && dt != DataType::GGML_TYPE_F16)
        throw std::runtime_error("paged_attention: HIP kernels take bf16 or f16 layers");
    for (const Tensor* t : {Q, K, V, static_cast<const Tensor*>(out)})
        if (!t || t->dtype != dt) throw std::runtime_error("paged_attention: tensor dtype differs from the layer's");

    const int32_t batch = int32_t(Q->dims[0]);
    const int32_t num_q_heads = int32_t(Q->dims[1]);
    const int32_t seq_len = int32_t(Q->dims[2]);
    const int32_t head_dim = int32_t(Q->dims[3]);
    const int32_t num_kv_heads = int32_t(K->dims[1]);
    const int32_t num_kv_groups = int32_t(out->op_params[3]);
    const float scale = out->op_params[1];
    const bool causal = int32_t(out->op_params[2]) != 0;

    mgr->commit_layer(layer_id);  // edits of a get_layer view (a no-op without one)
    // a staged layer (device-position decode) reads its position on the device
    auto* const entry = mgr->is_staged(layer_id) ? genllm_paged_attention_step : genllm_paged_attention;
    genllm_check(entry(mgr->handle(), layer_id, Q->data, K->data, V->data, out->data, batch, num_q_heads, seq_len,
                       head_dim, num_kv_heads, num_kv_groups, scale, causal ? 1 : 0, mgr->stream()),
                 "paged_attention");
    mgr->refresh_layer(layer_id);  // the op appended the chunk: keep get_layer's view current
}

// src/backend/cpu/attention.cpp:39-121
void FlashAttentionImpl<Device::HIP>::execute(Tensor* out, int32_t dev_id) {
    const Tensor* Q = out->src[0];
    const Tensor* K = out->src[1];
    const Tensor* V = out->src[2];
    for (const Tensor* t : {Q, K, V, static_cast<const Tensor*>(out)}) require_bf16(t, "flash_attention");

    const int32_t batch = int32_t(Q->dims[0]);
    const int32_t num_q_heads = int32_t(Q->dims[1]);
    const int32_t seq_len = int32_t(Q->dims[2]);
    const int32_t n_kv_h = int32_t(K->dims[1]);
    const int32_t head_dim = int32_t(out->op_params[0]);
    const int32_t num_kv_groups = int32_t(out->op_params[3]);
    const float scale = out->op_params[1];
    const bool causal = int32_t(out->op_params[2]) != 0;
    if (head_dim != int32_t(Q->dims[3]))
        throw std::runtime_error("flash_attention: op_params[0] differs from Q's head_dim");

    genllm_check(genllm_flash_attention(Q->data, K->data, V->data, out->data, batch, num_q_heads, seq_len, n_kv_h,
                                        head_dim, num_kv_groups, scale, causal ? 1 : 0,
                                        device_stream(out, dev_id)),
                 "flash_attention");
}

// src/backend/cpu/normalization.cpp:138-153
void RmsNormImpl<Device::HIP>::execute(Tensor* out, int32_t dev_id) {
    const Tensor* x = out->src[0];
    const Tensor* w = out->src[1];
    require_bf16(x, "rms_norm");
    require_bf16(out, "rms_norm");
    if (!w || w->dtype != DataType::GGML_TYPE_F32) throw std::runtime_error("rms_norm: gamma must be fp32");
    const float eps = out->op_params[0];
    const size_t hidden_size = w->num_elements();
    const size_t total_tokens = x->num_elements() / hidden_size;
    genllm_check(genllm_rms_norm(out->data, x->data, static_cast<const float*>(w->data), int64_t(total_tokens),
                                 int32_t(hidden_size), eps, device_stream(out, dev_id)),
                 "rms_norm");
}

// src/backend/cpu/rope.cpp:76-119
void ApplyRopeImpl<Device::HIP>::execute(Tensor* out, int32_t dev_id) {
    const Tensor* x = out->src[0];
    const Tensor* cos = out->src[1];
    const Tensor* sin = out->src[2];
    require_bf16(x, "apply_rope");
    require_bf16(out, "apply_rope");
    const int64_t head_dim = int64_t(out->op_params[0]);
    // op_params[1] = rope_dim, the width of the tables (op_factory.hpp:504-529);
    // the reference op reads it but indexes with head_dim, so only
    // rope_dim == head_dim matches it -- a smaller one rotates the leading dims
    const int64_t rope_dim = out->op_params[1] > 0 ? int64_t(out->op_params[1]) : head_dim;
    const int64_t start_pos = int64_t(out->op_params[2]);
    const int64_t B = x->dims[0], n_heads = x->dims[1], seq_len = x->dims[2];
    if (B != 1) throw std::runtime_error("apply_rope: batch must be 1");  // rope.cpp:89 asserts it
    // a node of a staged layer takes start_pos from the device position
    auto* mgr = g_mem_manager && out->layer_id >= 0 ? g_mem_manager->get_attention_manager(out->device, size_t(dev_id))
                                                    : nullptr;
    if (mgr && mgr->is_staged(out->layer_id)) {
        const int64_t max_seq = int64_t(cos->num_elements()) / rope_dim;
        genllm_check(genllm_apply_rope_step(mgr->handle(), out->layer_id, out->data, x->data,
                                            static_cast<const float*>(cos->data), static_cast<const float*>(sin->data),
                                            int32_t(n_heads), int32_t(seq_len), int32_t(head_dim), int32_t(rope_dim),
                                            int32_t(max_seq), mgr->stream()),
                     "apply_rope");
        return;
    }
    genllm_check(genllm_apply_rope(out->data, x->data, static_cast<const float*>(cos->data),
                                   static_cast<const float*>(sin->data), int32_t(n_heads), int32_t(seq_len),
                                   int32_t(head_dim), int32_t(rope_dim), start_pos, device_stream(out, dev_id)),
                 "apply_rope");
}

// src/backend/cpu/rope.cpp:121-148
void RopeCacheImpl<Device::HIP>::execute(Tensor* out, int32_t dev_id) {
    const float theta = out->op_params[0];
    const int32_t head_dim = int32_t(out->op_params[1]);
    const int32_t max_seq = int32_t(out->op_params[2]);
    const bool is_cos = out->name.find("_cos") != std::string::npos;
    std::vector<float> host(size_t(max_seq) * size_t(head_dim));
    genllm_check(genllm_rope_cache(host.data(), theta, head_dim, max_seq, is_cos ? 1 : 0), "rope_cache");
    hipStream_t s = static_cast<hipStream_t>(device_stream(out, dev_id));
    if (hipMemcpyAsync(out->data, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        throw std::runtime_error("rope_cache: copy to the device failed");
}

// src/backend/cpu/linear.cpp:325-345 (batch 1, transpose_w), linear.cu:72-126
void LinearImpl<Device::HIP>::execute(Tensor* out, int32_t dev_id) {
    const Tensor* x = out->src[0];
    const Tensor* w = out->src[1];
    const Tensor* bias = out->src[2];
    require_bf16(x, "linear");
    require_bf16(w, "linear");
    require_bf16(out, "linear");
    if (int32_t(out->op_params[0]) != 1) throw std::runtime_error("linear: only transpose_w = 1 is supported");
    if (x->dims[0] != 1) throw std::runtime_error("linear: batch must be 1");  // linear.cpp:332 asserts it
    const int64_t rows = x->dims[1], common = x->dims[2], cols = w->dims[0];
    const void* bp = bias && bias->data ? bias->data : nullptr;
    if (bp) require_bf16(bias, "linear");
    void* stream = device_stream(out, dev_id);
    // fp32 workspace of the GEMM path with a bias: the device's op workspace,
    // reserved before execution (MemoryManager::reserve_op_workspace); the op
    // itself never allocates
    const size_t need = bp ? genllm_linear_workspace_bytes(rows, common, cols) : 0;  // used only with a bias
    size_t have = 0;
    void* ws = g_mem_manager ? g_mem_manager->op_workspace(out->device, size_t(dev_id), &have) : nullptr;
    if (need > have)
        throw std::runtime_error("linear: this call needs " + std::to_string(need) +
                                 " bytes of op workspace, the device has " + std::to_string(have) +
                                 " reserved (MemoryManager::reserve_op_workspace, op_workspace_bytes)");
    genllm_check(genllm_linear(x->data, w->data, bp, out->data, rows, common, cols, ws, have, stream), "linear");
}

}  // namespace ops

namespace kernel {

// src/core/kernels.cpp:47-80
void rms_norm(Tensor* t, int32_t dev_id) {
    device::dispatchOp(t->device, [&]<Device D>() { ops::RmsNormImpl<D>::execute(t, dev_id); });
}
void apply_rope(Tensor* t, int32_t dev_id) {
    device::dispatchOp(t->device, [&]<Device D>() { ops::ApplyRopeImpl<D>::execute(t, dev_id); });
}
void rope_cache(Tensor* t, int32_t dev_id) {
    device::dispatchOp(t->device, [&]<Device D>() { ops::RopeCacheImpl<D>::execute(t, dev_id); });
}
void paged_attention(Tensor* t, int32_t dev_id) {
    device::dispatchOp(t->device, [&]<Device D>() { ops::PagedAttentionImpl<D>::execute(t, dev_id); });
}
void flash_attention(Tensor* t, int32_t dev_id) {
    device::dispatchOp(t->device, [&]<Device D>() { ops::FlashAttentionImpl<D>::execute(t, dev_id); });
}
void linear(Tensor* t, int32_t dev_id) {
    device::dispatchOp(t->device, [&]<Device D>() { ops::LinearImpl<D>::execute(t, dev_id); });
}

// src/core/executor.cpp:475-505
bool dispatch(Tensor* t, int32_t dev_id) {
    switch (t->op_type) {
        case OperationType::OP_TYPE_RMS_NORM: rms_norm(t, dev_id); return true;
        case OperationType::OP_TYPE_APPLY_ROPE: apply_rope(t, dev_id); return true;
        case OperationType::OP_TYPE_ROPE_CACHE: rope_cache(t, dev_id); return true;
        case OperationType::OP_TYPE_FLASH_ATTN: flash_attention(t, dev_id); return true;
        case OperationType::OP_TYPE_PAGED_ATTN: paged_attention(t, dev_id); return true;
        case OperationType::OP_TYPE_LINEAR: linear(t, dev_id); return true;
        default: return false;
    }
}

}  // namespace kernel
