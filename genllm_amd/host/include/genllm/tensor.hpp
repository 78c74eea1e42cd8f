// tensor.hpp -- the graph-node fields the attention path reads, with the
// reference's names and enum values (include/core/tensor.hpp:12-52,
// include/utils/utils.hpp:6-110), plus Device::HIP for the MI355X backend.
//
// Only the parts an operator's execute() touches are kept: data, src, layer_id,
// device, dtype, op_type, dims, op_params, strides, name.  The reference's
// value for each enumerator is kept so that graphs and op_params mean the
// same thing on both sides.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <string>

// include/utils/utils.hpp:6-12; value 2 is unused there and becomes the HIP
// backend (CPU = 0, CUDA = 1, VULKAN = 4 are pinned by tests/test_tensor.cpp:72-76).
enum class Device : uint8_t {
    CPU = 0,
    CUDA = 1,
    HIP = 2,
    SYCL = 3,
    VULKAN = 4,
    UNKNOWN = 255
};

inline const char* device_to_string(Device d) {
    switch (d) {
        case Device::CPU: return "CPU";
        case Device::CUDA: return "CUDA";
        case Device::HIP: return "HIP";
        case Device::SYCL: return "SYCL";
        case Device::VULKAN: return "VULKAN";
        default: return "UNKNOWN";
    }
}

// include/utils/utils.hpp:30-59 (the three types this path sees).
enum class DataType : uint8_t {
    GGML_TYPE_F32 = 0,
    GGML_TYPE_F16 = 1,
    GGML_TYPE_BF16 = 30,
};

inline size_t data_type_size(DataType t) {
    switch (t) {
        case DataType::GGML_TYPE_F32: return 4;
        case DataType::GGML_TYPE_F16:
        case DataType::GGML_TYPE_BF16: return 2;
    }
    return 0;
}

// include/utils/utils.hpp:16-28
enum class TensorType : uint8_t {
    TENSOR_TYPE_UNKNOWN = 0,
    TENSOR_TYPE_WEIGHT,
    TENSOR_TYPE_CACHE,
    TENSOR_TYPE_KV_CACHE,
    TENSOR_TYPE_INPUT,
    TENSOR_TYPE_ACTIVATION,
    TENSOR_TYPE_OUTPUT,
    TENSOR_TYPE_VIEW,
};

// include/utils/utils.hpp:80-110, same order (so the same values).
enum class OperationType : uint8_t {
    OP_TYPE_NONE,
    OP_TYPE_MEMCPY,
    OP_TYPE_ADD,
    OP_TYPE_SUB,
    OP_TYPE_MUL,
    OP_TYPE_DIV,
    OP_TYPE_MAT_MUL,
    OP_TYPE_TRANSPOSE,
    OP_TYPE_RESHAPE,
    OP_TYPE_PERMUTE,
    OP_TYPE_VIEW,
    OP_TYPE_CONCAT,
    OP_TYPE_REPEAT,
    OP_TYPE_SOFTMAX,
    OP_TYPE_RMS_NORM,
    OP_TYPE_LAYER_NORM,
    OP_TYPE_GELU,
    OP_TYPE_SILU,
    OP_TYPE_RELU,
    OP_TYPE_EMBEDDING,
    OP_TYPE_LINEAR,
    OP_TYPE_APPLY_ROPE,
    OP_TYPE_ROPE_CACHE,
    OP_TYPE_FLASH_ATTN,
    OP_TYPE_PAGED_ATTN,
    OP_TYPE_CAUSAL_CONV1D,
    OP_TYPE_SSM_SCAN,
    OP_TYPE_NARROW,
    OP_TYPE_SIGMOID
};

constexpr int32_t TENSOR_MAX_SRC = 6;
constexpr int32_t TENSOR_MAX_DIMS = 4;
constexpr int32_t TENSOR_MAX_OP_PARAMS = 4;

// include/core/tensor.hpp:12-52.  For Device::HIP, `data` is a device pointer.
struct Tensor {
    void* data = nullptr;
    size_t offset = 0;
    std::array<Tensor*, TENSOR_MAX_SRC> src = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};

    int layer_id = -1;
    size_t device_handle = 0;
    Device device = Device::CPU;
    DataType dtype = DataType::GGML_TYPE_F32;
    TensorType type = TensorType::TENSOR_TYPE_UNKNOWN;
    OperationType op_type = OperationType::OP_TYPE_NONE;
    std::array<int64_t, TENSOR_MAX_DIMS> dims = {0, 0, 0, 0};
    std::array<float, TENSOR_MAX_OP_PARAMS> op_params = {0, 0, 0, 0};
    std::array<uint64_t, TENSOR_MAX_DIMS> strides = {0, 0, 0, 0};  // bytes per step of each dim
    std::string name;

    size_t num_elements() const {
        size_t total = 1;
        for (int i = 0; i < TENSOR_MAX_DIMS && dims[i] != 0; ++i) total *= static_cast<size_t>(std::llabs(dims[i]));
        return total;
    }
    size_t bytes() const { return num_elements() * data_type_size(dtype); }
};
