// kernels.hpp -- kernel:: entry points and device::dispatchOp with the HIP
// case (include/core/kernels.h:17-39, src/core/kernels.cpp:47-76,
// include/utils/dtype_traits.hpp:76-88), and the executor's op switch for the
// ops of this path (src/core/executor.cpp:475-505).
#pragma once

#include <stdexcept>
#include <string>

#include "genllm/backend/hip/ops.hpp"
#include "genllm/tensor.hpp"

namespace device {

// Only the HIP backend is compiled into this library; other devices throw
// like the reference's default case.
template <typename Fn>
void dispatchOp(Device device, Fn&& fn) {
    switch (device) {
        case Device::HIP: fn.template operator()<Device::HIP>(); break;
        default:
            throw std::runtime_error(std::string("device::dispatchOp: unsupported device ") +
                                     device_to_string(device));
    }
}

}  // namespace device

namespace kernel {

void rms_norm(Tensor* out, int32_t dev_id = 0);
void apply_rope(Tensor* out, int32_t dev_id = 0);
void rope_cache(Tensor* out, int32_t dev_id = 0);
void paged_attention(Tensor* out, int32_t dev_id = 0);  // append + attend over the paged cache
void flash_attention(Tensor* out, int32_t dev_id = 0);  // attention over the node's own K/V
void linear(Tensor* out, int32_t dev_id = 0);           // the Q/K/V projections feeding the attention

// Executor::dispatch_kernel for these op types; false for any other op type.
bool dispatch(Tensor* t, int32_t dev_id = 0);

}  // namespace kernel
