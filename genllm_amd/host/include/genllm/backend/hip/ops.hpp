// ops.hpp -- the HIP specialisations of the reference's operator templates
// (include/backend/cpu/attention.h:7-27, normalization.h:7-20, rope.h:6-20).
// Each execute() reads the graph node exactly as the CPU/CUDA versions do and
// calls libgenllm_hip.so; a non-zero status becomes std::runtime_error.
#pragma once

#include <cstdint>

#include "genllm/tensor.hpp"

namespace ops {

template <Device D> struct PagedAttentionImpl;
template <Device D> struct FlashAttentionImpl;
template <Device D> struct RmsNormImpl;
template <Device D> struct ApplyRopeImpl;
template <Device D> struct RopeCacheImpl;
template <Device D> struct LinearImpl;

// src = {Q [1,Hq,S,D], K [1,Hkv,S,D], V [1,Hkv,S,D]}, op_params = {head_dim,
// scale, causal, groups}; appends K/V to layer out->layer_id, then attends
// (src/backend/cpu/attention.cpp:123-216).
template <> struct PagedAttentionImpl<Device::HIP> {
    static void execute(Tensor* out, int32_t dev_id);
};

// Non-paged attention over the node's own K/V (attention.cpp:39-121):
// src = {Q [B,Hq,S,D], K, V [B,Hkv,S,D]}, op_params = {head_dim, scale,
// causal, groups}; causal masks key s_kv > s_q.
template <> struct FlashAttentionImpl<Device::HIP> {
    static void execute(Tensor* out, int32_t dev_id);
};

// src = {x, gamma (fp32)}, op_params[0] = eps (normalization.cpp:138-153).
template <> struct RmsNormImpl<Device::HIP> {
    static void execute(Tensor* out, int32_t dev_id);
};

// src = {x [1,H,S,D], cos, sin [max_seq,D] fp32}, op_params = {head_dim,
// rope_dim, start_pos} (rope.cpp:76-119).
template <> struct ApplyRopeImpl<Device::HIP> {
    static void execute(Tensor* out, int32_t dev_id);
};

// op_params = {theta, head_dim, max_seq}; the cos table when the node's name
// contains "_cos", else sin (rope.cpp:121-148).  Computed in double on the
// host like the reference, then copied to out->data.
template <> struct RopeCacheImpl<Device::HIP> {
    static void execute(Tensor* out, int32_t dev_id);
};

// src = {x [1,M,common] bf16, w [cols,common] bf16, bias [cols] or null},
// op_params[0] = transpose_w (must be 1, as the CPU op asserts), out
// [1,M,cols] (linear.cpp:325-345, linear.cu:72-126).  Decode-sized M runs the
// reference's summation order exactly; larger M a rocBLAS GEMM whose fp32
// workspace this backend keeps per device.
template <> struct LinearImpl<Device::HIP> {
    static void execute(Tensor* out, int32_t dev_id);
};

}  // namespace ops
