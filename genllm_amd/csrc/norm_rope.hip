// norm_rope.hip -- the stand-alone RMSNorm and RoPE ops of the path.
//
// RmsNormImpl<CPU> / rms_norm, src/backend/cpu/normalization.cpp:44-107,138-153,
// for any row width: one wave per row; lane a < 32 runs running sum a of the
// CPU op (element e feeds sum e % 32 over whole 32-blocks, fused multiply-add),
// then lanes 0..7 combine (A[k]+A[8+k])+(A[16+k]+A[24+k]), fuse the remaining
// 8-blocks, reduce ((T0+T4)+(T1+T5))+((T2+T6)+(T3+T7)), and lane 0 adds the
// scalar tail with fused multiply-adds -- the reference's order exactly.
// Whole 8-blocks are stored by truncation, the tail by RNE (as the CPU op).
//
// ApplyRopeImpl<CPU>, src/backend/cpu/rope.cpp:76-119: one thread per NeoX pair
// (i, i + D/2) of a head-major [H][S][D] row at position start_pos + s.
#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

#pragma clang fp contract(off)

__global__ __launch_bounds__(256) void rms_norm_kernel(uint16_t* out, const uint16_t* x, const float* w,
                                                       int64_t rows, int hidden, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const uint16_t* xr = x + row * hidden;
    uint16_t* orow = out + row * hidden;
    const int n32 = hidden / 32;
    float A = 0.0f;
    if (lane < 32)
        for (int b = 0; b < n32; ++b) {
            const float v = bf16_to_f32(xr[32 * b + lane]);
            A = __builtin_fmaf(v, v, A);
        }
    const float a1 = __shfl(A, (lane + 8) & 63);
    const float a2 = __shfl(A, (lane + 16) & 63);
    const float a3 = __shfl(A, (lane + 24) & 63);
    float T = (A + a1) + (a2 + a3);  // meaningful on lanes 0..7
    int j = n32 * 32;
    for (; j + 8 <= hidden; j += 8)
        if (lane < 8) {
            const float v = bf16_to_f32(xr[j + lane]);
            T = __builtin_fmaf(v, v, T);
        }
    const float u = T + __shfl(T, (lane + 4) & 63);  // lanes 0..3: u[lane]
    const float u1 = __shfl(u, 1), u2 = __shfl(u, 2), u3 = __shfl(u, 3);
    float ss = (u + u1) + (u2 + u3);
    if (lane == 0)
        for (int t = j; t < hidden; ++t) {
            const float v = bf16_to_f32(xr[t]);
            ss = __builtin_fmaf(v, v, ss);
        }
    ss = __shfl(ss, 0);
    const float r = 1.0f / __builtin_sqrtf(ss / float(hidden) + eps);
    const int vec_end = (hidden / 8) * 8;
    for (int e = lane; e < hidden; e += 64) {
        const float y = (bf16_to_f32(xr[e]) * r) * w[e];
        orow[e] = uint16_t(e < vec_end ? f32_to_bf16_trunc(y) : f32_to_bf16_ref(y));
    }
}

// One thread per slot i < head_dim/2 of a row.  Slots below rope_dim/2 rotate
// the pair (i, i + rope_dim/2) with table entry [pos][i] (rows of rope_dim
// floats); slot i >= rope_dim/2 copies the two elements rope_dim + 2(i -
// rope_dim/2) + {0, 1} unchanged.  rope_dim == head_dim is the reference op.
// With `ctl` (a device-position decode step) the start position is the
// control block's pos; a step whose rows would pass the table's max_seq rows
// raises the block's error flag and writes nothing, as does any step after a
// refused one (the flag stays set until the host syncs the layer).
template <bool kDevPos>
__global__ __launch_bounds__(256) void apply_rope_kernel(uint16_t* out, const uint16_t* x, const float* cos_tab,
                                                         const float* sin_tab, int64_t rows, int seq_len,
                                                         int head_dim, int rope_dim, int64_t start_pos,
                                                         int32_t* ctl, int64_t max_seq) {
    const int half = head_dim / 2, rhalf = rope_dim / 2;
    if constexpr (kDevPos) {
        start_pos = __builtin_amdgcn_readfirstlane(
            __hip_atomic_load(ctl + kStepPos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (__hip_atomic_load(ctl + kStepError, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return;
        if (start_pos < 0 || start_pos + seq_len > max_seq) {
            if (blockIdx.x == 0 && threadIdx.x == 0)
                __hip_atomic_store(ctl + kStepError, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= rows * half) return;
    const int64_t row = idx / half;
    const int i = int(idx - row * half);
    const uint16_t* xr = x + row * head_dim;
    uint16_t* orow = out + row * head_dim;
    if (i >= rhalf) {
        const int e = rope_dim + 2 * (i - rhalf);
        orow[e] = xr[e];
        orow[e + 1] = xr[e + 1];
        return;
    }
    const int64_t pos = start_pos + row % seq_len;
    const float c = cos_tab[pos * rope_dim + i], s = sin_tab[pos * rope_dim + i];
    const float x0 = bf16_to_f32(xr[i]);
    const float x1 = bf16_to_f32(xr[i + rhalf]);
    orow[i] = uint16_t(f32_to_bf16_ref(__builtin_fmaf(x0, c, -(x1 * s))));
    orow[i + rhalf] = uint16_t(f32_to_bf16_ref(__builtin_fmaf(x0, s, x1 * c)));
}

int launch_rms_norm(uint16_t* out, const uint16_t* x, const float* w, int64_t rows, int hidden, float eps,
                    hipStream_t stream) {
    if (rows <= 0) return GENLLM_OK;
    const int64_t blocks = (rows + 3) / 4;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream, out, x, w, rows, hidden, eps);
    GENLLM_LAUNCH_CHECK("rms_norm_kernel");
    return GENLLM_OK;
}

int launch_apply_rope(uint16_t* out, const uint16_t* x, const float* cos_tab, const float* sin_tab, int n_heads,
                      int seq_len, int head_dim, int rope_dim, int64_t start_pos, hipStream_t stream, int32_t* ctl,
                      int64_t max_seq) {
    const int64_t rows = int64_t(n_heads) * seq_len;
    const int64_t n = rows * (head_dim / 2);
    if (n <= 0) return GENLLM_OK;
    const int64_t blocks = (n + 255) / 256;
    if (ctl)
        hipLaunchKernelGGL(apply_rope_kernel<true>, dim3(unsigned(blocks)), dim3(256), 0, stream, out, x, cos_tab,
                           sin_tab, rows, seq_len, head_dim, rope_dim, int64_t(0), ctl, max_seq);
    else
        hipLaunchKernelGGL(apply_rope_kernel<false>, dim3(unsigned(blocks)), dim3(256), 0, stream, out, x, cos_tab,
                           sin_tab, rows, seq_len, head_dim, rope_dim, start_pos, ctl, max_seq);
    GENLLM_LAUNCH_CHECK("apply_rope_kernel");
    return GENLLM_OK;
}

}  // namespace genllm
