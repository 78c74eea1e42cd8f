// util.hip -- synthetic seeded inputs and the MFMA operand-layout self-test.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

// Counter-based normal generator: h = mix64(seed + i * golden), two 24-bit
// uniforms u1 in (0,1], u2 in [0,1), z = sqrt(-2 ln u1) cos(2 pi u2) in fp32,
// rounded to bf16 like bfloat16_t (RNE).  genllm_amd/synth.py computes the same
// formula on the host.
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__global__ void fill_normal_kernel(uint16_t* dst, size_t n, uint64_t seed, uint64_t offset) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t h = mix64(seed + (offset + i) * 0x9E3779B97F4A7C15ull);
        const float u1 = float((h >> 40) + 1) * (1.0f / 16777216.0f);
        const float u2 = float((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
        const float r = sqrtf(-2.0f * logf(u1));
        const float z = r * cosf(6.2831853071795864f * u2);
        dst[i] = uint16_t(f32_to_bf16_ref(z));
    }
}

// One 16x16x32 bf16 MFMA with the operand layouts the kernels rely on:
// lane l gives A[l%16][8(l/16)..+7] and B[8(l/16)..+7][l%16]; D[4(l/16)+i][l%16]
// comes back in register i.
__global__ void selftest_mfma_kernel(const uint16_t* a, const uint16_t* b, float* c) {
    const int l = threadIdx.x;
    const int r = l & 15, g = l >> 4;
    uint4 ua = *reinterpret_cast<const uint4*>(a + r * 32 + 8 * g);
    uint16_t bb[8];
    for (int j = 0; j < 8; ++j) bb[j] = b[(8 * g + j) * 16 + r];
    uint4 ub = make_uint4(pack2(bb[0], bb[1]), pack2(bb[2], bb[3]), pack2(bb[4], bb[5]), pack2(bb[6], bb[7]));
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    acc = mfma16x16x32(as_bf16x8(ua), as_bf16x8(ub), acc);
    for (int i = 0; i < 4; ++i) c[(4 * g + i) * 16 + r] = acc[i];
}

}  // namespace genllm

using namespace genllm;

extern "C" int genllm_fill_normal_bf16(void* dst, size_t n, uint64_t seed, uint64_t offset, void* stream) {
    if (n == 0) return GENLLM_OK;
    if (!dst) return fail(GENLLM_ERR_INVALID, "fill_normal: null dst");
    const size_t blocks = std::min<size_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(fill_normal_kernel, dim3(unsigned(blocks)), dim3(256), 0, as_stream(stream),
                       static_cast<uint16_t*>(dst), n, seed, offset);
    GENLLM_LAUNCH_CHECK("fill_normal_kernel");
    return GENLLM_OK;
}

extern "C" int genllm_selftest_mfma(const void* a, const void* b, float* c, void* stream) {
    if (!a || !b || !c) return fail(GENLLM_ERR_INVALID, "selftest_mfma: null pointer");
    hipLaunchKernelGGL(selftest_mfma_kernel, dim3(1), dim3(64), 0, as_stream(stream),
                       static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), c);
    GENLLM_LAUNCH_CHECK("selftest_mfma_kernel");
    return GENLLM_OK;
}
