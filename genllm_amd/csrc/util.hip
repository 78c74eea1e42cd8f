// util.hip -- synthetic seeded inputs and the MFMA operand-layout self-test.
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

// Counter-based normal generator: h = mix64(seed + i * golden), two 24-bit
// uniforms u1 in (0,1], u2 in [0,1), z = sqrt(-2 ln u1) cos(2 pi u2) in fp32,
// rounded to bf16 like bfloat16_t or to fp16 like float16_t (RNE).
// genllm_amd/synth.py computes the same formula on the host.
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

template <bool F16>
__global__ void fill_normal_kernel(uint16_t* dst, size_t n, uint64_t seed, uint64_t offset) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t h = mix64(seed + (offset + i) * 0x9E3779B97F4A7C15ull);
        const float u1 = float((h >> 40) + 1) * (1.0f / 16777216.0f);
        const float u2 = float((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
        const float r = sqrtf(-2.0f * logf(u1));
        const float z = r * cosf(6.2831853071795864f * u2);
        dst[i] = uint16_t(F16 ? f32_to_f16_ref(z) : f32_to_bf16_ref(z));
    }
}

// One bf16 MFMA with the operand layouts the kernels rely on, K = 32
// (v_mfma_f32_16x16x32_bf16) or K = 16 (v_mfma_f32_16x16x16_bf16):
// lane l gives A[l%16][kk(l/16)..+kk-1] and B[kk(l/16)..+kk-1][l%16] with
// kk = K/4; D[4(l/16)+i][l%16] comes back in register i.

__global__ void selftest_mfma_kernel(const uint16_t* a, const uint16_t* b, float* c, int K) {
    const int l = threadIdx.x;
    const int r = l & 15, g = l >> 4;
    const int kk = K / 4;
    uint16_t aa[8], bb[8];
    for (int j = 0; j < kk; ++j) {
        aa[j] = a[r * K + kk * g + j];
        bb[j] = b[(kk * g + j) * 16 + r];
    }
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (K == 32) {
        const uint4 ua = make_uint4(pack2(aa[0], aa[1]), pack2(aa[2], aa[3]), pack2(aa[4], aa[5]), pack2(aa[6], aa[7]));
        const uint4 ub = make_uint4(pack2(bb[0], bb[1]), pack2(bb[2], bb[3]), pack2(bb[4], bb[5]), pack2(bb[6], bb[7]));
        acc = mfma16x16x32(as_bf16x8(ua), as_bf16x8(ub), acc);
    } else {
        const s16x4_t sa = __builtin_bit_cast(s16x4_t, make_uint2(pack2(aa[0], aa[1]), pack2(aa[2], aa[3])));
        const s16x4_t sb = __builtin_bit_cast(s16x4_t, make_uint2(pack2(bb[0], bb[1]), pack2(bb[2], bb[3])));
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(sa, sb, acc, 0, 0, 0);
    }
    for (int i = 0; i < 4; ++i) c[(4 * g + i) * 16 + r] = acc[i];
}

}  // namespace genllm

using namespace genllm;

namespace {
template <bool F16>
int fill_normal(void* dst, size_t n, uint64_t seed, uint64_t offset, void* stream) {
    if (n == 0) return GENLLM_OK;
    if (!dst) return fail(GENLLM_ERR_INVALID, "fill_normal: null dst");
    const size_t blocks = std::min<size_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(fill_normal_kernel<F16>, dim3(unsigned(blocks)), dim3(256), 0, as_stream(stream),
                       static_cast<uint16_t*>(dst), n, seed, offset);
    GENLLM_LAUNCH_CHECK("fill_normal_kernel");
    return GENLLM_OK;
}
}  // namespace

extern "C" int genllm_fill_normal_bf16(void* dst, size_t n, uint64_t seed, uint64_t offset, void* stream) {
    return fill_normal<false>(dst, n, seed, offset, stream);
}

extern "C" int genllm_fill_normal_f16(void* dst, size_t n, uint64_t seed, uint64_t offset, void* stream) {
    return fill_normal<true>(dst, n, seed, offset, stream);
}

extern "C" int genllm_selftest_mfma(int32_t k, const void* a, const void* b, float* c, void* stream) {
    if (!a || !b || !c) return fail(GENLLM_ERR_INVALID, "selftest_mfma: null pointer");
    if (k != 16 && k != 32) return fail(GENLLM_ERR_INVALID, "selftest_mfma: k must be 16 or 32");
    hipLaunchKernelGGL(selftest_mfma_kernel, dim3(1), dim3(64), 0, as_stream(stream),
                       static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), c, int(k));
    GENLLM_LAUNCH_CHECK("selftest_mfma_kernel");
    return GENLLM_OK;
}
