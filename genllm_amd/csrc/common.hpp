// common.hpp -- shared device helpers and host error plumbing for the gfx950
// paged-attention library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/genllm_paged.h"

namespace genllm {

constexpr int kPage = GENLLM_PAGE_BLOCK_SIZE;  // tokens per page
constexpr int kWave = 64;                      // CDNA wavefront

// ------------------------------------------------------------------ errors
// Thread-local message for genllm_last_error(); `fail` records and returns.
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

#define GENLLM_HIP_TRY(expr)                                   \
    do {                                                       \
        hipError_t _e = (expr);                                \
        if (_e != hipSuccess) return ::genllm::hip_fail(_e, #expr); \
    } while (0)

// Launch status check (configuration errors show up immediately).
#define GENLLM_LAUNCH_CHECK(name)                                       \
    do {                                                                \
        hipError_t _e = hipGetLastError();                              \
        if (_e != hipSuccess) return ::genllm::hip_fail(_e, name " launch"); \
    } while (0)

// ------------------------------------------------------------------- bf16
// bf16 -> fp32 is a 16-bit shift (include/utils/bfloat16.hpp:42-45).
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// fp32 -> bf16 exactly as bfloat16_t's constructor (bfloat16.hpp:18-41):
// inf/NaN -> sign|0x7F80|(mantissa!=0), exponent 0 (zero, subnormal) -> signed
// zero, else round to nearest even with carry (overflow reaches infinity).
__device__ __forceinline__ uint32_t f32_to_bf16_ref(float f) {
    uint32_t u = __float_as_uint(f);
    uint32_t e = u & 0x7F800000u;
    uint32_t rne = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    uint32_t special = ((u >> 16) & 0x8000u) | 0x7F80u | ((u & 0x7FFFFFu) ? 1u : 0u);
    uint32_t zero = (u >> 16) & 0x8000u;
    return e == 0x7F800000u ? special : (e == 0u ? zero : rne);
}
// Truncating store of the CPU rms_norm's 8-wide part (normalization.cpp:25-31).
__device__ __forceinline__ uint32_t f32_to_bf16_trunc(float f) { return __float_as_uint(f) >> 16; }

__device__ __forceinline__ uint32_t pack2(uint32_t lo, uint32_t hi) { return (lo & 0xFFFFu) | (hi << 16); }

// ----------------------------------------------------------- DPP reductions
// Row (16-lane) butterflies with DPP: quad_perm [1,0,3,2], [2,3,0,1], then
// half-row mirror and row mirror.  After the four steps every lane of the
// 16-lane row holds the reduction over the row.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp<kDppQuadXor1>(x));
    x = fmaxf(x, dpp<kDppQuadXor2>(x));
    x = fmaxf(x, dpp<kDppRowHalfMirror>(x));
    x = fmaxf(x, dpp<kDppRowMirror>(x));
    return x;
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp<kDppQuadXor1>(x);
    x += dpp<kDppQuadXor2>(x);
    x += dpp<kDppRowHalfMirror>(x);
    x += dpp<kDppRowMirror>(x);
    return x;
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

// s_waitcnt operand (gfx9 encoding) for "vmcnt(0)", leaving the LDS/scalar
// and export counters unconstrained: vmcnt bits [3:0] and [15:14] = 0,
// expcnt [6:4] = 7, lgkmcnt [11:8] = 15.
constexpr int kWaitVmcnt0 = 0x0F70;

// Buffer resource word 3 for raw (untyped) buffer accesses on gfx9-family
// GPUs: 32-bit data format, no swizzle, no index addressing.  Loads at or
// past the resource's size return zeros.
constexpr int kBufferFlags = 0x00020000;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));  // MFMA A/B operand (8 bf16 per lane)
typedef float f32x4_t __attribute__((ext_vector_type(4)));    // 16x16 MFMA C/D (4 fp32 per lane)

// 16 bytes of bf16 bit patterns <-> MFMA operand
__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& u) { return __builtin_bit_cast(bf16x8_t, u); }

__device__ __forceinline__ f32x4_t mfma16x16x32(const bf16x8_t& a, const bf16x8_t& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef short s16x4_t __attribute__((ext_vector_type(4)));  // 16x16x16 MFMA A/B operand (4 bf16)

__device__ __forceinline__ f32x4_t mfma16x16x16(const s16x4_t& a, const s16x4_t& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------ element type
// fp32 -> fp16 as float16_t's constructor (float16.hpp, float_to_f16_bits):
// round to nearest even with gradual underflow, overflow to infinity -- the
// hardware conversion -- except that a NaN becomes an infinity of its sign.
__device__ __forceinline__ uint32_t f32_to_f16_ref(float f) {
    const uint32_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
    return f != f ? ((__float_as_uint(f) >> 16) & 0x8000u) | 0x7C00u : h;
}

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t_ __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t_ __attribute__((ext_vector_type(2)));

// The 16-bit element type of q, the K/V pools and out: bf16 (F16 = false,
// every Qwen3 layer) or fp16.  The MFMAs take raw 16-byte (8 elements) or
// 8-byte (4 elements) operands: both types have the same lane layouts.
template <bool F16>
struct Elem;
template <>
struct Elem<false> {
    static __device__ __forceinline__ f32x4_t mma32(const uint4& a, const uint4& b, const f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                       c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4_t mma16(const uint2& a, const uint2& b, const f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b),
                                                        c, 0, 0, 0);
    }
    // two probabilities, round to nearest even (one v_cvt_pk_bf16_f32)
    static __device__ __forceinline__ uint32_t pack_p(float lo, float hi) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t_{lo, hi}, bf16x2_t_));
    }
    // an output element as the reference's from_f32_rt stores it
    static __device__ __forceinline__ uint32_t out(float f) { return f32_to_bf16_ref(f); }
    static __device__ __forceinline__ float lo(uint32_t w) { return bf16_lo(w); }
    static __device__ __forceinline__ float hi(uint32_t w) { return bf16_hi(w); }
    // either element of a packed pair is NaN or infinite
    static __device__ __forceinline__ bool nonfinite2(uint32_t w) {
        return (w & 0x7F80u) == 0x7F80u || (w & 0x7F800000u) == 0x7F800000u;
    }
};
template <>
struct Elem<true> {
    static __device__ __forceinline__ f32x4_t mma32(const uint4& a, const uint4& b, const f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                      0, 0, 0);
    }
    static __device__ __forceinline__ f32x4_t mma16(const uint2& a, const uint2& b, const f32x4_t& c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a), __builtin_bit_cast(f16x4_t, b), c,
                                                     0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack_p(float lo, float hi) {
        return __builtin_bit_cast(uint32_t, f16x2_t{static_cast<_Float16>(lo), static_cast<_Float16>(hi)});
    }
    static __device__ __forceinline__ uint32_t out(float f) { return f32_to_f16_ref(f); }
    static __device__ __forceinline__ float lo(uint32_t w) { return float(__builtin_bit_cast(_Float16, uint16_t(w))); }
    static __device__ __forceinline__ float hi(uint32_t w) {
        return float(__builtin_bit_cast(_Float16, uint16_t(w >> 16)));
    }
    static __device__ __forceinline__ bool nonfinite2(uint32_t w) {
        return (w & 0x7C00u) == 0x7C00u || (w & 0x7C000000u) == 0x7C000000u;
    }
};

// Every 64-byte line of the kernel's argument block requested at once, at
// entry.  Each launch has a fresh argument block, so its lines miss every
// cache; read where they are used, the arguments cost one memory round trip
// per dependent step of the prologue.  One word per line is loaded here
// (scalar loads, all in flight together) and consumed by an empty asm, so the
// later reads of the same lines hit the scalar cache.  Measured on MI355X:
// 0.1-0.4 us less per decode and append launch; the prefill kernel, which has
// many waves per tile and a long prologue anyway, ran 0.5 us slower with it
// and does not use it.
template <size_t kBytes>
__device__ __forceinline__ void prefetch_kernargs() {
    typedef const __attribute__((address_space(4))) uint32_t kernarg_word;  // constant address space: scalar loads
    kernarg_word* a = (kernarg_word*)__builtin_amdgcn_kernarg_segment_ptr();
    constexpr int kLines = int((kBytes + 63) / 64);
    uint32_t w[kLines];
#pragma unroll
    for (int i = 0; i < kLines; ++i) w[i] = a[16 * i];
#pragma unroll
    for (int i = 0; i < kLines; ++i) __asm__ volatile("" ::"s"(w[i]));
}

// Host helpers
int device_cu_count();
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace genllm
