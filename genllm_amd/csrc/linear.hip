// linear.hip -- bf16 linear layer: LinearImpl (src/backend/cpu/linear.cpp:46-122,
// :325-345; src/backend/cuda/linear.cu:72-126) for the Q/K/V projections that
// feed the paged attention op (Qwen3.cpp:130-134):
//   out[r][c] = bf16( sum_k x[r][k] * w[c][k] + bias[c] )
// x [rows][common], w [cols][common] (transpose_w = 1), bias [cols] or null,
// fp32 accumulation, one rounding (the bfloat16_t constructor's rules).
//
// rows <= kGemvRows (a decode step): linear_gemv_lds_kernel when every K-block
// is whole, else linear_gemv_kernel; both HBM-bound on the weights, both
// reproduce the CPU reference's summation order exactly, so the result is
// bit-identical to it.  The reference sums each output over K-blocks
// of 256 elements: inside a block two 8-lane accumulators (sum0 takes elements
// 16i+l, sum1 elements 16i+8+l, one fused multiply-add each, i ascending), then
// v = sum0 + sum1 lane-wise and the block adds (t0+t1)+(t2+t3), t[i] =
// v[i]+v[i+4], to the running fp32 sum; a trailing 8-element group adds the
// same tree of its rounded products.  Here one GPU lane carries the 8 lanes
// of one accumulator of one block (16-byte weight loads, 8 fused
// multiply-adds each), its partner lane the other accumulator; the pair forms
// the block's tree value, and one lane per output adds the blocks in order.
// (A product of two bf16 values is exact in fp32, so the fused and unfused
// forms of the 8-element group agree.)
//
// More rows: rocBLAS gemm_ex, bf16 inputs and fp32 compute.  With a bias, the
// fp32 result goes to the caller's workspace and linear_epilogue_kernel adds
// the bias in fp32 and rounds once; without one (Qwen3's projections), rocBLAS
// writes bf16 directly, rounding the fp32 result once to nearest even (an
// fp32 subnormal result stays a bf16 subnormal where the reference flushes it
// to zero).  The summation order is rocBLAS's, so results match the reference
// within fp32 accumulation error, not bit for bit.
#include <rocblas/rocblas.h>

#include <map>
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

namespace {

constexpr int kGemvRows = 4;     // rows handled by the order-exact kernel
constexpr int kBlockK = 256;     // the reference's K blocking (KR)
constexpr int kGemvThreads = 256;
// dynamic LDS of linear_gemv_lds_kernel: the weight rows of a workgroup (at
// most 64 KB) and the x rows; two workgroups still fit a CU (160 KB)
constexpr size_t kGemvLdsMax = 80 * 1024;

__device__ __forceinline__ void bf16x8_to_f32(const uint4& u, float f[8]) {
    f[0] = bf16_lo(u.x); f[1] = bf16_hi(u.x);
    f[2] = bf16_lo(u.y); f[3] = bf16_hi(u.y);
    f[4] = bf16_lo(u.z); f[5] = bf16_hi(u.z);
    f[6] = bf16_lo(u.w); f[7] = bf16_hi(u.w);
}

__device__ __forceinline__ float tree8(const float v[8]) {
    const float t0 = v[0] + v[4], t1 = v[1] + v[5], t2 = v[2] + v[6], t3 = v[3] + v[7];
    return (t0 + t1) + (t2 + t3);
}

// Work item = (output column c, K-block b, accumulator h); adjacent lanes hold
// the two accumulators of one block.  Items of a workgroup cover whole columns
// (cols_per_wg = 256 / (2 nb)), so the block values of a column meet in LDS.
template <int R>
__global__ __launch_bounds__(kGemvThreads) void linear_gemv_kernel(const uint16_t* __restrict__ x,
                                                                   const uint16_t* __restrict__ w,
                                                                   const uint16_t* __restrict__ bias,
                                                                   uint16_t* __restrict__ out, int common, int cols,
                                                                   int nb, int cols_per_wg) {
    __shared__ float s_h1[R][kGemvThreads / 2], s_h2[R][kGemvThreads / 2];
    const int t = threadIdx.x;
    const int pair = t >> 1, h = t & 1;
    const int col0 = int(blockIdx.x) * cols_per_wg;
    const int lc = pair / nb, b = pair - lc * nb;  // column within the workgroup, block
    const int c = col0 + lc;
    const bool item = lc < cols_per_wg && c < cols;
    const int k0 = b * kBlockK;
    const int k_len = min(kBlockK, common - k0);
    const int n16 = k_len >> 4;               // 16-element steps of the block
    const bool rem8 = (k_len - 16 * n16) >= 8;  // a trailing 8-element group (common % 8 == 0)

    float s[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int l = 0; l < 8; ++l) s[r][l] = 0.0f;
    if (item && n16 > 0) {
        const uint16_t* wp = w + int64_t(c) * common + k0 + 8 * h;
        const uint16_t* xp = x + k0 + 8 * h;
        // NB steps of weights and x in flight (all 16 of a block for one or two
        // rows), then their multiply-adds in order.  A block has at most 16
        // steps; loads past its n16 repeat the last step (in bounds) and are
        // not used.
        constexpr int NB = R <= 2 ? 16 : 8;
#pragma unroll
        for (int i0 = 0; i0 < 16; i0 += NB) {
            if (i0 >= n16) break;  // uniform over the kernel but for the last block
            uint4 wq[NB], xq[R][NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int i = min(i0 + u, n16 - 1);
                wq[u] = *reinterpret_cast<const uint4*>(wp + 16 * i);
#pragma unroll
                for (int r = 0; r < R; ++r) xq[r][u] = *reinterpret_cast<const uint4*>(xp + int64_t(r) * common + 16 * i);
            }
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const bool on = i0 + u < n16;
                float wf[8];
                bf16x8_to_f32(wq[u], wf);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float xf[8];
                    bf16x8_to_f32(xq[r][u], xf);
#pragma unroll
                    for (int l = 0; l < 8; ++l) {
                        const float f = __builtin_fmaf(xf[l], wf[l], s[r][l]);
                        s[r][l] = on ? f : s[r][l];
                    }
                }
            }
        }
    }
    // v = sum0 + sum1 (partner lane t ^ 1), the block's tree value
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float v[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const float o = __shfl_xor(s[r][l], 1);
            v[l] = h == 0 ? s[r][l] + o : o + s[r][l];
        }
        float h2 = 0.0f;
        if (item && h == 0 && rem8) {  // the trailing 8-element group, products rounded
            const int k8 = k0 + 16 * n16;
            float wf[8], xf[8];
            bf16x8_to_f32(*reinterpret_cast<const uint4*>(w + int64_t(c) * common + k8), wf);
            bf16x8_to_f32(*reinterpret_cast<const uint4*>(x + int64_t(r) * common + k8), xf);
            float pr[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) pr[l] = xf[l] * wf[l];
            h2 = tree8(pr);
        }
        if (h == 0) {
            s_h1[r][pair] = tree8(v);
            s_h2[r][pair] = h2;
        }
    }
    __syncthreads();
    // one lane per column adds the blocks in order, then the bias, then rounds
    if (t < cols_per_wg && col0 + t < cols) {
        const int cc = col0 + t;
        const float bv = bias ? bf16_to_f32(bias[cc]) : 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float acc = 0.0f;
            for (int bb = 0; bb < nb; ++bb) {
                const int kl = min(kBlockK, common - bb * kBlockK);
                if (kl >= 16) acc += s_h1[r][t * nb + bb];
                if (kl - 16 * (kl >> 4) >= 8) acc += s_h2[r][t * nb + bb];
            }
            float val = acc;
            if (bias) val += bv;
            out[int64_t(r) * cols + cc] = uint16_t(f32_to_bf16_ref(val));
        }
    }
}

// The same sums when every K-block is whole (common % 256 == 0), with the
// weight rows staged through LDS.  In linear_gemv_kernel a wave's 16-byte
// weight loads touch 32 cache lines each (a lane reads 32 B of every 512-byte
// block), and every lane also loads its 256 B of x: twice the weight bytes go
// through the L1.  Here the workgroup's weight rows -- cpw whole columns, one
// contiguous range -- come in with LDS-mode buffer loads of 1 KB per wave
// instruction, x once per workgroup the same way, and each lane then reads its
// block from LDS.  Lane pair P works on block P of the workgroup (column
// P / nb, block P % nb, as in linear_gemv_kernel).
//
// The weights arrive in four parts: part k holds bytes 128k..128k+127 of every
// block (its 16-byte chunks 8k..8k+7, the lane pair's iterations 4k..4k+3), and
// the parts are requested in order after x.  Each wave waits only for the
// parts it is about to use, and the workgroup multiplies part k while the later
// parts are still arriving; only the last part's multiply-adds follow the last
// load (Qwen3-4B projection: 8.2-8.3 against 9.0 us with one wait for
// everything, 8.5 with two halves, 9.3 with eight parts; A/B on one box,
// results bit-identical).
//
// LDS: part k is a region of 128-byte slots, slot P holding part k of block P
// with chunk q at position (q + 2 (P / 2)) % 8; x rows follow, block b rotated
// by 2b chunks of 16 B (chunk q at (q + 2b) % 32).  A read phase of 16 lanes
// (8 lane pairs: even and odd slots fill the two 128-byte halves of the 64
// banks) then hits 16 different bank groups.  The multiply-add order and the
// block sums are those of linear_gemv_kernel.  Loads past the weights or x (the
// last workgroup, a block count that does not fill a load) are bounded by the
// buffer resources and read zeros into LDS slots no lane reads.  (Measured
// against block-major slots, whose read phases share x's block, and x staged
// as fp32: both slower.)
// cache policy of the weight loads: nt (every weight byte is read once per
// call; 7.9-8.0 against 8.3-8.5 us at the Qwen3-4B projection, A/B on one box)
constexpr int kNtPolicy = 2;
constexpr int kGemvParts = 4;
constexpr int kGemvPartChunks = 32 / kGemvParts;          // 16-byte chunks of a block per part
constexpr int kGemvPartBlocks = 64 / kGemvPartChunks;     // part slots per 1 KB load
constexpr int kGemvRotShift = kGemvParts == 2 ? 0 : kGemvParts == 4 ? 1 : 2;  // slot pairs, quads per rotation step
__host__ __device__ constexpr size_t gemv_lds_bytes(int rows, int n_pairs, int nb) {
    return size_t(kGemvParts) * ((n_pairs + kGemvPartBlocks - 1) / kGemvPartBlocks) * 1024 +
           size_t(rows) * ((nb + 1) / 2) * 1024;
}

// s_waitcnt vmcnt(n) for the n a wave computes at run time (the count is an
// instruction immediate); counts past 15 wait for everything
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
        case 0: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 0); break;
        case 1: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 1); break;
        case 2: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 2); break;
        case 3: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 3); break;
        case 4: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 4); break;
        case 5: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 5); break;
        case 6: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 6); break;
        case 7: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 7); break;
        case 8: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 8); break;
        case 9: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 9); break;
        case 10: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 10); break;
        case 11: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 11); break;
        case 12: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 12); break;
        case 13: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 13); break;
        case 14: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 14); break;
        case 15: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | 15); break;
        default: __builtin_amdgcn_s_waitcnt(kWaitVmcnt0); break;
    }
}

template <int R>
__global__ __launch_bounds__(kGemvThreads) void linear_gemv_lds_kernel(const uint16_t* __restrict__ x,
                                                                       const uint16_t* __restrict__ w,
                                                                       const uint16_t* __restrict__ bias,
                                                                       uint16_t* __restrict__ out, int common,
                                                                       int cols, int nb, int cpw) {
    extern __shared__ __attribute__((aligned(16))) char lds_w[];
    __shared__ float s_h1[R][kGemvThreads / 2];
    const int t = threadIdx.x, lane = t & 63;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    constexpr int kWaves = kGemvThreads / 64;
    const int col0 = int(blockIdx.x) * cpw;
    const int n_pairs = cpw * nb;                                          // 512-byte blocks of this workgroup
    const int part_inst = (n_pairs + kGemvPartBlocks - 1) / kGemvPartBlocks;  // 1 KB loads per part
    const int part_bytes = part_inst * 1024;
    const int x_inst = (nb + 1) / 2;                                       // 1 KB loads per row of x
    const int x_base = kGemvParts * part_bytes;                            // x rows after the weights
    int n_part = 0;                                                        // this wave's loads per part
    {
        const int64_t left = int64_t(cols - col0) * common * 2;
        const uint32_t span = uint32_t(min<int64_t>(left, int64_t(n_pairs) * 512));
        const auto rw = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(w + int64_t(col0) * common), 0, span, kBufferFlags);
        const auto rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), 0, uint32_t(R * common * 2),
                                                          kBufferFlags);
        const int half = lane >> 5, pos = lane & 31;  // block of the 1 KB, LDS chunk position in it
        for (int e = wv; e < R * x_inst; e += kWaves) {
            const int r = e / x_inst, bb = 2 * (e - r * x_inst) + half;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rx, (__attribute__((address_space(3))) void*)(lds_w + x_base + e * 1024), 16,
                uint32_t(r * common * 2 + bb * 512 + ((pos - 2 * bb) & 31) * 16), 0, 0, 0);
        }
        constexpr int CH = kGemvPartChunks;
        const int slot = lane / CH, pc = lane % CH;  // part slot of the 1 KB, LDS chunk position in it
#pragma unroll
        for (int k = 0; k < kGemvParts; ++k)
            for (int e = wv; e < part_inst; e += kWaves) {
                const int P = kGemvPartBlocks * e + slot;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rw, (__attribute__((address_space(3))) void*)(lds_w + k * part_bytes + e * 1024), 16,
                    uint32_t(P * 512 + (CH * k + ((pc - 2 * (P >> kGemvRotShift)) & (CH - 1))) * 16), 0, 0,
                    kNtPolicy);
                if (k == 0) ++n_part;
            }
    }
    const int pair = t >> 1, h = t & 1;
    const int lc = pair / nb, b = pair - lc * nb;  // column within the workgroup, block
    const bool item = pair < n_pairs && col0 + lc < cols;

    float s[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int l = 0; l < 8; ++l) s[r][l] = 0.0f;
    const char* xl = lds_w + x_base + b * 512;
    // part k's multiply-adds: chunks CH k .. CH k + CH - 1 of the lane's block
    auto run_part = [&](int k) {
        constexpr int CH = kGemvPartChunks;
        const char* wl = lds_w + k * part_bytes + pair * (CH * 16);
#pragma unroll
        for (int i = 0; i < CH / 2; ++i) {
            const int q = 2 * i + h;  // chunk within the part
            float wf[8];
            bf16x8_to_f32(*reinterpret_cast<const uint4*>(wl + ((q + 2 * (pair >> kGemvRotShift)) & (CH - 1)) * 16),
                          wf);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float xf[8];
                bf16x8_to_f32(*reinterpret_cast<const uint4*>(xl + r * x_inst * 1024 + ((CH * k + q + 2 * b) & 31) * 16),
                              xf);
#pragma unroll
                for (int l = 0; l < 8; ++l) s[r][l] = __builtin_fmaf(xf[l], wf[l], s[r][l]);
            }
        }
    };
    // wait until part k has landed: this wave's loads of the later parts may
    // still be in flight, and the other waves' loads of parts up to k have
    // landed once they reach the barrier.  A bare barrier: a fence would wait
    // for every load.
    auto part_ready = [&](int k) {
        wait_vmcnt(n_part * (kGemvParts - 1 - k));
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
    };
    // (written out: the same sequence as a loop over k measured 8.65 against
    // 8.3 us -- the compiler then kept one LDS read in flight at a time)
    static_assert(kGemvParts == 4, "the part sequence below is written for four parts");
    part_ready(0);
    if (item) run_part(0);
    part_ready(1);
    if (item) run_part(1);
    part_ready(2);
    if (item) run_part(2);
    part_ready(3);
    if (item) run_part(3);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float v[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const float o = __shfl_xor(s[r][l], 1);
            v[l] = h == 0 ? s[r][l] + o : o + s[r][l];
        }
        if (h == 0) s_h1[r][pair] = tree8(v);
    }
    __syncthreads();
    if (t < cpw && col0 + t < cols) {
        const int cc = col0 + t;
        const float bv = bias ? bf16_to_f32(bias[cc]) : 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float acc = 0.0f;
            for (int bb = 0; bb < nb; ++bb) acc += s_h1[r][t * nb + bb];
            float val = acc;
            if (bias) val += bv;
            out[int64_t(r) * cols + cc] = uint16_t(f32_to_bf16_ref(val));
        }
    }
}

// out = bf16(acc + bias) over the fp32 GEMM result [rows][cols]
__global__ __launch_bounds__(256) void linear_epilogue_kernel(const float* __restrict__ acc,
                                                              const uint16_t* __restrict__ bias,
                                                              uint16_t* __restrict__ out, int64_t n, int cols) {
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256) {
        float v = acc[i];
        if (bias) v += bf16_to_f32(bias[i % cols]);
        out[i] = uint16_t(f32_to_bf16_ref(v));
    }
}

// one rocBLAS handle per device, created on first use
std::mutex g_blas_mu;
std::map<int, rocblas_handle> g_blas;

int blas_handle(rocblas_handle* out) {
    int dev = 0;
    GENLLM_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_blas_mu);
    auto it = g_blas.find(dev);
    if (it == g_blas.end()) {
        rocblas_handle h = nullptr;
        if (rocblas_create_handle(&h) != rocblas_status_success)
            return fail(GENLLM_ERR_HIP, "linear: rocblas_create_handle failed");
        rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed);  // deterministic sums
        it = g_blas.emplace(dev, h).first;
    }
    *out = it->second;
    return GENLLM_OK;
}

bool gemv_shape(int64_t rows, int64_t common) {
    const int64_t nb = (common + kBlockK - 1) / kBlockK;
    return rows >= 1 && rows <= kGemvRows && common % 8 == 0 && 2 * nb <= kGemvThreads;
}

}  // namespace

size_t linear_workspace_bytes(int64_t rows, int64_t common, int64_t cols) {
    if (rows <= 0 || common <= 0 || cols <= 0 || gemv_shape(rows, common)) return 0;
    return size_t(rows) * size_t(cols) * sizeof(float);
}

int launch_linear(const uint16_t* x, const uint16_t* w, const uint16_t* bias, uint16_t* out, int64_t rows,
                  int64_t common, int64_t cols, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!x || !w || !out) return fail(GENLLM_ERR_INVALID, "linear: null pointer");
    if (rows < 0 || common <= 0 || cols < 0) return fail(GENLLM_ERR_INVALID, "linear: negative or zero size");
    if (rows == 0 || cols == 0) return GENLLM_OK;
    if (rows > INT32_MAX || common > INT32_MAX || cols > INT32_MAX)
        return fail(GENLLM_ERR_INVALID, "linear: sizes must fit in 32 bits");
    if (gemv_shape(rows, common)) {
        const int nb = int((common + kBlockK - 1) / kBlockK);
        const int cpw = kGemvThreads / (2 * nb);
        const unsigned grid = unsigned((cols + cpw - 1) / cpw);
        const int c = int(common), n = int(cols);
        const size_t lds = gemv_lds_bytes(int(rows), cpw * nb, nb);
        if (common % kBlockK == 0 && lds <= kGemvLdsMax) {
            switch (rows) {
                case 1: hipLaunchKernelGGL(linear_gemv_lds_kernel<1>, dim3(grid), dim3(kGemvThreads), lds, stream, x, w, bias, out, c, n, nb, cpw); break;
                case 2: hipLaunchKernelGGL(linear_gemv_lds_kernel<2>, dim3(grid), dim3(kGemvThreads), lds, stream, x, w, bias, out, c, n, nb, cpw); break;
                case 3: hipLaunchKernelGGL(linear_gemv_lds_kernel<3>, dim3(grid), dim3(kGemvThreads), lds, stream, x, w, bias, out, c, n, nb, cpw); break;
                default: hipLaunchKernelGGL(linear_gemv_lds_kernel<4>, dim3(grid), dim3(kGemvThreads), lds, stream, x, w, bias, out, c, n, nb, cpw); break;
            }
            GENLLM_LAUNCH_CHECK("linear_gemv_lds_kernel");
            return GENLLM_OK;
        }
        switch (rows) {
            case 1: hipLaunchKernelGGL(linear_gemv_kernel<1>, dim3(grid), dim3(kGemvThreads), 0, stream, x, w, bias, out, c, n, nb, cpw); break;
            case 2: hipLaunchKernelGGL(linear_gemv_kernel<2>, dim3(grid), dim3(kGemvThreads), 0, stream, x, w, bias, out, c, n, nb, cpw); break;
            case 3: hipLaunchKernelGGL(linear_gemv_kernel<3>, dim3(grid), dim3(kGemvThreads), 0, stream, x, w, bias, out, c, n, nb, cpw); break;
            default: hipLaunchKernelGGL(linear_gemv_kernel<4>, dim3(grid), dim3(kGemvThreads), 0, stream, x, w, bias, out, c, n, nb, cpw); break;
        }
        GENLLM_LAUNCH_CHECK("linear_gemv_kernel");
        return GENLLM_OK;
    }
    const size_t need = linear_workspace_bytes(rows, common, cols);
    if (bias && (!workspace || workspace_bytes < need))
        return fail(GENLLM_ERR_INVALID, "linear: workspace too small (need " + std::to_string(need) + " bytes, have " +
                                            std::to_string(workspace_bytes) + ")");
    rocblas_handle hb = nullptr;
    if (int rc = blas_handle(&hb)) return rc;
    if (rocblas_set_stream(hb, stream) != rocblas_status_success)
        return fail(GENLLM_ERR_HIP, "linear: rocblas_set_stream failed");
    const float alpha = 1.0f, beta = 0.0f;
    if (!bias) {
        // column-major view: out^T [cols][rows] = (w as [common][cols])^T * (x as [common][rows])
        const rocblas_status st = rocblas_gemm_ex(
            hb, rocblas_operation_transpose, rocblas_operation_none, rocblas_int(cols), rocblas_int(rows),
            rocblas_int(common), &alpha, w, rocblas_datatype_bf16_r, rocblas_int(common), x, rocblas_datatype_bf16_r,
            rocblas_int(common), &beta, out, rocblas_datatype_bf16_r, rocblas_int(cols), out, rocblas_datatype_bf16_r,
            rocblas_int(cols), rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
        if (st != rocblas_status_success)
            return fail(GENLLM_ERR_HIP, std::string("linear: rocblas_gemm_ex failed: ") + rocblas_status_to_string(st));
        return GENLLM_OK;
    }
    float* acc = static_cast<float*>(workspace);
    // column-major view: acc^T [cols][rows] = (w as [common][cols])^T * (x as [common][rows])
    const rocblas_status st = rocblas_gemm_ex(
        hb, rocblas_operation_transpose, rocblas_operation_none, rocblas_int(cols), rocblas_int(rows),
        rocblas_int(common), &alpha, w, rocblas_datatype_bf16_r, rocblas_int(common), x, rocblas_datatype_bf16_r,
        rocblas_int(common), &beta, acc, rocblas_datatype_f32_r, rocblas_int(cols), acc, rocblas_datatype_f32_r,
        rocblas_int(cols), rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    if (st != rocblas_status_success)
        return fail(GENLLM_ERR_HIP, std::string("linear: rocblas_gemm_ex failed: ") + rocblas_status_to_string(st));
    const int64_t n = rows * cols;
    const unsigned grid = unsigned(std::min<int64_t>((n + 255) / 256, 4096));
    hipLaunchKernelGGL(linear_epilogue_kernel, dim3(grid), dim3(256), 0, stream, acc, bias, out, n, int(cols));
    GENLLM_LAUNCH_CHECK("linear_epilogue_kernel");
    return GENLLM_OK;
}

}  // namespace genllm

// ------------------------------------------------------------------- C ABI

extern "C" size_t genllm_linear_workspace_bytes(int64_t rows, int64_t common, int64_t cols) {
    return genllm::linear_workspace_bytes(rows, common, cols);
}

extern "C" int genllm_linear(const void* x, const void* w, const void* bias, void* out, int64_t rows, int64_t common,
                             int64_t cols, void* workspace, size_t workspace_bytes, void* stream) {
    return genllm::launch_linear(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                                 static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), rows, common, cols,
                                 workspace, workspace_bytes, genllm::as_stream(stream));
}
