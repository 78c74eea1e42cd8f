// kv_append.hip -- fused per-head RMSNorm -> RoPE -> page scatter of K/V (and q).
//
// Reference semantics (one kernel instead of four ops):
//   RmsNormImpl<CPU>   src/backend/cpu/normalization.cpp:44-107, 138-153
//   ApplyRopeImpl<CPU> src/backend/cpu/rope.cpp:76-119
//   append_kv_from_tensor src/core/page_attention.cpp:104-140
//
// Work split: one wave per task, a task = 8 rows (heads) of one token and one
// kind (q rows, k rows or v rows).  Row r of the task sits on lanes 8r..8r+7.
//
// K/q lanes: lane j of a row holds elements 4j + 32t + {0,1,2,3}, t = 0..D/32-1
// (one 8-byte load per t).  That puts the CPU rms_norm's 32 running sums
// (element e feeds sum e % 32, fused multiply-adds in increasing e) inside the
// lanes: lane j owns sums 4j..4j+3 and runs their chains itself, and three
// 8-lane shuffles reproduce the reference's combine order
//   T[k] = (A[k]+A[8+k]) + (A[16+k]+A[24+k]),  ss = ((T0+T4)+(T1+T5)) + ((T2+T6)+(T3+T7))
// bit for bit.  The NeoX pair (i, i+D/2) is (t, t+D/64) in the same lane, so
// RoPE needs no exchange.  Rounding follows the reference: truncation to bf16
// after the norm, then RNE (subnormal flush) after RoPE, with the rotation
// contracted as GCC contracts the CPU op: fma(x0,c,-(x1*s)), fma(x0,s,x1*c).
//
// V lanes: lane j copies elements 8j + 64u + {0..7} (16-byte loads/stores,
// 128 contiguous bytes per row per instruction); V is never rounded: bit-exact.
//
// Page address of token t (global position g = pos0 + t):
//   pool + id[g/16]*page_elems + (g%16)*Hkv*D + h*D        (page layout [16][Hkv][D])
// Ids of pages opened by this call may come in the launch arguments (decode
// opens at most one page); block 0 also writes them into the device table.
#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

#pragma clang fp contract(off)

template <int D>
struct AppendKernel {
    static constexpr int R = D / 32;   // rounds of 32 elements
    static constexpr int U = D / 64;   // 16-byte V chunks per lane

    __device__ static int32_t page_id(const AppendParams& p, int lp, int which) {
        int rel = lp - p.upd.first;
        if (rel >= 0 && rel < p.upd.count) return which ? p.upd.v[rel] : p.upd.k[rel];
        return which ? p.v_ids[lp] : p.k_ids[lp];
    }

    // Norm (optional) + RoPE (optional) of one row held as R pairs-of-pairs.
    __device__ static void norm_rope_row(uint2 (&x)[R], const float* gamma, float eps, const float* cos_row,
                                         const float* sin_row, int j, bool do_norm) {
        float v[R][4];
#pragma unroll
        for (int t = 0; t < R; ++t) {
            v[t][0] = bf16_lo(x[t].x);
            v[t][1] = bf16_hi(x[t].x);
            v[t][2] = bf16_lo(x[t].y);
            v[t][3] = bf16_hi(x[t].y);
        }
        if (do_norm) {
            float A[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float a = 0.0f;
#pragma unroll
                for (int t = 0; t < R; ++t) a = __builtin_fmaf(v[t][q], v[t][q], a);
                A[q] = a;
            }
            // A[k]+A[8+k] (lanes j, j+2) then +(A[16+k]+A[24+k]) (lanes j+4, j+6)
            float X[4], T[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) X[q] = A[q] + __shfl_down(A[q], 2, 8);
#pragma unroll
            for (int q = 0; q < 4; ++q) T[q] = X[q] + __shfl_down(X[q], 4, 8);
            // lane 0: T[0..3], lane 1: T[4..7]; u[i] = T[i] + T[i+4]
            float u[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) u[q] = T[q] + __shfl_down(T[q], 1, 8);
            float ss = (u[0] + u[1]) + (u[2] + u[3]);
            ss = __shfl(ss, 0, 8);
            float r = 1.0f / __builtin_sqrtf(ss / float(D) + eps);
#pragma unroll
            for (int t = 0; t < R; ++t) {
                float4 g = *reinterpret_cast<const float4*>(gamma + 4 * j + 32 * t);
                float gv[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float y = (v[t][q] * r) * gv[q];
                    v[t][q] = __uint_as_float(__float_as_uint(y) & 0xFFFF0000u);  // truncating store
                }
            }
        }
        uint32_t o[R][4];
        if (cos_row) {
#pragma unroll
            for (int t = 0; t < R / 2; ++t) {
                float4 c4 = *reinterpret_cast<const float4*>(cos_row + 4 * j + 32 * t);
                float4 s4 = *reinterpret_cast<const float4*>(sin_row + 4 * j + 32 * t);
                float c[4] = {c4.x, c4.y, c4.z, c4.w};
                float s[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float x0 = v[t][q], x1 = v[t + R / 2][q];
                    float y0 = __builtin_fmaf(x0, c[q], -(x1 * s[q]));
                    float y1 = __builtin_fmaf(x0, s[q], x1 * c[q]);
                    o[t][q] = f32_to_bf16_ref(y0);
                    o[t + R / 2][q] = f32_to_bf16_ref(y1);
                }
            }
        } else {
#pragma unroll
            for (int t = 0; t < R; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q) o[t][q] = __float_as_uint(v[t][q]) >> 16;
        }
#pragma unroll
        for (int t = 0; t < R; ++t) {
            x[t].x = pack2(o[t][0], o[t][1]);
            x[t].y = pack2(o[t][2], o[t][3]);
        }
    }

    __device__ static void run(const AppendParams& p) {
        const int lane = threadIdx.x & 63;
        const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
        const int r = lane >> 3, j = lane & 7;

        if (blockIdx.x == 0 && threadIdx.x < p.upd.count) {
            p.k_ids[p.upd.first + threadIdx.x] = p.upd.k[threadIdx.x];
            p.v_ids[p.upd.first + threadIdx.x] = p.upd.v[threadIdx.x];
        }
        const int T = p.nq_tasks + 2 * p.nkv_tasks;
        const int tok = wave / T;
        if (tok >= p.S) return;
        const int kind = wave - tok * T;

        if (kind < p.nq_tasks + p.nkv_tasks) {
            // q or k rows: norm + RoPE
            const bool is_q = kind < p.nq_tasks;
            const int h = (is_q ? kind : kind - p.nq_tasks) * 8 + r;
            const int H = is_q ? p.Hq : p.Hkv;
            if (h >= H) return;
            const uint16_t* src = is_q ? p.q + tok * p.q_tok_stride + h * p.q_head_stride
                                       : p.k + tok * p.k_tok_stride + h * p.k_head_stride;
            uint2 x[R];
#pragma unroll
            for (int t = 0; t < R; ++t) x[t] = *reinterpret_cast<const uint2*>(src + 4 * j + 32 * t);
            const float* gamma = is_q ? p.gamma_q : p.gamma_k;
            const float* crow = p.cos_tab ? p.cos_tab + (p.rope_pos0 + tok) * p.rope_stride : nullptr;
            const float* srow = p.sin_tab ? p.sin_tab + (p.rope_pos0 + tok) * p.rope_stride : nullptr;
            norm_rope_row(x, gamma, p.eps, crow, srow, j, gamma != nullptr);
            uint16_t* dst;
            if (is_q) {
                dst = p.q_out + tok * p.qo_tok_stride + h * p.qo_head_stride;
            } else {
                const int g = p.pos0 + tok;
                const int32_t id = page_id(p, g / kPage, 0);
                dst = p.k_pool + int64_t(id) * p.page_elems + int64_t(g % kPage) * p.Hkv * D + h * D;
            }
#pragma unroll
            for (int t = 0; t < R; ++t) *reinterpret_cast<uint2*>(dst + 4 * j + 32 * t) = x[t];
        } else {
            // v rows: plain copy
            const int h = (kind - p.nq_tasks - p.nkv_tasks) * 8 + r;
            if (h >= p.Hkv) return;
            const uint16_t* src = p.v + tok * p.v_tok_stride + h * p.v_head_stride;
            const int g = p.pos0 + tok;
            const int32_t id = page_id(p, g / kPage, 1);
            uint16_t* dst = p.v_pool + int64_t(id) * p.page_elems + int64_t(g % kPage) * p.Hkv * D + h * D;
            uint4 x[U];
#pragma unroll
            for (int u = 0; u < U; ++u) x[u] = *reinterpret_cast<const uint4*>(src + 8 * j + 64 * u);
#pragma unroll
            for (int u = 0; u < U; ++u) *reinterpret_cast<uint4*>(dst + 8 * j + 64 * u) = x[u];
        }
    }
};

template <int D>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p) {
    AppendKernel<D>::run(p);
}

int launch_kv_append(const AppendParams& p, int head_dim, hipStream_t stream) {
    const int T = p.nq_tasks + 2 * p.nkv_tasks;
    const int64_t waves = int64_t(p.S) * T;
    const int blocks = int((waves + 3) / 4);
    if (blocks <= 0) {
        // nothing to scatter, but a table update may still be pending
        if (p.upd.count == 0) return GENLLM_OK;
    }
    const int nblk = blocks > 0 ? blocks : 1;
    switch (head_dim) {
        case 64: hipLaunchKernelGGL(kv_append_kernel<64>, dim3(nblk), dim3(256), 0, stream, p); break;
        case 128: hipLaunchKernelGGL(kv_append_kernel<128>, dim3(nblk), dim3(256), 0, stream, p); break;
        case 256: hipLaunchKernelGGL(kv_append_kernel<256>, dim3(nblk), dim3(256), 0, stream, p); break;
        default: return fail(GENLLM_ERR_UNSUPPORTED, "kv append: head_dim must be 64, 128 or 256");
    }
    GENLLM_LAUNCH_CHECK("kv_append_kernel");
    return GENLLM_OK;
}

}  // namespace genllm
