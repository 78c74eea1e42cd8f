// kv_append.hip -- fused per-head RMSNorm -> RoPE -> page scatter of K/V (and q).
//
// Reference semantics (one kernel instead of four ops):
//   RmsNormImpl<CPU>   src/backend/cpu/normalization.cpp:44-107, 138-153
//   ApplyRopeImpl<CPU> src/backend/cpu/rope.cpp:76-119
//   append_kv_from_tensor src/core/page_attention.cpp:104-140
//
// Work split: a task = 8 rows (heads) of one token and one kind (q, k or v
// rows); row r of a task sits on lanes 8r..8r+7.  Tasks are numbered kind by
// kind, and each wave takes TPW consecutive tasks of one kind, issuing the
// loads of all of them before any arithmetic so that a wave keeps TPW * 2 KiB
// of reads in flight.
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

namespace {

constexpr int TPW = 4;  // tasks per wave

template <int D>
struct Append {
    static constexpr int R = D / 32;  // 8-byte chunks per q/k row and lane
    static constexpr int U = D / 64;  // 16-byte chunks per v row and lane

    __device__ static int32_t page_id(const AppendParams& p, int lp, int which) {
        const int rel = lp - p.upd.first;
        if (rel >= 0 && rel < p.upd.count) return which ? p.upd.v[rel] : p.upd.k[rel];
        return which ? p.v_ids[lp] : p.k_ids[lp];
    }

    __device__ static uint16_t* k_dst(const AppendParams& p, int tok, int h) {
        const int gpos = p.pos0 + tok;
        const int64_t id = page_id(p, gpos / kPage, 0);
        return p.k_pool + id * p.page_elems + int64_t(gpos % kPage) * p.Hkv * D + h * D;
    }

    // RMSNorm (optional) + RoPE (optional) of one row, in place.
    __device__ static void norm_rope(uint2 (&x)[R], const float* gamma, float eps, const float* cos_row,
                                     const float* sin_row, int j) {
        float v[R][4];
#pragma unroll
        for (int t = 0; t < R; ++t) {
            v[t][0] = bf16_lo(x[t].x);
            v[t][1] = bf16_hi(x[t].x);
            v[t][2] = bf16_lo(x[t].y);
            v[t][3] = bf16_hi(x[t].y);
        }
        if (gamma) {
            float A[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float a = 0.0f;
#pragma unroll
                for (int t = 0; t < R; ++t) a = __builtin_fmaf(v[t][q], v[t][q], a);
                A[q] = a;
            }
            float X[4], T[4], u[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) X[q] = A[q] + __shfl_down(A[q], 2, 8);  // A[k] + A[8+k]
#pragma unroll
            for (int q = 0; q < 4; ++q) T[q] = X[q] + __shfl_down(X[q], 4, 8);  // + (A[16+k] + A[24+k])
#pragma unroll
            for (int q = 0; q < 4; ++q) u[q] = T[q] + __shfl_down(T[q], 1, 8);  // T[i] + T[i+4]
            float ss = (u[0] + u[1]) + (u[2] + u[3]);
            ss = __shfl(ss, 0, 8);
            const float r = 1.0f / __builtin_sqrtf(ss / float(D) + eps);
#pragma unroll
            for (int t = 0; t < R; ++t) {
                const float4 gw = *reinterpret_cast<const float4*>(gamma + 4 * j + 32 * t);
                const float gv[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float y = (v[t][q] * r) * gv[q];
                    v[t][q] = __uint_as_float(__float_as_uint(y) & 0xFFFF0000u);  // truncating store
                }
            }
        }
        uint32_t o[R][4];
        if (cos_row) {
#pragma unroll
            for (int t = 0; t < R / 2; ++t) {
                const float4 c4 = *reinterpret_cast<const float4*>(cos_row + 4 * j + 32 * t);
                const float4 s4 = *reinterpret_cast<const float4*>(sin_row + 4 * j + 32 * t);
                const float c[4] = {c4.x, c4.y, c4.z, c4.w};
                const float s[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float x0 = v[t][q], x1 = v[t + R / 2][q];
                    o[t][q] = f32_to_bf16_ref(__builtin_fmaf(x0, c[q], -(x1 * s[q])));
                    o[t + R / 2][q] = f32_to_bf16_ref(__builtin_fmaf(x0, s[q], x1 * c[q]));
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
        const int r = lane >> 3, j = lane & 7;
        if (blockIdx.x == 0 && threadIdx.x < p.upd.count) {
            p.k_ids[p.upd.first + threadIdx.x] = p.upd.k[threadIdx.x];
            p.v_ids[p.upd.first + threadIdx.x] = p.upd.v[threadIdx.x];
        }
        // wave -> (kind, first task of the kind)
        const int ngq = p.nq_tasks, ngk = p.nkv_tasks;
        const int64_t nq = int64_t(p.S) * ngq, nk = int64_t(p.S) * ngk;
        const int64_t wq = (nq + TPW - 1) / TPW, wk = (nk + TPW - 1) / TPW;
        int64_t w = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
        int kind;
        int64_t t0, n_kind;
        int ng;
        if (w < wq) {
            kind = 0, t0 = w * TPW, n_kind = nq, ng = ngq;
        } else if (w < wq + wk) {
            kind = 1, t0 = (w - wq) * TPW, n_kind = nk, ng = ngk;
        } else {
            kind = 2, t0 = (w - wq - wk) * TPW, n_kind = nk, ng = ngk;
            if (t0 >= n_kind) return;
        }

        if (kind < 2) {
            const bool is_q = kind == 0;
            const int H = is_q ? p.Hq : p.Hkv;
            uint2 x[TPW][R];
            int tok[TPW], h[TPW];
            bool ok[TPW];
#pragma unroll
            for (int u = 0; u < TPW; ++u) {
                const int64_t t = t0 + u;
                tok[u] = int(t / ng);
                h[u] = int(t - int64_t(tok[u]) * ng) * 8 + r;
                ok[u] = t < n_kind && h[u] < H;
                const uint16_t* src = is_q ? p.q + tok[u] * p.q_tok_stride + h[u] * p.q_head_stride
                                           : p.k + tok[u] * p.k_tok_stride + h[u] * p.k_head_stride;
#pragma unroll
                for (int c = 0; c < R; ++c)
                    x[u][c] = ok[u] ? *reinterpret_cast<const uint2*>(src + 4 * j + 32 * c) : make_uint2(0, 0);
            }
            const float* gamma = is_q ? p.gamma_q : p.gamma_k;
#pragma unroll
            for (int u = 0; u < TPW; ++u) {
                if (t0 + u >= n_kind) break;  // wave-uniform
                const float* crow = p.cos_tab ? p.cos_tab + (p.rope_pos0 + tok[u]) * p.rope_stride : nullptr;
                const float* srow = p.sin_tab ? p.sin_tab + (p.rope_pos0 + tok[u]) * p.rope_stride : nullptr;
                norm_rope(x[u], gamma, p.eps, crow, srow, j);
                if (!ok[u]) continue;
                uint16_t* dst = is_q ? p.q_out + tok[u] * p.qo_tok_stride + h[u] * p.qo_head_stride
                                     : k_dst(p, tok[u], h[u]);
#pragma unroll
                for (int c = 0; c < R; ++c) *reinterpret_cast<uint2*>(dst + 4 * j + 32 * c) = x[u][c];
            }
        } else {
            uint4 x[TPW][U];
            uint16_t* dst[TPW];
#pragma unroll
            for (int u = 0; u < TPW; ++u) {
                const int64_t t = t0 + u;
                const int tk = int(t / ng);
                const int hh = int(t - int64_t(tk) * ng) * 8 + r;
                const bool ok = t < n_kind && hh < p.Hkv;
                dst[u] = nullptr;
                if (ok) {
                    const uint16_t* src = p.v + tk * p.v_tok_stride + hh * p.v_head_stride;
#pragma unroll
                    for (int c = 0; c < U; ++c) x[u][c] = *reinterpret_cast<const uint4*>(src + 8 * j + 64 * c);
                    const int gpos = p.pos0 + tk;
                    const int64_t id = page_id(p, gpos / kPage, 1);
                    dst[u] = p.v_pool + id * p.page_elems + int64_t(gpos % kPage) * p.Hkv * D + hh * D;
                }
            }
#pragma unroll
            for (int u = 0; u < TPW; ++u)
                if (dst[u])
#pragma unroll
                    for (int c = 0; c < U; ++c) *reinterpret_cast<uint4*>(dst[u] + 8 * j + 64 * c) = x[u][c];
        }
    }
};

template <int D>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendParams p) {
    Append<D>::run(p);
}

}  // namespace

int launch_kv_append(const AppendParams& p, int head_dim, hipStream_t stream) {
    const int64_t nq = int64_t(p.S) * p.nq_tasks, nk = int64_t(p.S) * p.nkv_tasks;
    const int64_t waves = (nq + TPW - 1) / TPW + 2 * ((nk + TPW - 1) / TPW);
    int64_t blocks = (waves + 3) / 4;
    if (blocks <= 0) {
        if (p.upd.count == 0) return GENLLM_OK;
        blocks = 1;  // table update only
    }
    switch (head_dim) {
        case 64: hipLaunchKernelGGL(kv_append_kernel<64>, dim3(unsigned(blocks)), dim3(256), 0, stream, p); break;
        case 128: hipLaunchKernelGGL(kv_append_kernel<128>, dim3(unsigned(blocks)), dim3(256), 0, stream, p); break;
        case 256: hipLaunchKernelGGL(kv_append_kernel<256>, dim3(unsigned(blocks)), dim3(256), 0, stream, p); break;
        default: return fail(GENLLM_ERR_UNSUPPORTED, "kv append: head_dim must be 64, 128 or 256");
    }
    GENLLM_LAUNCH_CHECK("kv_append_kernel");
    return GENLLM_OK;
}

}  // namespace genllm
