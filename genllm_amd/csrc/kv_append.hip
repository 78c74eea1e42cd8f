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
// loads of all of them before any arithmetic.  One task (2 KiB of reads) per
// wave and many waves keep more bytes in flight across the GPU than fewer
// waves with more tasks each: the loads of a wave's later tasks wait behind
// its first ones.
//
// K/q lanes: lane j of a row holds elements 4j + 32t + {0,1,2,3}, t = 0..D/32-1
// (one 8-byte load per t; K rows are stored 16 bytes at a time after a swap
// with lane j ^ 1).  That puts the CPU rms_norm's 32 running sums
// (element e feeds sum e % 32, fused multiply-adds in increasing e) inside the
// lanes: lane j owns sums 4j..4j+3 and runs their chains itself, and three
// 8-lane shuffles reproduce the reference's combine order
//   T[k] = (A[k]+A[8+k]) + (A[16+k]+A[24+k]),  ss = ((T0+T4)+(T1+T5)) + ((T2+T6)+(T3+T7))
// bit for bit.  The NeoX pair (i, i+D/2) is (t, t+D/64) in the same lane, so
// RoPE needs no exchange; a partial rotation over the first rope_dim dims
// (Qwen3.5: 64 of 256, Qwen35.hpp:14-16) pairs (i, i+rope_dim/2) = (t,
// t+rope_dim/64) with table rows of rope_dim floats and leaves the other dims
// as normed.  Rounding follows the reference: truncation to bf16
// after the norm, then RNE (subnormal flush) after RoPE, with the rotation
// contracted as GCC contracts the CPU op: fma(x0,c,-(x1*s)), fma(x0,s,x1*c).
//
// V lanes: lane j copies elements 8j + 64u + {0..7} (16-byte loads/stores,
// 128 contiguous bytes per row per instruction); V is never rounded: bit-exact.
//
// gamma: every q and K wave needs the same D floats.  Loaded by every wave,
// they are the same few cache lines requested by about a thousand waves per
// XCD at kernel start, and those requests queue on the L2 channels that hold
// them (config 2: 7.14 us with gamma taken as a constant, 7.51-7.53 us loaded
// per wave).  Here one wave per workgroup of kBlockWaves loads each gamma and
// stages it in LDS; every wave reads it after one barrier, met once its own
// loads are in flight (7.32-7.34 us with 8-wave workgroups; 4 waves 7.40-7.52,
// 16 waves 7.98 us; A/B on one box, two passes each).
//
// Page address of token t (global position g = pos0 + t):
//   pool + id[g/16]*page_elems + (g%16)*Hkv*D + h*D        (page layout [16][Hkv][D])
// Ids of pages opened by this call may come in the launch arguments (decode
// opens at most one page); block 0 also writes them into the device table.
#include <cstddef>

#include "common.hpp"
#include "kernels.hpp"

// Page rows are written with nontemporal stores: nothing reads them again
// within the call, and streaming them past L2 measured 11.6 -> 10.5 us
// (median C call) at 4096 tokens.
typedef unsigned int nt_u32x4 __attribute__((ext_vector_type(4)));

namespace genllm {

#pragma clang fp contract(off)

namespace {

constexpr int TPW = 1;  // tasks per wave (measured at config 2: 1 and 2 beat 4; 8 is 1.5x slower than 4)
constexpr int kBlockWaves = 8;  // waves per workgroup, sharing one staged copy of each gamma

// TR = rope_dim / 64: chunk t < TR of a lane rotates with chunk t + TR (the
// pair (i, i + rope_dim/2)); chunks from 2 TR on pass through.  TR = D/64 is
// the reference's full rotation.
template <int D, int TR>
struct Append {
    static constexpr int R = D / 32;  // 8-byte chunks per q/k row and lane
    static constexpr int U = D / 64;  // 16-byte chunks per v row and lane
    static_assert(TR >= 1 && 2 * TR <= R, "rotated chunks");
    static_assert(R % 2 == 0, "K rows are stored as pairs of 8-byte chunks");

    // Block id of local page lp (K: which = 0, V: 1): opened by this call ->
    // from the launch arguments, else from the device table.  -1 when the id
    // is outside the pool, so no store can leave it.
    // Both candidates are loaded from their own address space (launch
    // arguments, device table) and the value is selected: a pointer select
    // would make a flat load that waits on every outstanding access.
    __device__ __forceinline__ static void page_id_loads(const AppendParams& p, int lp, int which, int32_t& from_args,
                                                         int32_t& from_table) {
        const int rel = lp - p.upd.first;
        const bool opened = rel >= 0 && rel < p.upd.count;
        from_args = (which ? p.upd.v : p.upd.k)[opened ? rel : 0];
        from_table = (which ? p.v_ids : p.k_ids)[lp];
    }
    __device__ __forceinline__ static int32_t page_id_pick(const AppendParams& p, int lp, int32_t from_args,
                                                           int32_t from_table) {
        const int rel = lp - p.upd.first;
        const bool opened = rel >= 0 && rel < p.upd.count;
        const int32_t id = opened ? from_args : from_table;
        return (id >= 0 && id < p.max_blocks) ? id : -1;
    }
    __device__ __forceinline__ static int32_t page_id(const AppendParams& p, int lp, int which) {
        int32_t a, t;
        page_id_loads(p, lp, which, a, t);
        return page_id_pick(p, lp, a, t);
    }

    __device__ __forceinline__ static uint16_t* k_dst(const AppendParams& p, int tok, int h, int32_t from_args,
                                                      int32_t from_table) {
        const int gpos = p.pos0 + tok;
        const int64_t id = page_id_pick(p, gpos / kPage, from_args, from_table);
        if (id < 0) return nullptr;
        return p.k_pool + id * p.page_elems + int64_t(gpos % kPage) * p.Hkv * D + h * D;
    }

    // RMSNorm (optional, gamma chunks gw) + RoPE (optional, table chunks c4/s4
    // of the row's position) of one row, in place.
    __device__ __forceinline__ static void norm_rope(uint2 (&x)[R], bool norm, const float4 (&gw)[R], float eps, bool rope,
                                     const float4 (&c4)[TR], const float4 (&s4)[TR]) {
        float v[R][4];
#pragma unroll
        for (int t = 0; t < R; ++t) {
            v[t][0] = bf16_lo(x[t].x);
            v[t][1] = bf16_hi(x[t].x);
            v[t][2] = bf16_lo(x[t].y);
            v[t][3] = bf16_hi(x[t].y);
        }
        if (norm) {
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
                const float gv[4] = {gw[t].x, gw[t].y, gw[t].z, gw[t].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float y = (v[t][q] * r) * gv[q];
                    v[t][q] = __uint_as_float(__float_as_uint(y) & 0xFFFF0000u);  // truncating store
                }
            }
        }
        uint32_t o[R][4];
#pragma unroll
        for (int t = 0; t < R; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) o[t][q] = __float_as_uint(v[t][q]) >> 16;  // unrotated: exact
        if (rope) {
#pragma unroll
            for (int t = 0; t < TR; ++t) {
                const float c[4] = {c4[t].x, c4[t].y, c4[t].z, c4[t].w};
                const float s[4] = {s4[t].x, s4[t].y, s4[t].z, s4[t].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float x0 = v[t][q], x1 = v[t + TR][q];
                    o[t][q] = f32_to_bf16_ref(__builtin_fmaf(x0, c[q], -(x1 * s[q])));
                    o[t + TR][q] = f32_to_bf16_ref(__builtin_fmaf(x0, s[q], x1 * c[q]));
                }
            }
        }
#pragma unroll
        for (int t = 0; t < R; ++t) {
            x[t].x = pack2(o[t][0], o[t][1]);
            x[t].y = pack2(o[t][2], o[t][3]);
        }
    }

    __device__ static void run(const AppendParams& p) {
        __shared__ __attribute__((aligned(16))) float s_gamma[2][D];  // gamma_q, gamma_k of the workgroup
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
        // wave-uniform (scalar) wave index: kind, task and the gamma / table
        // pointers are then chosen in scalar registers, not by per-lane selects
        // that turn kernel-argument reads into vector loads (and a wait for
        // every load in flight)
        const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        int64_t w = int64_t(blockIdx.x) * kBlockWaves + wv;
        // Wave 0 loads gamma_q if the workgroup holds q tasks, wave 1 gamma_k if
        // it holds K tasks, first of all their loads; stage_gamma, called exactly
        // once by every wave, stores them to LDS and meets the barrier.
        constexpr int GE = D / 64;  // gamma floats per lane
        const int64_t w_first = int64_t(blockIdx.x) * kBlockWaves, w_last = w_first + kBlockWaves - 1;
        const float* gsrc = wv == 0 && w_first < wq                      ? p.gamma_q
                            : wv == 1 && w_first < wq + wk && w_last >= wq ? p.gamma_k
                                                                           : nullptr;
        float gst[GE];
        if (gsrc) {
#pragma unroll
            for (int e = 0; e < GE; ++e) gst[e] = gsrc[GE * lane + e];
        }
        auto stage_gamma = [&]() {
            if (gsrc) {
#pragma unroll
                for (int e = 0; e < GE; ++e) s_gamma[wv][GE * lane + e] = gst[e];
            }
            __syncthreads();
        };
        int kind;
        int64_t t0, n_kind;
        int ng;
        if (w < wq) {
            kind = 0, t0 = w * TPW, n_kind = nq, ng = ngq;
        } else if (w < wq + wk) {
            kind = 1, t0 = (w - wq) * TPW, n_kind = nk, ng = ngk;
        } else {
            kind = 2, t0 = (w - wq - wk) * TPW, n_kind = nk, ng = ngk;
            if (t0 >= n_kind) {
                stage_gamma();
                return;
            }
        }

        if (kind < 2) {
            const bool is_q = kind == 0;
            const int H = is_q ? p.Hq : p.Hkv;
            // Every load of the wave is issued before any arithmetic: the K page
            // ids first (the address is formed from the first load to land; the
            // load counter is in order), then the rows and the RoPE table
            // chunks of each row's position; gamma comes from LDS.
            uint2 x[TPW][R];
            float4 c4[TPW][TR], s4[TPW][TR];
            int tok[TPW], h[TPW];
            bool ok[TPW];
            int32_t id_args[TPW], id_table[TPW];  // K: the two candidates of the page id
            const bool rope = p.cos_tab != nullptr;
#pragma unroll
            for (int u = 0; u < TPW; ++u) {
                const int64_t t = t0 + u;
                tok[u] = int(t / ng);
                h[u] = int(t - int64_t(tok[u]) * ng) * 8 + r;
                ok[u] = t < n_kind && h[u] < H;
                id_args[u] = id_table[u] = -1;
                // the token (not the row) picks the page: a wave-uniform load, no divergent branch
                if (!is_q) page_id_loads(p, (p.pos0 + (t < n_kind ? tok[u] : 0)) / kPage, 0, id_args[u], id_table[u]);
            }
            const float* gamma = is_q ? p.gamma_q : p.gamma_k;
            float4 gw[R];
#pragma unroll
            for (int u = 0; u < TPW; ++u) {
                const uint16_t* src = is_q ? p.q + tok[u] * p.q_tok_stride + h[u] * p.q_head_stride
                                           : p.k + tok[u] * p.k_tok_stride + h[u] * p.k_head_stride;
#pragma unroll
                for (int c = 0; c < R; ++c)
                    x[u][c] = ok[u] ? *reinterpret_cast<const uint2*>(src + 4 * j + 32 * c) : make_uint2(0, 0);
            }
            if (rope) {
#pragma unroll
                for (int u = 0; u < TPW; ++u) {
                    const bool live = t0 + u < n_kind;
                    const int64_t row = (p.rope_pos0 + (live ? tok[u] : 0)) * p.rope_stride + 4 * j;
#pragma unroll
                    for (int c = 0; c < TR; ++c) {
                        c4[u][c] = *reinterpret_cast<const float4*>(p.cos_tab + row + 32 * c);
                        s4[u][c] = *reinterpret_cast<const float4*>(p.sin_tab + row + 32 * c);
                    }
                }
            }
            stage_gamma();
            if (gamma) {
#pragma unroll
                for (int c = 0; c < R; ++c) gw[c] = *reinterpret_cast<const float4*>(&s_gamma[is_q ? 0 : 1][4 * j + 32 * c]);
            }
            // the page ids are used only now, with every load of the wave in flight
            uint16_t* dsts[TPW];
#pragma unroll
            for (int u = 0; u < TPW; ++u) {
                __asm__ volatile("" : "+v"(id_args[u]), "+v"(id_table[u])::"memory");
                dsts[u] = !ok[u] ? nullptr
                          : is_q ? p.q_out + tok[u] * p.qo_tok_stride + h[u] * p.qo_head_stride
                                 : k_dst(p, tok[u], h[u], id_args[u], id_table[u]);
            }
#pragma unroll
            for (int u = 0; u < TPW; ++u) {
                if (t0 + u >= n_kind) break;  // wave-uniform
                norm_rope(x[u], gamma != nullptr, gw, p.eps, rope, c4[u], s4[u]);
                uint16_t* const dst = dsts[u];
                if (!dst) continue;
                if (is_q) {  // q_out is read by the attention kernel right after: plain stores keep it cached
#pragma unroll
                    for (int c = 0; c < R; ++c) *reinterpret_cast<uint2*>(dst + 4 * j + 32 * c) = x[u][c];
                } else {  // K page rows: not read again within the call
                    // 16-byte stores: lanes j and j ^ 1 swap one 8-byte part per
                    // chunk pair (c, c + 1), so that the even lane holds elements
                    // 4j .. 4j + 7 of chunk c and the odd one 4(j - 1) .. 4(j - 1) + 7
                    // of chunk c + 1 (config 2: 7.54-7.58 against 8.18-8.24 us with
                    // 8-byte stores, A/B on one box; the same swap on the q_out
                    // stores as well, written with the store kind chosen inside
                    // the loop or per chunk pair, measured 9.1-19.3 us)
                    const bool odd = j & 1;
#pragma unroll
                    for (int c = 0; c < R; c += 2) {
                        const uint2 give = odd ? x[u][c] : x[u][c + 1];
                        uint2 got;
                        got.x = __shfl_xor(give.x, 1);
                        got.y = __shfl_xor(give.y, 1);
                        const uint2 lo = odd ? got : x[u][c], hi = odd ? x[u][c + 1] : got;
                        const uint4 v = make_uint4(lo.x, lo.y, hi.x, hi.y);
                        __builtin_nontemporal_store(__builtin_bit_cast(nt_u32x4, v),
                                                    reinterpret_cast<nt_u32x4*>(dst + 4 * (j & ~1) + 32 * (c + (odd ? 1 : 0))));
                    }
                }
            }
        } else {
            uint4 xv[TPW][U];
            int64_t dst[TPW];  // element offset in the V pool, -1 = nothing to store
#pragma unroll
            for (int u = 0; u < TPW; ++u) {
                const int64_t t = t0 + u;
                const int tk = int(t / ng);
                const int hh = int(t - int64_t(tk) * ng) * 8 + r;
                const bool ok = t < n_kind && hh < p.Hkv;
                const uint16_t* src = p.v + tk * p.v_tok_stride + hh * p.v_head_stride;
#pragma unroll
                for (int c = 0; c < U; ++c)
                    xv[u][c] = ok ? *reinterpret_cast<const uint4*>(src + 8 * j + 64 * c) : make_uint4(0, 0, 0, 0);
                const int gpos = p.pos0 + tk;
                const int64_t id = ok ? page_id(p, gpos / kPage, 1) : -1;
                dst[u] = id >= 0 ? id * p.page_elems + int64_t(gpos % kPage) * p.Hkv * D + hh * D : -1;
            }
            stage_gamma();
#pragma unroll
            for (int u = 0; u < TPW; ++u)
                if (dst[u] >= 0)
#pragma unroll
                    for (int c = 0; c < U; ++c)
                        __builtin_nontemporal_store(__builtin_bit_cast(nt_u32x4, xv[u][c]),
                                                    reinterpret_cast<nt_u32x4*>(p.v_pool + dst[u] + 8 * j + 64 * c));
        }
    }
};

template <int D, int TR>
__global__ __launch_bounds__(kBlockWaves * 64) void kv_append_kernel(AppendParams p) {
    // the scalar fields and the table-update header; the opened pages' ids
    // that follow are read per lane where needed
    prefetch_kernargs<offsetof(AppendParams, upd) + 2 * sizeof(int32_t)>();
    Append<D, TR>::run(p);
}

}  // namespace

int launch_kv_append(const AppendParams& p, int head_dim, hipStream_t stream) {
    const int64_t nq = int64_t(p.S) * p.nq_tasks, nk = int64_t(p.S) * p.nkv_tasks;
    const int64_t waves = (nq + TPW - 1) / TPW + 2 * ((nk + TPW - 1) / TPW);
    int64_t blocks = (waves + kBlockWaves - 1) / kBlockWaves;
    if (blocks <= 0) {
        if (p.upd.count == 0) return GENLLM_OK;
        blocks = 1;  // table update only
    }
    // rope_dim: the rotated dims (head_dim for the reference's full rotation;
    // without tables it does not matter)
    const int rd = p.cos_tab ? (p.rope_dim ? p.rope_dim : head_dim) : head_dim;
    const dim3 g{unsigned(blocks)}, b{unsigned(kBlockWaves * 64)};
    switch (head_dim * 1000 + rd) {
        case 64 * 1000 + 64: hipLaunchKernelGGL((kv_append_kernel<64, 1>), g, b, 0, stream, p); break;
        case 128 * 1000 + 64: hipLaunchKernelGGL((kv_append_kernel<128, 1>), g, b, 0, stream, p); break;
        case 128 * 1000 + 128: hipLaunchKernelGGL((kv_append_kernel<128, 2>), g, b, 0, stream, p); break;
        case 256 * 1000 + 64: hipLaunchKernelGGL((kv_append_kernel<256, 1>), g, b, 0, stream, p); break;
        case 256 * 1000 + 128: hipLaunchKernelGGL((kv_append_kernel<256, 2>), g, b, 0, stream, p); break;
        case 256 * 1000 + 256: hipLaunchKernelGGL((kv_append_kernel<256, 4>), g, b, 0, stream, p); break;
        default:
            return fail(GENLLM_ERR_UNSUPPORTED,
                        "kv append: head_dim must be 64, 128 or 256 and rope_dim a multiple of 64 up to it");
    }
    GENLLM_LAUNCH_CHECK("kv_append_kernel");
    return GENLLM_OK;
}

}  // namespace genllm
