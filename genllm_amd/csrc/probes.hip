// probes.hip -- read-floor probes for the benchmark (libgenllm_probe.so; the
// product library does not contain them).  Each probe moves exactly the bytes
// of one hot-path kernel with that kernel's launch shape and access pattern
// and no arithmetic, so that bench.py can report, next to each kernel's time,
// what the same memory traffic costs on its own:
//   * genllm_probe_stream_read: a contiguous stream of `bytes` (one 16-byte
//     nontemporal load per thread) -- the best case for that many bytes;
//   * genllm_probe_decode_read: the split decode kernel's page loads (grid
//     (Hkv / heads per workgroup, splits), 8 waves up to 128 pages per split
//     or with 4 heads per workgroup, else 4, each head's pages dealt to its
//     waves round-robin, one page in flight per wave, K operand chunks and V
//     rows with 16-byte nt buffer loads), folded with XOR instead of the
//     attention math and the split merge;
//   * genllm_probe_append_copy: the fused append's data movement (one wave per
//     8 rows of one token: K rows as 8-byte loads and, after a lane-pair swap,
//     16-byte nt stores; V rows as 16-byte loads and nt stores; page ids from
//     the device table) without the norm and RoPE.
// A probe result never reaches memory except through an impossible branch
// (the fold equal to a constant), which keeps the loads alive.
#include <climits>
#include <cstdint>

#include "common.hpp"

namespace genllm {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kNt = 2;  // buffer-access cache policy: nontemporal

__device__ __forceinline__ uint32_t fold4(u32x4 a) { return a.x ^ a.y ^ a.z ^ a.w; }

// one 16-byte load per thread, as many workgroups as the buffer needs: of the
// shapes measured (grid-stride with 1-8 loads in flight per thread, block-
// contiguous chunks) the fastest at 33.6 and 134 MB
__global__ __launch_bounds__(256) void probe_stream_kernel(const u32x4* p, int64_t n, uint32_t* sink) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const uint32_t acc = i < n ? fold4(__builtin_nontemporal_load(p + i)) : 0u;
    if (acc == 0x9E3779B9u) sink[blockIdx.x & 0xFFFF] = acc;
}

template <int D, int W, int HPW>
__global__ __launch_bounds__(W * 64) void probe_decode_kernel(const uint16_t* k_pool, const uint16_t* v_pool,
                                                              const int32_t* k_ids, const int32_t* v_ids, int n_pages,
                                                              int pps, int64_t page_elems, int64_t kv_row,
                                                              uint32_t* sink) {
    constexpr int KS = D / 32, VH = D / 128;
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n16 = lane & 15, g = lane >> 4;
    constexpr int WP = W / HPW;  // waves per kv head
    const int h = int(blockIdx.x) * HPW + wv / WP, wi = wv % WP, sp = blockIdx.y;
    const int begin = sp * pps, end = min(begin + pps, n_pages);
    const int np = end - begin - wi > 0 ? (end - begin - wi + WP - 1) / WP : 0;  // <= 64 (checked by the host)
    const int kid = lane < np ? k_ids[begin + wi + WP * lane] : 0;
    const int vid = lane < np ? v_ids[begin + wi + WP * lane] : 0;
    const int kcol_b = int(2 * (h * D + n16 * kv_row + 8 * g)), vcol_b = int(2 * (h * D + 4 * g * kv_row + 8 * n16));
    const int row_b = int(2 * kv_row), page_b = int(2 * page_elems);
    uint32_t acc = 0;
    u32x4 k[KS], v[4][VH];
    auto load = [&](int j) {
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(k_pool) + int64_t(__builtin_amdgcn_readlane(kid, j)) * page_elems, 0, page_b,
            kBufferFlags);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t*>(v_pool) + int64_t(__builtin_amdgcn_readlane(vid, j)) * page_elems, 0, page_b,
            kBufferFlags);
#pragma unroll
        for (int c = 0; c < KS; ++c)
            k[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, kcol_b + 64 * c, 0, kNt));
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int hh = 0; hh < VH; ++hh)
                v[i][hh] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, vcol_b + 256 * hh,
                                                                                          i * row_b, kNt));
    };
    // one page in flight: page j + 1 is requested once page j has landed
    if (np > 0) load(0);
    for (int j = 0; j < np; ++j) {
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        uint32_t f = 0;
#pragma unroll
        for (int c = 0; c < KS; ++c) f ^= fold4(k[c]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int hh = 0; hh < VH; ++hh) f ^= fold4(v[i][hh]);
        acc += f;
        if (j + 1 < np) load(j + 1);
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.y * gridDim.x + blockIdx.x] = acc;
}

// one wave per task (8 rows = 8 kv heads of one token) of K, then of V
template <int D>
__global__ __launch_bounds__(256) void probe_append_kernel(const uint16_t* k, const uint16_t* v, uint16_t* k_pool,
                                                           uint16_t* v_pool, const int32_t* k_ids,
                                                           const int32_t* v_ids, int S, int Hkv, int64_t page_elems) {
    constexpr int R = D / 32, U = D / 64;
    const int lane = threadIdx.x & 63, r = lane >> 3, j = lane & 7;
    const int ng = (Hkv + 7) / 8;
    const int64_t nk = int64_t(S) * ng;
    const int64_t w = int64_t(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (w >= 2 * nk) return;
    const bool is_v = w >= nk;
    const int64_t t = is_v ? w - nk : w;
    const int tok = int(t / ng), h = int(t % ng) * 8 + r;
    if (h >= Hkv) return;
    const int64_t id = (is_v ? v_ids : k_ids)[tok / kPage];
    const int64_t dst = id * page_elems + int64_t(tok % kPage) * Hkv * D + int64_t(h) * D;
    const int64_t src = (int64_t(tok) * Hkv + h) * D;  // token-major [S][Hkv][D]
    if (!is_v) {
        uint2 x[R];
#pragma unroll
        for (int c = 0; c < R; ++c) x[c] = *reinterpret_cast<const uint2*>(k + src + 4 * j + 32 * c);
        const bool odd = j & 1;
#pragma unroll
        for (int c = 0; c < R; c += 2) {
            const uint2 give = odd ? x[c] : x[c + 1];
            uint2 got;
            got.x = __shfl_xor(give.x, 1);
            got.y = __shfl_xor(give.y, 1);
            const uint2 lo = odd ? got : x[c], hi = odd ? x[c + 1] : got;
            __builtin_nontemporal_store(u32x4{lo.x, lo.y, hi.x, hi.y},
                                        reinterpret_cast<u32x4*>(k_pool + dst + 4 * (j & ~1) + 32 * (c + (odd ? 1 : 0))));
        }
    } else {
        u32x4 x[U];
#pragma unroll
        for (int c = 0; c < U; ++c) x[c] = *reinterpret_cast<const u32x4*>(v + src + 8 * j + 64 * c);
#pragma unroll
        for (int c = 0; c < U; ++c)
            __builtin_nontemporal_store(x[c], reinterpret_cast<u32x4*>(v_pool + dst + 8 * j + 64 * c));
    }
}

}  // namespace
}  // namespace genllm

using namespace genllm;

extern "C" int genllm_probe_stream_read(const void* p, size_t bytes, void* sink, void* stream) {
    if (!p || !sink || bytes % 16) return GENLLM_ERR_INVALID;
    const int64_t n = int64_t(bytes / 16);
    if (n <= 0 || (n + 255) / 256 > INT32_MAX) return GENLLM_ERR_INVALID;
    hipLaunchKernelGGL(probe_stream_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const u32x4*>(p), n, static_cast<uint32_t*>(sink));
    return hipGetLastError() == hipSuccess ? GENLLM_OK : GENLLM_ERR_HIP;
}

// The decode's page loads for n_pages pages of n_kv_heads heads (page layout
// [16][Hkv][D]) in splits of pages_per_split pages, heads_per_wg (1 or 4) kv
// heads per workgroup.
extern "C" int genllm_probe_decode_read(const void* k_pool, const void* v_pool, const int32_t* k_ids,
                                        const int32_t* v_ids, int32_t n_pages, int32_t n_kv_heads, int32_t head_dim,
                                        int32_t pages_per_split, int32_t heads_per_wg, void* sink, void* stream) {
    if (!k_pool || !v_pool || !k_ids || !v_ids || !sink || n_pages <= 0 || n_kv_heads <= 0 || pages_per_split <= 0)
        return GENLLM_ERR_INVALID;
    if (head_dim != 128 || pages_per_split > 64 * 4) return GENLLM_ERR_UNSUPPORTED;
    if (heads_per_wg != 1 && (heads_per_wg != 4 || n_kv_heads % 4 || pages_per_split > 64 * 2))
        return GENLLM_ERR_UNSUPPORTED;
    const int splits = (n_pages + pages_per_split - 1) / pages_per_split;
    const int64_t kv_row = int64_t(n_kv_heads) * head_dim, page_elems = kPage * kv_row;
    const auto s = static_cast<hipStream_t>(stream);
    const auto* kp = static_cast<const uint16_t*>(k_pool);
    const auto* vp = static_cast<const uint16_t*>(v_pool);
    auto* o = static_cast<uint32_t*>(sink);
    if (heads_per_wg == 4)
        hipLaunchKernelGGL((probe_decode_kernel<128, 8, 4>), dim3(n_kv_heads / 4, splits), dim3(512), 0, s, kp, vp,
                           k_ids, v_ids, n_pages, pages_per_split, page_elems, kv_row, o);
    else if (pages_per_split <= 128)
        hipLaunchKernelGGL((probe_decode_kernel<128, 8, 1>), dim3(n_kv_heads, splits), dim3(512), 0, s, kp, vp, k_ids,
                           v_ids, n_pages, pages_per_split, page_elems, kv_row, o);
    else
        hipLaunchKernelGGL((probe_decode_kernel<128, 4, 1>), dim3(n_kv_heads, splits), dim3(256), 0, s, kp, vp, k_ids,
                           v_ids, n_pages, pages_per_split, page_elems, kv_row, o);
    return hipGetLastError() == hipSuccess ? GENLLM_OK : GENLLM_ERR_HIP;
}

// The append's movement of S tokens of token-major k, v [S][Hkv][D] into the
// pages of k_ids / v_ids (positions 0 .. S-1).
extern "C" int genllm_probe_append_copy(const void* k, const void* v, void* k_pool, void* v_pool, const int32_t* k_ids,
                                        const int32_t* v_ids, int32_t seq_len, int32_t n_kv_heads, int32_t head_dim,
                                        void* stream) {
    if (!k || !v || !k_pool || !v_pool || !k_ids || !v_ids || seq_len <= 0 || n_kv_heads <= 0)
        return GENLLM_ERR_INVALID;
    if (head_dim != 128) return GENLLM_ERR_UNSUPPORTED;
    const int64_t tasks = 2 * int64_t(seq_len) * ((n_kv_heads + 7) / 8);
    hipLaunchKernelGGL((probe_append_kernel<128>), dim3(unsigned((tasks + 3) / 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(k),
                       static_cast<const uint16_t*>(v), static_cast<uint16_t*>(k_pool), static_cast<uint16_t*>(v_pool),
                       k_ids, v_ids, seq_len, n_kv_heads, int64_t(kPage) * n_kv_heads * head_dim);
    return hipGetLastError() == hipSuccess ? GENLLM_OK : GENLLM_ERR_HIP;
}
