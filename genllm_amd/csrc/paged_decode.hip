// paged_decode.hip -- split-K paged decode attention for GQA, one launch.
//
// Computes the attention loop of PagedAttentionImpl<CPU>::execute
// (src/backend/cpu/attention.cpp:148-215) for short query chunks:
//   out[q] = sum_t softmax_t(scale * q.k_t) v_t over keys t <= q_abs (causal)
// with kv head h = q head / groups (:158) and q_abs = n_cached - S + s (:164).
//
// Grid (splits, Hkv, row chunks), 256 threads = 4 waves.  A workgroup owns one
// kv head and a contiguous range of pages; its 4 waves take pages round-robin.
// Rows = the (query, q-head) pairs of the kv head, 4 per chunk, so the K/V of a
// kv head is read once for all its GQA q heads.
//
// Per page (16 tokens) and wave:
//   S = Q K^T on v_mfma_f32_16x16x32_bf16: A = Q (rows 0..3 real, 4..15 zero),
//     B = K^T read straight from the page: lane l loads token l%16, dims
//     32c + 8(l/16) .. +7 (16 B; 64 contiguous bytes per token row per load).
//     D[m][n] lands in lane n + 16(m/4), register m%4, so lanes 0..15 hold the
//     4 rows of token l.
//   softmax: 16-lane DPP max, exp2 with scale*log2(e) folded in, running
//     (m, l) kept per lane; the row max is made wave-uniform with readfirstlane.
//   O += P V on VALU: lane l owns dims 8(l%16)..+7 of tokens 4i + l/16
//     (16-byte V loads, 4 token rows of 256 B per instruction); P goes through
//     LDS as [token][row].
// End of range: lanes and waves are reduced, the workgroup's (m, l, o) for its
// split go to the workspace, and the last workgroup of the kv head (atomic
// counter, agent-scope fences) merges all splits with the log-sum-exp rule
//   M = max m_s, L = sum l_s 2^(m_s-M), O = sum o_s 2^(m_s-M), out = O * (1/L)
// and resets the counter.  With one split the workgroup writes out directly.
#include <cfloat>

#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

namespace {
constexpr int kRows = 4;     // q rows per chunk
constexpr int kWaves = 4;

__device__ __forceinline__ float uniform(float x) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}

template <int D>
__global__ __launch_bounds__(256) void paged_decode_kernel(AttnParams p) {
    static_assert(D == 128, "decode kernel: head_dim 128");
    constexpr int KS = D / 32;     // MFMA k-steps
    constexpr int PART = D + 2;    // o[D], m, l

    __shared__ float4 lds_p[kWaves][kPage];           // p[token][row]
    __shared__ float lds_m[kWaves][kRows], lds_l[kWaves][kRows];
    __shared__ float lds_o[kWaves][kRows][D];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int n16 = lane & 15, g = lane >> 4;
    const int sp = blockIdx.x, h = blockIdx.y, z = blockIdx.z;
    const int rows_total = p.G * p.S;

    // Q operand: row m = n16 (only 0..3 are real), k-slice of lane group g.
    bf16x8_t qa[KS];
    {
        const int R = z * kRows + n16;
        const bool ok = n16 < kRows && R < rows_total;
        const uint16_t* qrow = p.q;
        if (ok) qrow = p.q + int64_t(h * p.G + R % p.G) * p.q_head_stride + int64_t(R / p.G) * p.q_tok_stride;
#pragma unroll
        for (int c = 0; c < KS; ++c) {
            uint4 u = make_uint4(0, 0, 0, 0);
            if (ok) u = *reinterpret_cast<const uint4*>(qrow + 32 * c + 8 * g);
            qa[c] = as_bf16x8(u);
        }
    }
    int qabs[kRows];
    bool rvalid[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
        const int R = z * kRows + i;
        rvalid[i] = R < rows_total;
        qabs[i] = p.causal ? p.n_cached - p.S + R / p.G : p.n_cached - 1;
    }

    const int begin = sp * p.pages_per_split;
    const int end = min(begin + p.pages_per_split, p.n_pages);
    const int last_page = (p.n_cached - 1) / kPage;

    float m_run[kRows], l_run[kRows], o[kRows][8];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) o[i][d] = 0.0f;
    }

    for (int pg = begin + wv; pg < end; pg += kWaves) {
        const int64_t kid = p.k_ids[pg], vid = p.v_ids[pg];
        const uint16_t* kbase = p.k_pool + kid * p.page_elems + h * D;
        const uint16_t* vbase = p.v_pool + vid * p.page_elems + h * D;
        uint4 kb[KS], vv[4];
#pragma unroll
        for (int c = 0; c < KS; ++c)
            kb[c] = *reinterpret_cast<const uint4*>(kbase + n16 * p.kv_row + 32 * c + 8 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            vv[i] = *reinterpret_cast<const uint4*>(vbase + (4 * i + g) * p.kv_row + 8 * n16);

        f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < KS; ++c) acc = mfma16x16x32(qa[c], as_bf16x8(kb[c]), acc);

        const int tok = pg * kPage + n16;
        float s[kRows], mx[kRows];
#pragma unroll
        for (int i = 0; i < kRows; ++i) {
            const bool ok = rvalid[i] && tok < p.n_cached && tok <= qabs[i];
            s[i] = ok ? acc[i] * p.scale_log2 : -INFINITY;
            mx[i] = uniform(row16_max(s[i]));
        }
        float alpha[kRows], pr[kRows];
#pragma unroll
        for (int i = 0; i < kRows; ++i) {
            const float mn = fmaxf(m_run[i], mx[i]);
            const float mu = mn == -INFINITY ? 0.0f : mn;
            alpha[i] = exp2_fast(m_run[i] - mu);
            pr[i] = exp2_fast(s[i] - mu);
            l_run[i] = l_run[i] * alpha[i] + pr[i];
            m_run[i] = mn;
        }
        if (g == 0) lds_p[wv][n16] = make_float4(pr[0], pr[1], pr[2], pr[3]);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < kRows; ++i)
#pragma unroll
            for (int d = 0; d < 8; ++d) o[i][d] *= alpha[i];
        const bool tail = pg == last_page;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 4 * i + g;
            const float4 pp = lds_p[wv][t];
            uint4 u = vv[i];
            if (tail && pg * kPage + t >= p.n_cached) u = make_uint4(0, 0, 0, 0);  // unfilled slots
            const float v[8] = {bf16_lo(u.x), bf16_hi(u.x), bf16_lo(u.y), bf16_hi(u.y),
                                bf16_lo(u.z), bf16_hi(u.z), bf16_lo(u.w), bf16_hi(u.w)};
            const float pw[4] = {pp.x, pp.y, pp.z, pp.w};
#pragma unroll
            for (int r = 0; r < kRows; ++r)
#pragma unroll
                for (int d = 0; d < 8; ++d) o[r][d] = __builtin_fmaf(pw[r], v[d], o[r][d]);
        }
        __builtin_amdgcn_wave_barrier();
    }

    // lane reductions: l over the 16 token lanes, o over the 4 token groups
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
        l_run[i] = row16_sum(l_run[i]);
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            o[i][d] += __shfl_xor(o[i][d], 16);
            o[i][d] += __shfl_xor(o[i][d], 32);
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < kRows; ++i) {
            lds_m[wv][i] = m_run[i];
            lds_l[wv][i] = l_run[i];
        }
    }
    if (g == 0) {
#pragma unroll
        for (int i = 0; i < kRows; ++i)
#pragma unroll
            for (int d = 0; d < 8; ++d) lds_o[wv][i][8 * n16 + d] = o[i][d];
    }
    __syncthreads();

    // workgroup merge: thread -> (row i, dims d2, d2+1)
    const int i = threadIdx.x >> 6;
    const int d2 = (threadIdx.x & 63) * 2;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, lds_m[w][i]);
    float L = 0.0f, O0 = 0.0f, O1 = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float e = exp2_fast(lds_m[w][i] - M);
            L += lds_l[w][i] * e;
            O0 += lds_o[w][i][d2] * e;
            O1 += lds_o[w][i][d2 + 1] * e;
        }
    }
    const int R = z * kRows + i;
    const bool row_ok = R < rows_total;
    uint16_t* orow = row_ok ? p.out + int64_t(h * p.G + R % p.G) * p.o_head_stride + int64_t(R / p.G) * p.o_tok_stride
                            : nullptr;

    if (p.n_splits == 1) {
        if (row_ok) {
            const float inv = 1.0f / L;
            *reinterpret_cast<uint32_t*>(orow + d2) = pack2(f32_to_bf16_ref(O0 * inv), f32_to_bf16_ref(O1 * inv));
        }
        return;
    }

    const int unit = h * p.n_chunks + z;
    float* part = p.partial + ((int64_t(unit) * p.n_splits + sp) * kRows + i) * PART;
    part[d2] = O0;
    part[d2 + 1] = O1;
    if (d2 == 0) {
        part[D] = M;
        part[D + 1] = L;
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = atomicAdd(p.counters + unit, 1);
        s_last = prev == p.n_splits - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    // last workgroup of this kv head: merge every split
    M = -INFINITY;
    L = 0.0f;
    O0 = 0.0f;
    O1 = 0.0f;
    const float* base = p.partial + (int64_t(unit) * p.n_splits * kRows + i) * PART;
    for (int s2 = 0; s2 < p.n_splits; ++s2) {
        const float* ps = base + int64_t(s2) * kRows * PART;
        const float ms = __builtin_nontemporal_load(ps + D);
        const float ls = __builtin_nontemporal_load(ps + D + 1);
        const float o0 = __builtin_nontemporal_load(ps + d2);
        const float o1 = __builtin_nontemporal_load(ps + d2 + 1);
        const float mn = fmaxf(M, ms);
        if (mn == -INFINITY) continue;
        const float a = exp2_fast(M - mn), b = exp2_fast(ms - mn);
        L = L * a + ls * b;
        O0 = O0 * a + o0 * b;
        O1 = O1 * a + o1 * b;
        M = mn;
    }
    if (row_ok) {
        const float inv = 1.0f / L;
        *reinterpret_cast<uint32_t*>(orow + d2) = pack2(f32_to_bf16_ref(O0 * inv), f32_to_bf16_ref(O1 * inv));
    }
    if (threadIdx.x == 0) p.counters[unit] = 0;
}

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

}  // namespace

size_t decode_workspace_bytes(int Hq, int Hkv, int S, int D, int n_pages) {
    if (Hkv <= 0 || Hq <= 0 || S <= 0 || D <= 0 || n_pages <= 0) return 0;
    const int G = Hq / Hkv;
    const int chunks = (G * S + kRows - 1) / kRows;
    const size_t units = size_t(Hkv) * chunks;
    return round_up(units * sizeof(int32_t), 256) + units * size_t(n_pages) * kRows * (D + 2) * sizeof(float);
}

// Choose pages per split: about two workgroups per CU over all kv heads and row
// chunks.  GENLLM_DECODE_PPS overrides (tuning).
int decode_plan(AttnParams& p, int D, size_t ws_bytes, void* ws) {
    p.n_chunks = (p.G * p.S + kRows - 1) / kRows;
    const int64_t units = int64_t(p.Hkv) * p.n_chunks;
    int pps = 0;
    if (const char* e = getenv("GENLLM_DECODE_PPS")) pps = atoi(e);
    if (pps <= 0) {
        const int64_t target = 2 * int64_t(device_cu_count());
        pps = int((int64_t(p.n_pages) * units + target - 1) / target);
        if (pps < 4) pps = 4;  // one page per wave at least
    }
    p.pages_per_split = pps;
    p.n_splits = (p.n_pages + pps - 1) / pps;
    if (p.n_splits > 1) {
        const size_t cnt_bytes = round_up(size_t(units) * sizeof(int32_t), 256);
        const size_t need = cnt_bytes + size_t(units) * p.n_splits * kRows * (D + 2) * sizeof(float);
        if (!ws || ws_bytes < need)
            return fail(GENLLM_ERR_INVALID, "paged decode: workspace too small (need " + std::to_string(need) +
                                                " bytes, have " + std::to_string(ws_bytes) + ")");
        p.counters = reinterpret_cast<int32_t*>(ws);
        p.partial = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + cnt_bytes);
    }
    return GENLLM_OK;
}

int launch_paged_decode(const AttnParams& p, int head_dim, hipStream_t stream) {
    if (head_dim != 128) return fail(GENLLM_ERR_UNSUPPORTED, "paged decode: head_dim must be 128");
    if (p.n_pages <= 0) return GENLLM_OK;
    dim3 grid(p.n_splits, p.Hkv, p.n_chunks);
    hipLaunchKernelGGL(paged_decode_kernel<128>, grid, dim3(256), 0, stream, p);
    GENLLM_LAUNCH_CHECK("paged_decode_kernel");
    return GENLLM_OK;
}

}  // namespace genllm
