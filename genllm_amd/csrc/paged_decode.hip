// paged_decode.hip -- split-K paged decode attention for GQA.
//
// Computes the attention loop of PagedAttentionImpl<CPU>::execute
// (src/backend/cpu/attention.cpp:148-215) for short query chunks:
//   out[q] = sum_t softmax_t(scale * q.k_t) v_t over keys t <= q_abs (causal)
// with kv head h = q head / groups (:158) and q_abs = n_cached - S + s (:164).
//
// Split kernel: grid (Hkv / HPW, splits), W = 4 or 8 waves.  A workgroup owns
// HPW kv heads (1, or 4 for long page ranges) and a contiguous range of
// pages; the W / HPW waves of each head take its pages round-robin.
// The kv head is the fastest grid index: the dispatcher deals workgroups to the
// 8 XCDs round-robin, so with 8 kv heads and one head per workgroup every
// split of head h (and, with the same order in the merge grid, that head's
// merge) runs on XCD h.  8 waves serve ranges of up to kWideMaxPps pages at
// D = 128 (config 3's 17) and every 4-head workgroup: each wave then owns half
// the pages of a 4-wave form, so a split finishes in fewer dependent memory
// round trips.  Longer one-head ranges, and D = 256, keep 4 waves.  The rows of the kv head -- its (query, GQA q-head) pairs, at
// most 16 -- are the 16 columns of the MFMA tiles, so K/V are read once for all
// of them.
//
// Per page (16 tokens) and wave, on MFMA only:
//   S^T = K Q^T  v_mfma_f32_16x16x32_bf16 x D/32: A = K straight from the page
//        (lane l: token l%16, dims 32c+8(l/16)..+7, 16-byte loads), B = Q^T held
//        in registers (lane l: row l%16).  D[tok][row] lands in lane row + 16g,
//        register i = tok - 4g: each lane holds 4 keys of ONE row, so the row
//        max is an in-lane max plus two cross-lane steps, and the running
//        (m, l) of a row live in its lanes.
//   O^T += V^T P^T  v_mfma_f32_16x16x16_bf16 x D/16: B = P^T is the lane's own 4
//        probabilities (tokens 4g..4g+3 of its row) as bf16; A = V^T: each lane
//        loads V for tokens 4g..4g+3, dims 8(l%16)..+7 (16-byte loads) and writes
//        them to LDS transposed ([dim][token], 8-byte stores), then reads the
//        A operand (dim l%16 of a 16-dim block, tokens 4g..4g+3) back.
//        O^T[dim][row] is again lane-local to the row, so the rescale by
//        2^(m_old - m_new) needs no exchange.
// Memory-level parallelism: the wave reads the block-table entries of all its
// pages with one load up front and keeps PF pages of K/V in flight in
// registers (page j+PF-1 is requested before page j is computed).
//
// End of range: the 4 waves are merged through LDS and the workgroup's
// (m, l, o) per row go to the workspace; a second kernel merges the splits with
// the log-sum-exp rule  M = max m_s, L = sum l_s 2^(m_s-M),
// O = sum o_s 2^(m_s-M), out = O * (1/L).  With one split the workgroup writes
// the output directly.  (A single launch in which the last workgroup merges
// needs agent-scope fences -- an L2 write-back and invalidate per workgroup on
// gfx950 -- and measured slower.)
#include <atomic>
#include <cfloat>
#include <string>

#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

namespace {
constexpr int kRows = 16;      // rows (query x q-head pairs) per kv head
constexpr int kWaves = 4;       // waves of a split workgroup (long page ranges)
constexpr int kWideWaves = 8;   // waves of a split workgroup over short ranges (D = 128)
// pages per split up to which the 8-wave form runs (measured at config 5, 64
// pages: 29.5 against 31.0 us per layer with 4 waves, and 30.1 against 31.2
// for the captured decode step, whose plan covers 65)
constexpr int kWideMaxPps = 128;
// Long page ranges: 4 kv heads per 8-wave workgroup (2 waves per head), so
// that a workgroup reads 1 KB of every token row of its pages instead of one
// head's 256 bytes at a 2 KB stride, for 4x the splits.  Used when a one-head
// plan would give kMultiHeadMinPps pages per split or more (config 5's 64;
// config 3's 16 keeps one head).  Measured at config 5 (A/B on one box, two
// passes): 27.6-27.8 against 28.8-28.9 us per layer eager, 29.1 against 30.2
// as a replayed graph; 2 heads per workgroup 27.8-28.0 (graph 28.6), 8 heads
// 29.7, 4 heads with two pages in flight per wave 28.2.
constexpr int kMultiHead = 4;
constexpr int kMultiHeadMinPps = 48;
constexpr int kMergeU = 16;     // splits in flight per merge lane
constexpr size_t kSplitLeadArgBytes = 56;  // the split kernel's scalar arguments ahead of the parameter block
constexpr int kMergeDims = 64;  // dims per merge workgroup
constexpr int kMaxSplits = 256;
// pages in flight per wave: 1 at D = 128 (a wave requests page j+1 only after
// page j's data has arrived; measured faster than 2 or 3 at 8K and 32K keys:
// more bytes in flight per CU only lengthen the memory queues), 2 at D = 256
template <int D>
constexpr int kPagesInFlight = D == 128 ? 1 : 2;
constexpr int VT_ROW = kPage + 4;  // LDS V^T row: 16 tokens + pad (bf16 elements)
constexpr int kNonTemporal = 2;    // buffer-access cache policy bit nt (gfx950: sc0 = 1, nt = 2, sc1 = 16)
// Cache policy sc1 (agent scope): a store completes at the device's coherence
// point and a load reads from it, past the XCD-local caches.  This is what the
// compiler emits for relaxed agent-scope atomic stores and loads on gfx950.
constexpr int kCoherent = 16;
typedef unsigned int v2u32 __attribute__((ext_vector_type(2)));

// Buffer resource over the split partials: o [Hkv][split][row][D], then
// {m, l} [Hkv][split][row].
template <int D>
__device__ __forceinline__ auto part_rsrc(const AttnParams& p) {
    const int rows = p.G * p.S;
    const int bytes = int(int64_t(p.Hkv) * p.n_splits * rows * (D + 2) * 4);
    return __builtin_amdgcn_make_buffer_rsrc(p.partial, 0, bytes, kBufferFlags);
}

// Single-launch merge, run by every split workgroup after it has stored its
// partial (sc1): the workgroup counts its arrival on its kv head, and the last
// one to arrive merges all splits of that head with the log-sum-exp rule
//   M = max m_s, L = sum l_s 2^(m_s-M), O = sum o_s 2^(m_s-M), out = O * (1/L)
// and resets the counter for the next launch.  Ordering: each wave waits for
// its own partial stores to complete (vmcnt(0)) before the barrier that
// precedes the count, and the last workgroup loads the partials only after the
// count has returned, from the coherence point (sc1) -- so no L2 write-back or
// invalidate is needed.  Merge work: W waves over (row, split) pairs -- for
// R < W rows, W/R waves share a row's splits -- with up to kMergeU splits in
// flight per lane, then the per-wave states meet in LDS.
template <int D, int W, bool F16>
__device__ __forceinline__ void merge_last_arrival(const AttnParams& p, int h, float (&lds_m)[W][kRows],
                                                   float (&lds_l)[W][kRows], float (&lds_o)[W][kRows][D + 4]) {
    constexpr int VH = D / 128;
    constexpr int U = kMergeU;
    __shared__ int s_last;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int R = p.G * p.S, ns = p.n_splits;
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(p.counters + h, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old == ns - 1;
        if (last) __hip_atomic_store(p.counters + h, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;

    const auto rs = part_rsrc<D>(p);
    const int64_t ml_base = int64_t(p.Hkv) * ns * R * D;  // float index of {m, l}
    const int wpr = R < W ? W / R : 1;                     // waves per row
    const int sub = wv % wpr;
    for (int r = wv / wpr; r < R; r += W / wpr) {
        float mw = -INFINITY, lw = 0.0f, o0[VH], o1[VH];
#pragma unroll
        for (int hh = 0; hh < VH; ++hh) o0[hh] = o1[hh] = 0.0f;
        for (int s0 = sub; s0 < ns; s0 += wpr * U) {
            float2 ov[U][VH], mv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int s2 = s0 + wpr * u;
                const int64_t row = (int64_t(h) * ns + s2) * R + r;
#pragma unroll
                for (int hh = 0; hh < VH; ++hh)
                    ov[u][hh] = s2 < ns ? __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                                                         rs, int(4 * (row * D + 128 * hh + 2 * lane)),
                                                                         0, kCoherent))
                                        : make_float2(0.0f, 0.0f);
                mv[u] = s2 < ns ? __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                                                 rs, int(4 * (ml_base + 2 * row)), 0, kCoherent))
                                : make_float2(-INFINITY, 0.0f);
            }
            float bm = mw;
#pragma unroll
            for (int u = 0; u < U; ++u) bm = fmaxf(bm, mv[u].x);
            if (bm == -INFINITY) continue;  // nothing visible yet
            const float a = mw == -INFINITY ? 0.0f : exp2_fast(mw - bm);
            lw *= a;
#pragma unroll
            for (int hh = 0; hh < VH; ++hh) {
                o0[hh] *= a;
                o1[hh] *= a;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float w = mv[u].x == -INFINITY ? 0.0f : exp2_fast(mv[u].x - bm);
                lw += mv[u].y * w;
#pragma unroll
                for (int hh = 0; hh < VH; ++hh) {
                    o0[hh] += ov[u][hh].x * w;
                    o1[hh] += ov[u][hh].y * w;
                }
            }
            mw = bm;
        }
#pragma unroll
        for (int hh = 0; hh < VH; ++hh) {
            lds_o[sub][r][128 * hh + 2 * lane] = o0[hh];
            lds_o[sub][r][128 * hh + 2 * lane + 1] = o1[hh];
        }
        if (lane == 0) {
            lds_m[sub][r] = mw;
            lds_l[sub][r] = lw;
        }
    }
    __syncthreads();
    for (int r = wv; r < R; r += W) {
        float M = -INFINITY;
        for (int w2 = 0; w2 < wpr; ++w2) M = fmaxf(M, lds_m[w2][r]);
        float L = 0.0f, O0[VH], O1[VH];
#pragma unroll
        for (int hh = 0; hh < VH; ++hh) O0[hh] = O1[hh] = 0.0f;
        for (int w2 = 0; w2 < wpr; ++w2) {
            const float e = lds_m[w2][r] == -INFINITY ? 0.0f : exp2_fast(lds_m[w2][r] - M);
            L += lds_l[w2][r] * e;
#pragma unroll
            for (int hh = 0; hh < VH; ++hh) {
                O0[hh] += lds_o[w2][r][128 * hh + 2 * lane] * e;
                O1[hh] += lds_o[w2][r][128 * hh + 2 * lane + 1] * e;
            }
        }
        const float inv = 1.0f / L;
        uint16_t* orow = p.out + int64_t(h * p.G + r % p.G) * p.o_head_stride + int64_t(r / p.G) * p.o_tok_stride;
#pragma unroll
        for (int hh = 0; hh < VH; ++hh)
            *reinterpret_cast<uint32_t*>(orow + 128 * hh + 2 * lane) =
                pack2(Elem<F16>::out(O0[hh] * inv), Elem<F16>::out(O1[hh] * inv));
    }
}

// Two probabilities as the PV MFMA's 16-bit operand, round to nearest even.
// bf16: converted one by one and packed (measured 0.15 us faster per config-3
// decode than one v_cvt_pk_bf16_f32 per pair, which the compiler schedules
// differently around the V^T reads).
template <bool F16>
__device__ __forceinline__ uint32_t pack_p(float lo, float hi) {
    if constexpr (F16) {
        return Elem<true>::pack_p(lo, hi);
    } else {
        const __bf16 a = static_cast<__bf16>(lo), b = static_cast<__bf16>(hi);
        return uint32_t(__builtin_bit_cast(uint16_t, a)) | (uint32_t(__builtin_bit_cast(uint16_t, b)) << 16);
    }
}

template <int D>
struct PageRegs {
    uint4 k[D / 32];       // K^T operand chunks
    uint4 v[4][D / 128];   // V rows of tokens 4g..4g+3, dims 8 n16 + 128 hh
    int kid, vid;          // the page's block ids (wave-uniform)
};

// Reads a word of the step control block at the device's coherence point
// (written by the previous step's last workgroup on another XCD).
__device__ __forceinline__ int step_load(const int32_t* at) {
    return __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(const_cast<int32_t*>(at), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// The fields the first loads need (block table, split range, the ids opened
// by this call, q) come first as scalars (14 dwords), ahead of the parameter
// block, so that they can be preloaded into SGPRs at wave launch: the page-id
// and q loads then leave without an argument read before them.
template <int D, int W, bool kStep, bool F16, int HPW>
__global__ __launch_bounds__(W * 64) void paged_decode_kernel(const int32_t* k_ids, const int32_t* v_ids,
                                                              const uint16_t* q, int32_t q_head_stride,
                                                              int32_t q_tok_stride, int32_t G, int32_t S,
                                                              int32_t pages_per_split, int32_t n_pages_arg,
                                                              int32_t upd_first, int32_t upd_count, AttnParams p) {
    using E = Elem<F16>;
    static_assert(D == 128 || D == 256, "decode kernel: head_dim 128 or 256");
    constexpr int KS = D / 32;   // S^T k-steps
    constexpr int DB = D / 16;   // O^T dim blocks
    constexpr int VH = D / 128;  // 128-dim halves of a V row per lane
    constexpr int PF = kPagesInFlight<D>;

    __shared__ __attribute__((aligned(16))) uint16_t lds_vt[W][D * VT_ROW];
    __shared__ float lds_m[W][kRows], lds_l[W][kRows];
    __shared__ float lds_o[W][kRows][D + 4];

    // the wave index in a scalar register: page ranges and the special-page
    // branches below are then wave-uniform to the compiler as well
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n16 = lane & 15, g = lane >> 4;
    // HPW kv heads per workgroup: waves [WP lh, WP lh + WP) serve head
    // blockIdx.x HPW + lh and take its pages round-robin
    constexpr int WP = W / HPW;
    static_assert(W % HPW == 0, "decode kernel: whole waves per kv head");
    const int lh = HPW == 1 ? 0 : wv / WP, wi = HPW == 1 ? wv : wv - lh * WP;
    const int h = int(blockIdx.x) * HPW + lh, sp = blockIdx.y;
    const int rows_total = G * S;  // <= 16

    // q rows and the block-table entries of the wave's planned page range are
    // requested first: neither depends on the cache position, so in a
    // device-position step their round trip overlaps the position's.  (The
    // table holds ids up to the planned end; the wave uses only those below
    // the step's own end.)
    const int r = n16;  // this lane's row (MFMA column): q head h*G + r%G, query r/G
    const bool row_ok = r < rows_total;
    uint4 qb[KS];  // Q^T operand chunks (raw 16-bit elements)
    {
        const uint16_t* qrow = q + int64_t(h * G + r % G) * q_head_stride + int64_t(r / G) * q_tok_stride;
#pragma unroll
        for (int c = 0; c < KS; ++c) {
            uint4 u = make_uint4(0, 0, 0, 0);
            if (row_ok) u = *reinterpret_cast<const uint4*>(qrow + 32 * c + 8 * g);
            qb[c] = u;
        }
    }
    const int begin = sp * pages_per_split;
    const int end_plan = min(begin + pages_per_split, n_pages_arg);
    const int np_plan = end_plan - begin - wi > 0 ? (end_plan - begin - wi + WP - 1) / WP : 0;
    // fused append: page ids opened by this call come from the launch arguments
    if (sp == 0 && blockIdx.x == 0 && threadIdx.x < upd_count) {
        p.k_ids_w[upd_first + threadIdx.x] = p.upd.k[threadIdx.x];
        p.v_ids_w[upd_first + threadIdx.x] = p.upd.v[threadIdx.x];
    }
    // Block-table entries of the wave's pages, 64 at a time: lane i holds the
    // ids of the wave's page 64 b + i of id block b.  The current block is in
    // my_kid / my_vid, the next one (requested as the wave enters the current
    // one) in nx_kid / nx_vid, so a split may span any number of pages.
    // (Loading both candidates, from the launch arguments and the table, and
    // selecting the value measured 0.25 us slower at config 3: every lane then
    // reads the launch arguments.)
    auto fetch_ids = [&](int b, int& kid, int& vid) {
        kid = vid = 0;
        const int jj = 64 * b + lane;
        if (jj < np_plan) {
            const int pg = begin + wi + WP * jj;
            const int rel = pg - upd_first;
            if (rel >= 0 && rel < upd_count) {
                kid = p.upd.k[rel];
                vid = p.upd.v[rel];
            } else {
                kid = k_ids[pg];
                vid = v_ids[pg];
            }
        }
    };
    int my_kid, my_vid, nx_kid = 0, nx_vid = 0;
    fetch_ids(0, my_kid, my_vid);
    if (np_plan > 64) fetch_ids(1, nx_kid, nx_vid);  // wave-uniform
    // the parameter block's lines, all at once, with the id and q loads already
    // in flight (the block's reads below then hit the scalar cache)
    prefetch_kernargs<kSplitLeadArgBytes + sizeof(AttnParams)>();

    // Cache position: from the launch arguments, or (device-position step)
    // from the control block, where a step that would pass the staged limit
    // or the pages the grid was planned for only raises the error flag.
    int n_cached = p.n_cached, n_pages = n_pages_arg, new_from = p.new_from, step_pos = 0;
    if constexpr (kStep) {
        step_pos = step_load(p.step + kStepPos);
        const int limit = step_load(p.step + kStepLimit);
        if (step_load(p.step + kStepError)) return;  // an earlier kernel of this or a previous step was refused
        if (step_pos < 0 || step_pos > limit - S || (step_pos + S + kPage - 1) / kPage > n_pages_arg) {
            if (threadIdx.x == 0)
                __hip_atomic_store(p.step + kStepError, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        n_cached = step_pos + p.S;
        n_pages = (n_cached + kPage - 1) / kPage;
        new_from = step_pos;
    }

    const int qabs = p.causal ? n_cached - p.S + r / p.G : n_cached - 1;
    const int end = min(begin + pages_per_split, n_pages);
    const int np = end - begin - wi > 0 ? (end - begin - wi + WP - 1) / WP : 0;  // <= np_plan
    // Element offsets inside a page (< 2^31): lane's K operand chunk (token
    // n16, dims 8g + 32c) and V row chunk (token 4g + i, dims 8 n16).  Page
    // bases are wave-uniform, so a load is a scalar base plus this offset.
    const uint32_t kcol = uint32_t(h * D + n16 * p.kv_row + 8 * g);
    const uint32_t vcol = uint32_t(h * D + 4 * g * p.kv_row + 8 * n16);
    const int kcol_b = int(2 * kcol), vcol_b = int(2 * vcol);  // the same in bytes
    const int kv_row_b = int(2 * p.kv_row), page_bytes = int(2 * p.page_elems);
    const bool fused = p.k_new != nullptr;
    uint16_t* vt = lds_vt[wv];
    // Pages from special_from on hold the end of the cache: keys a query may
    // not see (causal), slots past n_cached and, in the fused op, the appended
    // tokens.  Only they take the per-token conditions below.
    const int lo_tok = min(p.causal ? n_cached - p.S + 1 : n_cached, new_from);
    const int special_from = lo_tok / kPage;
    auto page_of = [&](int j) { return begin + wi + WP * j; };

    // Token t >= new_from is this call's append: read it from k_new / v_new.
    auto load_page = [&](int j, PageRegs<D>& pr, bool special) {
        const int pg = page_of(j);
        const uint16_t* kb = p.k_pool + int64_t(pr.kid) * p.page_elems;
        const uint16_t* vb = p.v_pool + int64_t(pr.vid) * p.page_elems;
        if (!special) {
            // buffer loads: scalar page base in the resource (whose size bounds
            // every lane offset), 32-bit lane offset, row offset as immediate
            // (K) or scalar offset (V); cache policy nt (2): every byte is read
            // once per step, so the pages stream past L2 instead of evicting
            // the page ids and partials (measured 13.33 -> 12.87 us at 8K keys,
            // 30.2 -> 29.8 us per layer at 32K)
            const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kb), 0, page_bytes, kBufferFlags);
            const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vb), 0, page_bytes, kBufferFlags);
#pragma unroll
            for (int c = 0; c < KS; ++c)
                pr.k[c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, kcol_b + 64 * c, 0, kNonTemporal));
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int hh = 0; hh < VH; ++hh)
                    pr.v[i][hh] = __builtin_bit_cast(
                        uint4, __builtin_amdgcn_raw_buffer_load_b128(rv, vcol_b + 256 * hh, i * kv_row_b, kNonTemporal));
            return;
        }
        const uint16_t* kr = kb + kcol;
        if (fused) {
            const int tk = pg * kPage + n16;
            if (tk >= new_from && tk < n_cached)
                kr = p.k_new + h * p.new_head_stride + int64_t(tk - new_from) * p.new_tok_stride + 8 * g;
        }
#pragma unroll
        for (int c = 0; c < KS; ++c) pr.k[c] = *reinterpret_cast<const uint4*>(kr + 32 * c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint16_t* src = vb + i * p.kv_row + vcol;
            if (fused) {
                const int tv = pg * kPage + 4 * g + i;
                if (tv >= new_from && tv < n_cached)
                    src = p.v_new + h * p.new_head_stride + int64_t(tv - new_from) * p.new_tok_stride + 8 * n16;
            }
#pragma unroll
            for (int hh = 0; hh < VH; ++hh) pr.v[i][hh] = *reinterpret_cast<const uint4*>(src + 128 * hh);
        }
    };
    // ... and write the appended rows into their page slots (bit-exact copies)
    auto store_new = [&](int j, const PageRegs<D>& pr) {
        const int pg = page_of(j);
        if (pg * kPage + kPage <= new_from) return;  // wave-uniform: no new token in this page
        uint16_t* kb = p.k_pool_w + int64_t(pr.kid) * p.page_elems;
        uint16_t* vb = p.v_pool_w + int64_t(pr.vid) * p.page_elems;
        const int tk = pg * kPage + n16;
        if (tk >= new_from && tk < n_cached) {
#pragma unroll
            for (int c = 0; c < KS; ++c) *reinterpret_cast<uint4*>(kb + kcol + 32 * c) = pr.k[c];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tv = pg * kPage + 4 * g + i;
            if (tv >= new_from && tv < n_cached)
#pragma unroll
                for (int hh = 0; hh < VH; ++hh) *reinterpret_cast<uint4*>(vb + i * p.kv_row + vcol + 128 * hh) = pr.v[i][hh];
        }
    };

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4_t acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // Keys from chunk_from on are the query chunk's own (S > 1, causal): some
    // rows may not see them.  Every row of the kv head multiplies every key of
    // the page in the P.V MFMA, with a zero probability where it may not see
    // it, and 0 x NaN is NaN: a NaN or infinite V row of such a key would reach
    // rows the reference never lets it reach.  A page holding one leaves those
    // keys out of the MFMA and adds them per row, over the rows that see them.
    const int chunk_from = p.causal && S > 1 ? n_cached - S + 1 : n_cached;
    auto compute_page = [&](int j, const PageRegs<D>& pr, bool special) {
        const int tok0 = page_of(j) * kPage + 4 * g;  // this lane's 4 keys: tok0 .. tok0+3
        bool split_v = false;  // wave-uniform
        if (special && chunk_from < n_cached) {
            bool bad = false;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int hh = 0; hh < VH; ++hh) {
                    const uint4 u = pr.v[i][hh];
                    const bool nf = E::nonfinite2(u.x) | E::nonfinite2(u.y) | E::nonfinite2(u.z) | E::nonfinite2(u.w);
                    bad |= nf && tok0 + i >= chunk_from && tok0 + i < n_cached;
                }
            split_v = __any(bad);
        }
        // V^T into LDS first (its latency hides behind the S^T MFMAs)
#pragma unroll
        for (int hh = 0; hh < VH; ++hh) {
            uint4 v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = pr.v[i][hh];
                // unfilled slots, and the chunk's keys when they are added per row
                if (special && (tok0 + i >= n_cached || (split_v && tok0 + i >= chunk_from))) v[i] = make_uint4(0, 0, 0, 0);
            }
            const uint32_t w[4][4] = {{v[0].x, v[0].y, v[0].z, v[0].w}, {v[1].x, v[1].y, v[1].z, v[1].w},
                                      {v[2].x, v[2].y, v[2].z, v[2].w}, {v[3].x, v[3].y, v[3].z, v[3].w}};
            const int d0 = 128 * hh + 8 * n16;
#pragma unroll
            for (int e = 0; e < 4; ++e) {  // dims d0 + 2e (low halves) and + 2e + 1 (high halves)
                const uint2 lo = make_uint2(__builtin_amdgcn_perm(w[1][e], w[0][e], 0x05040100u),
                                            __builtin_amdgcn_perm(w[3][e], w[2][e], 0x05040100u));
                const uint2 hi = make_uint2(__builtin_amdgcn_perm(w[1][e], w[0][e], 0x07060302u),
                                            __builtin_amdgcn_perm(w[3][e], w[2][e], 0x07060302u));
                *reinterpret_cast<uint2*>(&vt[(d0 + 2 * e) * VT_ROW + 4 * g]) = lo;
                *reinterpret_cast<uint2*>(&vt[(d0 + 2 * e + 1) * VT_ROW + 4 * g]) = hi;
            }
        }
        // S^T = K Q^T
        f32x4_t s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < KS; ++c) s = E::mma32(pr.k[c], qb[c], s);
        // Rows past rows_total have q = 0 (score 0) and are never written out.
        float x[4], lmx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = tok0 + i;
            x[i] = (!special || (t < n_cached && t <= qabs)) ? s[i] * p.scale_log2 : -INFINITY;
            lmx = fmaxf(lmx, x[i]);
        }
        // Lazy rescale: the row's reference max m_run only moves (and o, l are
        // rescaled) when the page max exceeds it by more than 2^8, so p <= 256.
        // A lane's own 4 keys decide whether any row may grow; the row max
        // (two cross-lane steps) is formed only then.
        if (__any(lmx > m_run + 8.0f)) {
            float mx = fmaxf(lmx, __shfl_xor(lmx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const bool grow = mx > m_run + 8.0f;
            const float mn = grow ? mx : m_run;
            const float alpha = grow ? exp2_fast(m_run - mn) : 1.0f;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db) acc[db] *= alpha;
            m_run = mn;
        }
        const float mu = m_run == -INFINITY ? 0.0f : m_run;
        float pw[4], sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pw[i] = exp2_fast(x[i] - mu);
            sum += pw[i];
        }
        l_run += sum;
        const uint2 pb = make_uint2(pack_p<F16>(pw[0], pw[1]), pack_p<F16>(pw[2], pw[3]));
        __builtin_amdgcn_wave_barrier();
        // O^T += V^T P^T
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const uint2 a = *reinterpret_cast<const uint2*>(&vt[(16 * db + n16) * VT_ROW + 4 * g]);
            acc[db] = E::mma16(a, pb, acc[db]);
        }
        __builtin_amdgcn_wave_barrier();
        if (split_v) {
            // the chunk's keys of this page, per row: lane (row n16, g) adds key t
            // to its dims 16 db + 4g .. + 3 when the row sees t
            const int pg0 = page_of(j) * kPage;
            const int t_hi = min(pg0 + kPage, n_cached);
            for (int t = max(pg0, chunk_from); t < t_hi; ++t) {
                const int kk = t - pg0, ki = kk & 3;
                const float sel = ki == 0 ? pw[0] : ki == 1 ? pw[1] : ki == 2 ? pw[2] : pw[3];
                const float pk = __shfl(sel, n16 + 16 * (kk >> 2));  // P[row][t]
                const uint16_t* vrow = fused && t >= new_from
                                           ? p.v_new + h * p.new_head_stride + int64_t(t - new_from) * p.new_tok_stride
                                           : p.v_pool + int64_t(pr.vid) * p.page_elems + int64_t(kk) * p.kv_row + h * D;
                if (t > qabs) continue;  // per lane: this row does not see t
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    const uint2 u = *reinterpret_cast<const uint2*>(vrow + 16 * db + 4 * g);
                    acc[db][0] = __builtin_fmaf(pk, E::lo(u.x), acc[db][0]);
                    acc[db][1] = __builtin_fmaf(pk, E::hi(u.x), acc[db][1]);
                    acc[db][2] = __builtin_fmaf(pk, E::lo(u.y), acc[db][2]);
                    acc[db][3] = __builtin_fmaf(pk, E::hi(u.y), acc[db][3]);
                }
            }
        }
    };

    // pages are loaded in increasing j, each once: the wave moves to id block
    // j / 64 when it first loads a page of it
    auto load_any = [&](int j, PageRegs<D>& pr) {
        if (j > 0 && (j & 63) == 0) {  // wave-uniform
            my_kid = nx_kid;
            my_vid = nx_vid;
            if (j + 64 < np_plan) fetch_ids(j / 64 + 1, nx_kid, nx_vid);
        }
        pr.kid = __builtin_amdgcn_readlane(my_kid, j & 63);
        pr.vid = __builtin_amdgcn_readlane(my_vid, j & 63);
        if (page_of(j) >= special_from)
            load_page(j, pr, true);
        else
            load_page(j, pr, false);
    };
    if constexpr (PF == 1) {
        // One page in flight: page j + 1 is requested as soon as page j has
        // landed, before page j's math, so the math runs under the next
        // page's round trip while the memory queues stay as deep as with one
        // request at a time (A/B on one box: config 3 kernel pair 12.70
        // against 12.76-12.80 us, config 5 29.45-29.59 against 29.79-29.92
        // us per layer).
        PageRegs<D> buf[2];
        if (np > 0) load_any(0, buf[0]);
        for (int j0 = 0; j0 < np; j0 += 2) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int j = j0 + u;
                if (j < np) {
                    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // page j landed
                    if (j + 1 < np) load_any(j + 1, buf[u ^ 1]);
                    if (page_of(j) >= special_from) {  // wave-uniform
                        if (fused) store_new(j, buf[u]);
                        compute_page(j, buf[u], true);
                    } else {
                        compute_page(j, buf[u], false);
                    }
                }
            }
        }
    } else {
        PageRegs<D> buf[PF];
    #pragma unroll
        for (int u = 0; u < PF - 1; ++u)
            if (u < np) load_any(u, buf[u]);
        for (int j0 = 0; j0 < np; j0 += PF) {
    #pragma unroll
            for (int u = 0; u < PF; ++u) {
                const int j = j0 + u;
                if (j < np) {
                    if (j + PF - 1 < np) load_any(j + PF - 1, buf[(u + PF - 1) % PF]);
                    if (page_of(j) >= special_from) {  // wave-uniform
                        if (fused) store_new(j, buf[u]);
                        compute_page(j, buf[u], true);
                    } else {
                        compute_page(j, buf[u], false);
                    }
                }
            }
        }
    }

    // l over the 4 lane groups of the row; o is already complete per lane
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (g == 0) {
        lds_m[wv][n16] = m_run;
        lds_l[wv][n16] = l_run;
    }
    if (n16 < rows_total) {  // rows past rows_total are never written out
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) lds_o[wv][n16][16 * db + 4 * g + i] = acc[db][i];
    }
    __syncthreads();

    // workgroup merge of each head's waves: wave -> (head, row) pairs wv,
    // wv + W, ...; lane -> dims d2, d2+1 of each 128-dim half
    for (int idx = wv; idx < HPW * rows_total; idx += W) {
        const int mh = HPW == 1 ? 0 : idx / rows_total, ri = idx - mh * rows_total;
        const int h = int(blockIdx.x) * HPW + mh, w0 = WP * mh;  // the pair's kv head, its first wave
        float M = -INFINITY;
#pragma unroll
        for (int w2 = w0; w2 < w0 + WP; ++w2) M = fmaxf(M, lds_m[w2][ri]);
        float L = 0.0f, O0[VH], O1[VH];
#pragma unroll
        for (int hh = 0; hh < VH; ++hh) O0[hh] = O1[hh] = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int w2 = w0; w2 < w0 + WP; ++w2) {
                const float e = exp2_fast(lds_m[w2][ri] - M);
                L += lds_l[w2][ri] * e;
#pragma unroll
                for (int hh = 0; hh < VH; ++hh) {
                    O0[hh] += lds_o[w2][ri][128 * hh + 2 * lane] * e;
                    O1[hh] += lds_o[w2][ri][128 * hh + 2 * lane + 1] * e;
                }
            }
        }
        if (p.n_splits == 1) {
            uint16_t* orow = p.out + int64_t(h * p.G + ri % p.G) * p.o_head_stride + int64_t(ri / p.G) * p.o_tok_stride;
            const float inv = 1.0f / L;
#pragma unroll
            for (int hh = 0; hh < VH; ++hh)
                *reinterpret_cast<uint32_t*>(orow + 128 * hh + 2 * lane) =
                    pack2(E::out(O0[hh] * inv), E::out(O1[hh] * inv));
        } else {
            // partials: o [h][split][row][D], then {m, l} [h][split][row],
            // stored agent-coherent (sc1: the store completes at the device's
            // coherence point, not in this XCD's L2).  The in-kernel merge then
            // needs no cache write-back before the arrival count below; before
            // the merge kernel, the kernel end has no dirty partial lines to
            // write back (Qwen3.5 decode 12.04 against 12.28 us with plain
            // stores, config 3 the same; nt stores 12.71 us; A/B on one box)
            const int64_t o_off = ((int64_t(h) * p.n_splits + sp) * rows_total + ri) * D;
            const int64_t ml_off = int64_t(p.Hkv) * p.n_splits * rows_total * D +
                                   2 * ((int64_t(h) * p.n_splits + sp) * rows_total + ri);
            const auto rs = part_rsrc<D>(p);
            auto store = [&](float2 v, int64_t at) {  // at: float index
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u32, v), rs, int(4 * at), 0, kCoherent);
            };
#pragma unroll
            for (int hh = 0; hh < VH; ++hh) store(make_float2(O0[hh], O1[hh]), o_off + 128 * hh + 2 * lane);
            if (lane == 0) store(make_float2(M, L), ml_off);
        }
    }
    if constexpr (kStep) {
        // Without a merge kernel (one split, or the single-launch merge) the
        // last workgroup to arrive advances the position: every workgroup
        // read it before it counts here.  The kernel boundary publishes the
        // position and the re-armed counter to the next launch.  With a merge
        // kernel, that kernel advances it.
        if (threadIdx.x == 0 && (p.n_splits == 1 || p.counters)) {
            const int total = int(gridDim.x * gridDim.y);
            const int old =
                __hip_atomic_fetch_add(p.step + kStepArrivals, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (old == total - 1) {
                __hip_atomic_store(p.step + kStepArrivals, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(p.step + kStepPos, step_pos + p.S, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if constexpr (HPW == 1) {
        if (p.counters && p.n_splits > 1) merge_last_arrival<D, W, F16>(p, h, lds_m, lds_l, lds_o);
    }
}

// Merge of the splits: one workgroup of MW waves per (kv head, row, 64-dim
// block), grid (Hkv, rows, D / 64) in the split grid's XCD order.  Wave w
// reduces the splits w, w+MW, ... to its own log-sum-exp partial (M_w, L_w,
// O_w): each lane loads the o of its dim and, as a broadcast, the (m, l) of
// each of those splits, up to kMergeU splits before any arithmetic (one memory
// round trip for up to MW * kMergeU splits); the MW partials then meet in LDS
// with the same rule
//   M = max M_w, L = sum L_w 2^(M_w - M), O = sum O_w 2^(M_w - M), out = O / L.
// MW is 4, or 8 above 4 * kMergeU splits (measured: 8 waves cost about 0.4 us
// at 31-32 splits and save 0.6 us at 103; 2 waves at 31 splits cost 0.3 us).  Blocks of 64 dims rather than one
// workgroup per row (D dims) spread a row's partials over D / 64 CUs; on one
// box, 128-dim blocks against 64: Qwen3.5 (D = 256, 103 splits) 12.8 -> 12.3
// us per decode, config 3 13.1 -> 12.9 us (whole rows measured 14.2 us on the
// Qwen3.5 shape, on a box where config 3 took 13.6).
//
// The arguments are scalars (14 dwords), not the parameter block, so that they
// can be preloaded into SGPRs at wave launch: the partial loads then need no
// argument read before them.  ml_off: float index of {m, l} in the partials.
template <int D, int MW, bool F16>
__global__ __launch_bounds__(MW * 64) void paged_decode_merge_kernel(const float* partial, uint16_t* out,
                                                                     int64_t o_head_stride, int64_t o_tok_stride,
                                                                     int32_t n_splits, int32_t G, int32_t S,
                                                                     int32_t ml_off, int32_t* step) {
    constexpr int U = kMergeU;  // splits in flight per lane
    constexpr int PL = 1;       // dims per lane (the workgroup's kMergeDims dims)
    static_assert(kMergeDims == 64 * PL, "merge: one lane per dim group");
    __shared__ float s_o[MW][kMergeDims];
    __shared__ float s_m[MW], s_l[MW];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int h = blockIdx.x, ri = blockIdx.y, d0 = kMergeDims * int(blockIdx.z);
    if (step) {
        // device-position step refused by the split kernel: no partials to merge
        if (step_load(step + kStepError)) return;
        // every split workgroup has read the position (they ran before this
        // launch): advance it for the next step, without waiting for the result
        if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0)
            __hip_atomic_fetch_add(step + kStepPos, S, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int rows = G * S;
    const int ns = n_splits;  // <= kMaxSplits
    const float2* ml = reinterpret_cast<const float2*>(partial + ml_off) + int64_t(h) * ns * rows + ri;
    const float* po = partial + (int64_t(h) * ns * rows + ri) * D + d0 + PL * lane;
    const int64_t sstride = int64_t(rows) * D;  // floats between splits
    static_assert(PL == 1, "merge: one dim per lane");
    auto load_o = [&](int s2, float (&o)[PL]) { o[0] = po[s2 * sstride]; };

    float mw = -INFINITY, lw = 0.0f, ow[PL];
#pragma unroll
    for (int e = 0; e < PL; ++e) ow[e] = 0.0f;
    for (int s0 = wv; s0 < ns; s0 += MW * U) {
        float ov[U][PL];
        float2 mv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s2 = s0 + MW * u;
            if (s2 < ns) {
                load_o(s2, ov[u]);
                mv[u] = ml[s2 * rows];
            } else {
#pragma unroll
                for (int e = 0; e < PL; ++e) ov[u][e] = 0.0f;
                mv[u] = make_float2(-INFINITY, 0.0f);
            }
        }
        float bm = mw;
#pragma unroll
        for (int u = 0; u < U; ++u) bm = fmaxf(bm, mv[u].x);
        if (bm == -INFINITY) continue;  // nothing visible yet
        const float a = mw == -INFINITY ? 0.0f : exp2_fast(mw - bm);
        lw *= a;
#pragma unroll
        for (int e = 0; e < PL; ++e) ow[e] *= a;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float w = mv[u].x == -INFINITY ? 0.0f : exp2_fast(mv[u].x - bm);
            lw += mv[u].y * w;
#pragma unroll
            for (int e = 0; e < PL; ++e) ow[e] += ov[u][e] * w;
        }
        mw = bm;
    }
#pragma unroll
    for (int e = 0; e < PL; ++e) s_o[wv][PL * lane + e] = ow[e];
    if (lane == 0) {
        s_m[wv] = mw;
        s_l[wv] = lw;
    }
    __syncthreads();
    if (wv == 0) {
        float M = -INFINITY;
#pragma unroll
        for (int w2 = 0; w2 < MW; ++w2) M = fmaxf(M, s_m[w2]);
        float L = 0.0f, O[PL];
#pragma unroll
        for (int e = 0; e < PL; ++e) O[e] = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < MW; ++w2) {
            const float f = s_m[w2] == -INFINITY ? 0.0f : exp2_fast(s_m[w2] - M);
            L += s_l[w2] * f;
#pragma unroll
            for (int e = 0; e < PL; ++e) O[e] += s_o[w2][PL * lane + e] * f;
        }
        const float inv = 1.0f / L;
        uint16_t* orow = out + int64_t(h * G + ri % G) * o_head_stride + int64_t(ri / G) * o_tok_stride + d0 + PL * lane;
        *orow = uint16_t(Elem<F16>::out(O[0] * inv));
    }
}

}  // namespace

size_t decode_workspace_bytes(int Hq, int Hkv, int S, int D, int n_pages) {
    if (Hkv <= 0 || Hq <= 0 || S <= 0 || D <= 0 || n_pages <= 0) return 0;
    const size_t rows = size_t(Hq / Hkv) * S;
    const size_t splits = std::min<size_t>(size_t(n_pages), kMaxSplits);
    return kDecodeCounterBytes + size_t(Hkv) * splits * rows * (D + 2) * sizeof(float);
}

// Decode settings, process-wide: initialised once from the environment
// (GENLLM_DECODE_PPS, GENLLM_DECODE_WG_PER_CU, GENLLM_DECODE_MERGE = kernel |
// fused) and changed only through genllm_decode_tuning, so a decode call
// reads no environment.  The split merge runs in a second kernel (default)
// or, fused, in the split kernel: the last split workgroup of each kv head to
// finish merges it.  Measured at config 3 (MI355X, 400 back-to-back launches
// over 16 rotating layers): two kernels 12.7 us per decode (split 10.3 us +
// merge 3.7 us in the kernel trace), single launch 14.6 us: the last
// workgroup's serial tail -- coherent stores completing, the arrival count,
// then coherent loads of every partial -- costs more than the second launch.
namespace {
struct DecodeSettings {
    std::atomic<int> pps{0};          // > 0: forced pages per split
    std::atomic<double> wg_per_cu{1.0};
    std::atomic<int> merge{kDecodeMergeKernel};
    std::atomic<int> heads{0};        // kv heads per split workgroup: 0 automatic, 1 or kMultiHead forced
    DecodeSettings() {
        if (const char* e = getenv("GENLLM_DECODE_PPS")) pps = atoi(e);
        if (const char* e = getenv("GENLLM_DECODE_HEADS")) heads = atoi(e);
        if (const char* e = getenv("GENLLM_DECODE_WG_PER_CU")) wg_per_cu = atof(e);
        if (const char* e = getenv("GENLLM_DECODE_MERGE")) {
            const std::string m(e);
            merge = m == "fused" ? kDecodeMergeFused : kDecodeMergeKernel;
        }
    }
};
DecodeSettings& decode_settings() {
    static DecodeSettings s;
    return s;
}
}  // namespace

int set_decode_tuning(int pages_per_split, int merge, int heads_per_wg) {
    if (merge != kDecodeMergeKernel && merge != kDecodeMergeFused)
        return fail(GENLLM_ERR_INVALID, "decode tuning: merge must be 0 (merge kernel) or 1 (fused)");
    if (heads_per_wg != 0 && heads_per_wg != 1 && heads_per_wg != kMultiHead)
        return fail(GENLLM_ERR_INVALID, "decode tuning: heads per workgroup must be 0 (automatic), 1 or 4");
    decode_settings().pps = std::max(pages_per_split, 0);
    decode_settings().merge = merge;
    decode_settings().heads = heads_per_wg;
    return GENLLM_OK;
}

// Pages per split: about wg_per_cu (default 1) workgroups per CU over all kv
// heads, at most 256 splits (a forced value, genllm_decode_tuning, wins).
// Heads per workgroup: kMultiHead where the one-head plan reaches
// kMultiHeadMinPps pages per split (or where forced), for head_dim 128, kv
// heads in groups of 4 and the merge kernel; else 1.
int decode_plan(AttnParams& p, int D, size_t ws_bytes, void* ws) {
    if (p.G * p.S > kRows) return fail(GENLLM_ERR_INVALID, "paged decode: seq_len * groups must be <= 16");
    DecodeSettings& cfg = decode_settings();
    p.heads_per_wg = 1;
    int pps = cfg.pps.load(std::memory_order_relaxed);
    const int heads = cfg.heads.load(std::memory_order_relaxed);
    const int cus = device_cu_count();
    const bool multi_ok =
        D == 128 && p.Hkv % kMultiHead == 0 && cfg.merge.load(std::memory_order_relaxed) == kDecodeMergeKernel;
    if (pps <= 0) {
        const int64_t target = std::max<int64_t>(1, int64_t(cfg.wg_per_cu.load(std::memory_order_relaxed) * cus));
        pps = int((int64_t(p.n_pages) * p.Hkv + target - 1) / target);
        if (pps < 2) pps = 2;
        // long ranges: kMultiHead kv heads per workgroup, the same workgroup count
        if (multi_ok && (heads == kMultiHead || (heads == 0 && pps >= kMultiHeadMinPps))) {
            p.heads_per_wg = kMultiHead;
            pps = std::max(2, int((int64_t(p.n_pages) * (p.Hkv / kMultiHead) + target - 1) / target));
        }
    } else if (multi_ok && heads == kMultiHead) {
        p.heads_per_wg = kMultiHead;
    }
    pps = std::max(pps, (p.n_pages + kMaxSplits - 1) / kMaxSplits);
    p.pages_per_split = pps;
    p.n_splits = (p.n_pages + pps - 1) / pps;
    p.partial = nullptr;
    p.counters = nullptr;
    if (p.n_splits > 1) {
        if (p.Hkv > kDecodeMaxKvHeads)
            return fail(GENLLM_ERR_UNSUPPORTED, "paged decode: at most 256 kv heads");
        const size_t need =
            kDecodeCounterBytes + size_t(p.Hkv) * p.n_splits * (p.G * p.S) * (D + 2) * sizeof(float);
        if (!ws || ws_bytes < need)
            return fail(GENLLM_ERR_INVALID, "paged decode: workspace too small (need " + std::to_string(need) +
                                                " bytes, have " + std::to_string(ws_bytes) + ")");
        p.partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kDecodeCounterBytes);
        if (cfg.merge.load(std::memory_order_relaxed) == kDecodeMergeFused) p.counters = static_cast<int32_t*>(ws);
    }
    return GENLLM_OK;
}

template <int D, bool kStep, bool F16>
void launch_split(const AttnParams& p, hipStream_t stream) {
    auto* k = paged_decode_kernel<D, kWaves, kStep, F16, 1>;
    int w = kWaves, hpw = 1;
    if constexpr (D == 128) {
        if (p.heads_per_wg == kMultiHead) {
            k = paged_decode_kernel<D, kWideWaves, kStep, F16, kMultiHead>;
            w = kWideWaves;
            hpw = kMultiHead;
        } else if (p.pages_per_split <= kWideMaxPps) {
            k = paged_decode_kernel<D, kWideWaves, kStep, F16, 1>;
            w = kWideWaves;
        }
    }
    hipLaunchKernelGGL(k, dim3(p.Hkv / hpw, p.n_splits), dim3(w * 64), 0, stream, p.k_ids, p.v_ids, p.q,
                       int32_t(p.q_head_stride), int32_t(p.q_tok_stride), p.G, p.S, p.pages_per_split, p.n_pages,
                       p.upd.first, p.upd.count, p);
}

template <int D, bool F16>
int launch_decode_d(const AttnParams& p, hipStream_t stream) {
    if (p.step)
        launch_split<D, true, F16>(p, stream);
    else
        launch_split<D, false, F16>(p, stream);
    GENLLM_LAUNCH_CHECK("paged_decode_kernel");
    if (p.n_splits > 1 && !p.counters) {
        const dim3 grid(p.Hkv, p.G * p.S, D / kMergeDims);
        const int32_t ml_off = p.Hkv * p.n_splits * p.G * p.S * D;  // < 2^31: the plan's workspace is far smaller
        auto* mk = p.n_splits > 4 * kMergeU ? paged_decode_merge_kernel<D, 8, F16> : paged_decode_merge_kernel<D, 4, F16>;
        const int mw = p.n_splits > 4 * kMergeU ? 8 : 4;
        hipLaunchKernelGGL(mk, grid, dim3(mw * 64), 0, stream, static_cast<const float*>(p.partial), p.out,
                           p.o_head_stride, p.o_tok_stride, p.n_splits, p.G, p.S, ml_off, p.step);
        GENLLM_LAUNCH_CHECK("paged_decode_merge_kernel");
    }
    return GENLLM_OK;
}

int launch_paged_decode(const AttnParams& p, int head_dim, hipStream_t stream) {
    if (head_dim != 128 && head_dim != 256) return fail(GENLLM_ERR_UNSUPPORTED, "paged decode: head_dim must be 128 or 256");
    if (p.n_pages <= 0) return GENLLM_OK;
    if (p.n_splits > kMaxSplits || p.pages_per_split <= 0 || p.G * p.S > kRows ||
        (p.heads_per_wg != 1 && (p.heads_per_wg != kMultiHead || head_dim != 128 || p.Hkv % kMultiHead || p.counters)))
        return fail(GENLLM_ERR_INVALID, "paged decode: split plan out of range");
    if (p.q_head_stride > INT32_MAX || p.q_tok_stride > INT32_MAX || p.q_head_stride < 0 || p.q_tok_stride < 0)
        return fail(GENLLM_ERR_INVALID, "paged decode: q strides must be below 2^31 elements");
    if (p.f16) return head_dim == 128 ? launch_decode_d<128, true>(p, stream) : launch_decode_d<256, true>(p, stream);
    return head_dim == 128 ? launch_decode_d<128, false>(p, stream) : launch_decode_d<256, false>(p, stream);
}

}  // namespace genllm
