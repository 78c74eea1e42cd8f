// paged_prefill.hip -- causal paged FlashAttention on bf16 MFMA (gfx950).
//
// Same result as the attention loop of PagedAttentionImpl<CPU>::execute
// (src/backend/cpu/attention.cpp:148-215) for a chunk of S queries: query s sits
// at q_abs = n_cached - S + s and attends keys 0..q_abs (causal, :164-181),
// kv head = q head / groups (:158).
//
// Grid: pairs of query tiles of 64 rows x Hq workgroups of 8 waves, one
// workgroup per CU; the workgroup of pair r runs query tile n_qt-1-r, then
// query tile r, so that under causal masking every workgroup carries the same
// number of key tiles (the dispatcher hands workgroups out in grid order, not
// by work).  A query tile's queries form two groups of 32; each group is
// served by four waves that split every key tile of 64 tokens (4 pages) by
// page: wave (qg, kq) takes keys 16kq..16kq+15 of each tile for the 32
// queries of group qg, and the four partial softmax states of a group are
// merged through LDS at the end.
// Key tiles are staged in four LDS buffers (three tiles in flight), K and V
// each as [token][dim] rows of 256 B whose 16-byte chunks are swizzled: chunk c
// of row r sits at position cperm(c) ^ swz(r % 16), with swz(r) = 2 (r % 8) +
// r / 8 and cperm swapping bits 1 and 3 of c.  The K operand reads (16 rows,
// one chunk each) cover 16 distinct positions; in a transposing V read the
// two 16-lane halves of a 32-lane group (dims 0-15 and 16-31 of a 32-dim
// block, chunk bit 1) land in different 128-byte halves of the rows (position
// bit 3), so the row XOR no longer folds them onto the same banks.  Wave (qg, kq) moves the K (qg 0) or V (qg 1) rows of page
// kq of every tile straight from HBM into LDS with 16-byte buffer loads in LDS
// mode (lane i's 16 bytes land at base + 16 i), so a tile costs no registers,
// no VALU and no LDS store instructions; one buffer resource per page (base =
// the page of this kv head, size = the bytes its rows below the key limit
// span) bounds every load.
// Per tile and wave:
//   S^T = K Q^T  (v_mfma_f32_16x16x32_bf16 x 8; A = K from LDS: lane l ->
//        key l%16, dims 32ks+8(l/16)..; B = Q^T held in registers).
//        D[key][q] lands in lane q%16 + 16*(key/4), register key%4: every
//        lane holds 4 keys of ONE query row per 16-query block, so the online
//        softmax state (m, l) of a row is per lane.
//   O^T += V^T P^T  (v_mfma_f32_32x32x16_bf16 x 4, the full-rate form for 16
//        keys -- the 16x16x16 form runs at half the bf16 rate on gfx950;
//        B = P^T from the lane's own exponentials, regrouped by one
//        v_permlane16_swap per dword; A = V^T from two ds_read_b64_tr_b16 per
//        32 dims).  O^T[dim][q] belongs to the lane's own query column, so
//        the rescale by 2^(m_old-m_new) stays lane-local.
// Causal masking is applied only to the pages that reach past the first
// query of the wave (the diagonal) or past the cache end.
#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

namespace {

constexpr int KT = 64;          // keys per tile (4 pages)
constexpr int QW = 32;          // queries per wave (one 32-column block of O^T)
constexpr int QT = 2 * QW;      // queries per query tile: two query groups
constexpr int KQ = KT / 4;      // keys of a tile per wave: one page
constexpr int WAVES = 8;        // query group (2) x key quarter (4)
constexpr int NBUF = 4;         // LDS tile buffers: three tiles in flight
constexpr int IDS_BLOCK = 64;   // tiles whose page ids one vector load brings

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) float lds_float;

// two fp32 -> packed bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t bf16_pair_rne(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// chunk-position swizzle of a 256-byte LDS row: bijective on r % 16, and
// 2 (r % 8) separates the 32-byte chunk pairs of eight consecutive rows
__device__ __forceinline__ constexpr int swz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }
// chunk-index bit swap (1 <-> 3) applied before the row XOR (an involution)
__device__ __forceinline__ constexpr int cperm(int c) { return (c & 5) | ((c & 2) << 2) | ((c & 8) >> 2); }

__device__ __forceinline__ s16x4_t ds_read_tr(const lds_char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<__attribute__((address_space(3))) s16x4_t*>(const_cast<lds_char*>(p)));
}

// v_mfma_f32_32x32x16_bf16: lane l gives A[l%32][8(l/32)..+7] and
// B[8(l/32)..+7][l%32]; D[8(r/4) + 4(l/32) + r%4][l%32] comes back in register r.
__device__ __forceinline__ f32x16_t mfma32x32x16(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Two fp32 -> packed bf16 for an output, bfloat16_t's constructor
// (bfloat16.hpp:18-41) for every input: round to nearest even, an fp32
// subnormal becomes a signed zero, a NaN becomes sign | 0x7F81 (the
// constructor keeps only "mantissa != 0") -- v_cvt_pk_bf16_f32 plus selects
// instead of the integer form's branches.
__device__ __forceinline__ uint32_t bf16_pair_out(float lo, float hi) {
    const uint32_t nan_lo = ((__float_as_uint(lo) >> 16) & 0x8000u) | 0x7F81u;
    const uint32_t nan_hi = (__float_as_uint(hi) & 0x80000000u) | 0x7F810000u;
    const bool lo_nan = lo != lo, hi_nan = hi != hi;
    lo = fabsf(lo) < __FLT_MIN__ ? __builtin_copysignf(0.0f, lo) : lo;
    hi = fabsf(hi) < __FLT_MIN__ ? __builtin_copysignf(0.0f, hi) : hi;
    uint32_t r = bf16_pair_rne(lo, hi);
    r = lo_nan ? (r & 0xFFFF0000u) | nan_lo : r;
    return hi_nan ? (r & 0xFFFFu) | nan_hi : r;
}

// s_waitcnt operand: vmcnt(n) for n < 16, other counters unconstrained
constexpr int wait_vmcnt(int n) { return (kWaitVmcnt0 & ~0xF) | n; }

// Workgroup barrier for the tile pipeline.  A release fence here would wait
// for every LDS-mode load still in flight (they write LDS); the tiles are
// instead waited for explicitly, by count, before it.  The LDS reads before
// it have all been consumed (their results feed the MFMAs), and the empty
// asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void tile_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

template <int D>
__global__ __launch_bounds__(WAVES * 64) void paged_prefill_kernel(AttnParams p) {
    static_assert(D == 128, "prefill kernel: head_dim 128");
    constexpr int KS = D / 32;          // k-steps of the S^T product
    constexpr int DJ = D / 32;          // 32-dim blocks of O^T
    constexpr int ROWB = D * 2;         // bytes per token row (16 chunks of 16 B)
    constexpr int TILEB = KT * ROWB;    // bytes of a K (or V) tile
    constexpr int PAGEB = kPage * ROWB; // bytes of one page's rows of a tile
    static_assert(ROWB == 16 * 16, "16 chunks per row: the swizzle acts on r % 16");
    constexpr int XCH = DJ * 16 + 4;    // floats per lane handed over at the end: O^T, m, l
    static_assert(XCH * 64 * 4 <= 2 * TILEB, "a hand-over fits one buffer");

    // four buffers [K tile][V tile], separate arrays so that the compiler sees
    // the tiles being loaded and the tile being read as distinct memory
    __shared__ __attribute__((aligned(16))) char lds_b0[2 * TILEB];
    __shared__ __attribute__((aligned(16))) char lds_b1[2 * TILEB];
    __shared__ __attribute__((aligned(16))) char lds_b2[2 * TILEB];
    __shared__ __attribute__((aligned(16))) char lds_b3[2 * TILEB];
    lds_char* const buf0 = (lds_char*)lds_b0;
    lds_char* const buf1 = (lds_char*)lds_b1;
    lds_char* const buf2 = (lds_char*)lds_b2;
    lds_char* const buf3 = (lds_char*)lds_b3;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS bases go to scalar registers
    const int qg = wv >> 2, kq = wv & 3;                      // query group, key quarter
    const int n16 = lane & 15, g = lane >> 4;
    const int hb = g & 1;  // the lane's O^T column is query 16 hb + n16 of the group
    // Grid: query-tile pairs x Hq.  Pair r runs query tile n_qt-1-r, then
    // query tile r: under causal masking their key-tile counts add up to the
    // same total for every pair, so every workgroup carries the same work
    // whatever order the dispatcher hands them out in.
    const int n_qt = (p.S + QT - 1) / QT;
    const int pair = int(blockIdx.x) / p.Hq;
    const int hq = int(blockIdx.x) - pair * p.Hq;
    const int hkv = hq / p.G;
    const int qabs0 = p.n_cached - p.S;  // absolute position of query 0
    const int n_cached = p.n_cached;
    // The scale (>= 0, checked by the host) is raised to at least FLT_MIN, so
    // that a masked score of -inf gives exp2(-inf * c - m) = 0 without a
    // select; at scale 0 every weight stays exp2(~0) = 1.
    const float c = fmaxf(p.scale_log2, __FLT_MIN__);
    const float inv_c = 1.0f / c;  // may be inf (then no row grows after its first tile)

    // ---- tile staging.  Wave (qg, kq) moves page kq of every tile: its K
    // rows (qg 0) or its V rows (qg 1).
    const bool paged = p.k_ids != nullptr;
    const int32_t* const my_ids = qg == 0 ? p.k_ids : p.v_ids;
    const int64_t head_off = int64_t(hkv) * (p.kv_head_stride ? p.kv_head_stride : D);
    const uint16_t* const src = (qg == 0 ? p.k_pool : p.v_pool) + head_off;
    const int64_t kv_row = p.kv_row, page_elems = p.page_elems;
    const int kv_row_bytes = int(kv_row) * 2;
    // Lane byte offsets inside a page, the same for every tile: instruction e
    // fills rows 4e..4e+3, lane -> row 4e + lane/16 (rows start on page
    // boundaries, so row % 16 is that slot), position lane%16 <- chunk
    // cperm((lane%16) ^ swz(slot)).
    uint32_t dma_off[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int slot = 4 * e + (lane >> 4);
        dma_off[e] = uint32_t(slot * kv_row_bytes + 16 * cperm((lane & 15) ^ swz(slot)));
    }
    const int dst_wave = qg * TILEB + kq * PAGEB;

    const int qt_hi = n_qt - 1 - pair;
    const int n_pass = pair < qt_hi ? 2 : 1;  // the middle tile of an odd count runs alone
    for (int pass = 0; pass < n_pass; ++pass) {
        const int qt = pass == 0 ? qt_hi : pair;
        const int q0 = qt * QT + qg * QW;  // first query of this wave's group

        // Q^T operands (B of S^T), block b: lane -> query q0 + 16b + n16, dims
        // 32ks + 8g..+7.  Loads are unconditional (row clamped), zeroed after.
        bf16x8_t qb[2][KS];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int s = q0 + 16 * b + n16;
            const bool ok = s < p.S;
            const uint16_t* qrow = p.q + int64_t(hq) * p.q_head_stride + int64_t(ok ? s : p.S - 1) * p.q_tok_stride;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                uint4 u = *reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * g);
                if (!ok) u = make_uint4(0, 0, 0, 0);
                qb[b][ks] = as_bf16x8(u);
            }
        }

        // softmax state of query 16b + n16 (per lane, equal over the lane's
        // 16-lane row group for m), O^T columns of query 16 hb + n16
        float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
        // kept beside m: nm = -m (0 while m = -inf), and th = the raw score
        // above which the scaled score exceeds m + 8 (-inf while m = -inf)
        float nm[2] = {0.0f, 0.0f}, th[2] = {-INFINITY, -INFINITY};
        f32x16_t acc[DJ];
#pragma unroll
        for (int j = 0; j < DJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;

        const int wg_last = min(qt * QT + QT, p.S) - 1;
        const int kv_end = p.causal ? min(qabs0 + wg_last + 1, n_cached) : n_cached;
        const int n_tiles = (kv_end + KT - 1) / KT;
        const bool wave_has_rows = q0 < p.S;
        // keys below wave_lim are visible to every query of the wave, keys at or
        // past wave_end to none of them
        const int wave_lim = p.causal ? min(qabs0 + q0 + 1, n_cached) : n_cached;
        const int wave_end = !wave_has_rows ? 0 : p.causal ? min(qabs0 + min(q0 + QW, p.S), n_cached) : n_cached;

        // lane i <- the id of this wave's page of tile t0 + i
        auto load_ids = [&](int t0) -> int {
            const int page = 4 * (t0 + lane) + kq;
            return page * kPage < kv_end ? my_ids[page] : 0;
        };
        // The buffer resource of a page spans exactly its rows below kv_end
        // (paged: the page of id k starts at k * page_elems; head-major tensor:
        // the "page" starts at its first token).  Rows at or past kv_end -- past
        // the causal limit, the cache end or the table -- come back as zeros:
        // their keys are masked and their zero values meet zero probabilities.
        auto issue_tile = [&](int t, int ids, lds_char* buf) {
            const int tok_page = t * KT + kPage * kq;
            const int valid = min(max(kv_end - tok_page, 0), kPage);
            const uint32_t span = uint32_t(__builtin_amdgcn_readfirstlane(valid > 0 ? (valid - 1) * kv_row_bytes + ROWB : 0));
            const int64_t base = paged ? int64_t(__builtin_amdgcn_readlane(ids, t & (IDS_BLOCK - 1))) * page_elems
                                       : int64_t(tok_page) * kv_row;
            const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)(src + base), 0, span, kBufferFlags);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(buf + (dst_wave + e * 1024)),
                                                         16, dma_off[e], 0, 0, 0);
        };

        // ---- this wave's 16 keys of one tile against its 32 queries (buf: K
        // at 0, V at TILEB).  masked: the keys reach past the first query of
        // the wave or past the cache end.
        auto compute_tile = [&](int t, const lds_char* buf, bool masked) {
            const int tok0 = t * KT + KQ * kq;  // first key of the quarter
            // S^T = K Q^T (v_mfma_f32_16x16x32_bf16; A = K from LDS: lane l ->
            // key l%16, dims 32ks + 8(l/16)..).  s[b][i] = key tok0 + 4g + i x
            // query q0 + 16b + n16.
            f32x4_t s[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
            const int krow = KQ * kq + n16;  // row % 16 == n16
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const u32x4_t a = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
                    buf + (krow * ROWB + ((cperm(4 * ks + g) ^ swz(n16)) * 16)));
#pragma unroll
                for (int b = 0; b < 2; ++b) s[b] = mfma16x16x32(__builtin_bit_cast(bf16x8_t, a), qb[b][ks], s[b]);
            }

            if (masked) {
                // wave-uniform; the empty asm keeps this a branch of its own
                // instead of selects on every tile.  A key is visible to a query
                // when kpos < lim (lim = n_cached, or q_abs + 1 when causal).
                __asm__ volatile("");
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const int qpos = qabs0 + q0 + 16 * b + n16;
                    const int lim = p.causal ? min(qpos + 1, n_cached) : n_cached;
                    const int rel = lim - tok0 - 4 * g;
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[b][i] = i < rel ? s[b][i] : -INFINITY;
                }
            }
            // Online softmax with a lazy rescale: a row's reference max only
            // moves (and its l, O^T are rescaled) when the tile max exceeds it
            // by about 2^8 (its raw max passes th), so p <= 256 or so; a
            // lane's own keys decide whether any row may grow, and the row max
            // (two cross-lane steps) is formed only then.
            float mx[2];
#pragma unroll
            for (int b = 0; b < 2; ++b)  // IEEE maximum (NaN-propagating): v_maximum3_f32, no quieting
                mx[b] = __builtin_elementwise_maximum(__builtin_elementwise_maximum(s[b][0], s[b][1]),
                                                      __builtin_elementwise_maximum(s[b][2], s[b][3]));
            if (__any(mx[0] > th[0] || mx[1] > th[1])) {
                float alpha[2];
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    float r = fmaxf(mx[b], __shfl_xor(mx[b], 16));
                    r = fmaxf(r, __shfl_xor(r, 32));
                    const bool grow = r > th[b];
                    const float mn = grow ? r * c : m[b];
                    alpha[b] = grow ? exp2_fast(m[b] - mn) : 1.0f;
                    l[b] *= alpha[b];
                    m[b] = mn;
                    nm[b] = grow ? -mn : nm[b];
                    th[b] = grow ? (mn + 8.0f) * inv_c : th[b];
                }
                const float as = hb ? alpha[1] : alpha[0];
#pragma unroll
                for (int j = 0; j < DJ; ++j) acc[j] *= as;
            }
            uint32_t pk[2][2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                float e[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) e[i] = exp2_fast(__builtin_fmaf(s[b][i], c, nm[b]));  // masked: exactly 0
                l[b] += (e[0] + e[1]) + (e[2] + e[3]);
                pk[b][0] = bf16_pair_rne(e[0], e[1]);
                pk[b][1] = bf16_pair_rne(e[2], e[3]);
            }
            // O^T += V^T P^T with v_mfma_f32_32x32x16_bf16 over the 16 keys.
            // B = P^T, lane l -> query 16 ((l/16) % 2) + n16, keys 8(l/32)..+7:
            // the lane holds keys 4g.. of queries n16 and 16 + n16, and one
            // v_permlane16_swap per dword (odd 16-lane rows of block 0 <-> even
            // rows of block 1) gathers them into that layout.
            const auto w0 = __builtin_amdgcn_permlane16_swap(pk[0][0], pk[1][0], false, false);
            const auto w1 = __builtin_amdgcn_permlane16_swap(pk[0][1], pk[1][1], false, false);
            const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, u32x4_t{w0[0], w1[0], w0[1], w1[1]});
            // A = V^T[32 dims][16 keys], lane l -> dim 16 ((l/16) % 2) + n16,
            // keys 8(l/32)..+7: two transposing reads, keys +0..3 and +4..7.  In
            // each 16-lane group, lane 4j'+q points at V[key0+j'][dim0+4q..+3]
            // (chunk dim/8, half q%2) and lane i receives V[key0+0..3][dim0+i].
            // The byte offset is formed as one integer added to the buffer: the
            // compiler attributes an LDS access to its array (and so can tell it
            // apart from the loads still streaming into the other buffers,
            // without waiting for them) only through a short chain of pointer
            // arithmetic.
            const int vrow0 = KQ * kq + 8 * (g >> 1) + (n16 >> 2), vrow1 = vrow0 + 4;
            const int vsw0 = swz(vrow0 & 15), vsw1 = swz(vrow1 & 15);
#pragma unroll
            for (int j = 0; j < DJ; ++j) {
                const int chunk = 4 * j + 2 * hb + ((n16 & 3) >> 1), half = (n16 & 1) * 8;
                const s16x4_t lo = ds_read_tr(buf + (TILEB + vrow0 * ROWB + ((cperm(chunk) ^ vsw0) * 16) + half));
                const s16x4_t hi = ds_read_tr(buf + (TILEB + vrow1 * ROWB + ((cperm(chunk) ^ vsw1) * 16) + half));
                const s16x4_t a8[2] = {lo, hi};
                acc[j] = mfma32x32x16(__builtin_bit_cast(bf16x8_t, a8), pb, acc[j]);
            }
        };

        // ---- pipeline: three tiles in flight, one barrier per tile.  Step t
        // waits for its own loads of tile t (the loads of tiles t+1 and t+2 may
        // still be in flight: every step issues exactly 4 loads per wave, so
        // the count is always 8), meets the other waves (tile t complete in
        // LDS; everybody done reading tile t-1), starts tile t+3 into the
        // buffer of tile t-1, then computes its quarter of tile t.  Tiles past
        // the last one have no rows below kv_end: their loads return zeros and
        // touch no memory.  Page ids arrive IDS_BLOCK tiles per load; the rare
        // reload drains the loads in flight.
        // the previous pass's hand-over has been read: LDS is free (the first
        // pass waits for nothing here, so its waves start their loads as they
        // launch: 42.1-42.5 against 42.8 us at config 4, A/B on one box)
        if (pass > 0) __syncthreads();
        int ids = 0;
        if (paged) ids = load_ids(0);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // q and ids landed
        issue_tile(0, ids, buf0);
        issue_tile(1, ids, buf1);
        issue_tile(2, ids, buf2);
        auto step = [&](int t, const lds_char* cur, lds_char* nxt) {
            __builtin_amdgcn_s_waitcnt(wait_vmcnt(8));
            tile_barrier();
            if (((t + 3) & (IDS_BLOCK - 1)) == 0 && t + 3 < n_tiles) {
                if (paged) ids = load_ids(t + 3);
                __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            }
            issue_tile(t + 3, ids, nxt);
            const int tok0 = t * KT + KQ * kq;
            if (t < n_tiles && tok0 < wave_end) compute_tile(t, cur, tok0 + KQ > wave_lim);
        };
        for (int t = 0; t < n_tiles; t += NBUF) {
            step(t, buf0, buf3);
            step(t + 1, buf1, buf0);
            step(t + 2, buf2, buf1);
            step(t + 3, buf3, buf2);
        }
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // the trailing (empty) loads have landed: LDS is free

        // ---- merge the four key quarters of each query group in two rounds:
        // quarter 1 into 0 and 3 into 2, then 2 into 0.  The sending wave
        // stores (O^T, m, l) as [value][lane] floats; the receiving wave
        // combines m = max(m0, m1), O = O0 2^(m0-m) + O1 2^(m1-m), l likewise
        // (a quarter that saw no key of a row has m = -inf, weight 0).
        auto lane_base = [&](lds_float* xch) {
            int off = lane;
            __asm__ volatile("" : "+v"(off));
            return xch + off;
        };
        auto send = [&](lds_float* slot) {
            lds_float* const xch = lane_base(slot);
#pragma unroll
            for (int j = 0; j < DJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) xch[(j * 16 + r) * 64] = acc[j][r];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                xch[(DJ * 16 + b) * 64] = m[b];
                xch[(DJ * 16 + 2 + b) * 64] = l[b];
            }
        };
        auto receive = [&](lds_float* slot) {
            const lds_float* const xch = lane_base(slot);
            float a0[2], a1[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const float m1 = xch[(DJ * 16 + b) * 64];
                const float l1 = xch[(DJ * 16 + 2 + b) * 64];
                const float mt = fmaxf(m[b], m1);
                a0[b] = mt == -INFINITY ? 0.0f : exp2_fast(m[b] - mt);
                a1[b] = mt == -INFINITY ? 0.0f : exp2_fast(m1 - mt);
                l[b] = l[b] * a0[b] + l1 * a1[b];
                m[b] = mt;
            }
            const float s0 = hb ? a0[1] : a0[0], s1 = hb ? a1[1] : a1[0];
#pragma unroll
            for (int j = 0; j < DJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[j][r] = acc[j][r] * s0 + xch[(j * 16 + r) * 64] * s1;
        };
        lds_float* const slot_a = (lds_float*)(qg == 0 ? buf0 : buf1);  // quarter 1 -> 0
        lds_float* const slot_b = (lds_float*)(qg == 0 ? buf2 : buf3);  // quarter 3 -> 2, then 2 -> 0
        __syncthreads();  // every wave is done with the tiles
        if (kq == 1) send(slot_a);
        if (kq == 3) send(slot_b);
        __syncthreads();
        if (kq == 0) receive(slot_a);
        if (kq == 2) {
            receive(slot_b);
            send(slot_b);  // the same wave read it: program order keeps the reads first
        }
        __syncthreads();
        if (kq == 0 && wave_has_rows) {
            receive(slot_b);
            float lt[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                lt[b] = l[b];
                lt[b] += __shfl_xor(lt[b], 16);
                lt[b] += __shfl_xor(lt[b], 32);
            }
            const float inv = 1.0f / (hb ? lt[1] : lt[0]);
            const int s = q0 + 16 * hb + n16;
            if (s < p.S) {
                // register r of block j: dim 32j + 8(r/4) + 4(g/2) + r%4
                uint16_t* orow = p.out + int64_t(hq) * p.o_head_stride + int64_t(s) * p.o_tok_stride + 4 * (g >> 1);
#pragma unroll
                for (int j = 0; j < DJ; ++j)
#pragma unroll
                    for (int rr = 0; rr < 4; ++rr) {
                        uint2 w;
                        w.x = bf16_pair_out(acc[j][4 * rr] * inv, acc[j][4 * rr + 1] * inv);
                        w.y = bf16_pair_out(acc[j][4 * rr + 2] * inv, acc[j][4 * rr + 3] * inv);
                        *reinterpret_cast<uint2*>(orow + 32 * j + 8 * rr) = w;
                    }
            }
        }
    }
}

// ---------------------------------------------------------------- D = 256
// Qwen3.5's head_dim (Qwen35.hpp:14-16).  A token row is 512 B (32 chunks of
// 16 B); both 256-byte halves carry the swizzle above (chunk c of row r at
// position 16 (c / 16) + ((c % 16) ^ swz(r % 16))).  Two query blocks per wave
// would need 128 accumulator registers here, so a wave owns one 16-query block
// and one half of every key tile.  Workgroup: 8 waves, query blocks 0..3 (64
// queries) x key halves 0..1 of key tiles of 64 tokens (4 pages), one
// workgroup per CU (two 64 KB tile buffers); the two halves of a query block
// are merged through LDS at the end.  Wave w moves the K (w even) or V (w odd)
// rows of page w / 2 of each tile; one tile is in flight while the other is
// computed.  The grid runs from the query tile with the most keys down.
constexpr int KT256 = 64;
constexpr int QW256 = 16;
constexpr int WAVES256 = 8;
constexpr int QT256 = 4 * QW256;

__global__ __launch_bounds__(WAVES256 * 64) void paged_prefill_d256_kernel(AttnParams p) {
    constexpr int D = 256;
    constexpr int KS = D / 32, DB = D / 16;
    constexpr int ROWB = D * 2;          // 512 bytes per token row
    constexpr int TILEB = KT256 * ROWB;  // 32 KB of K (or V) per tile
    constexpr int KH = KT256 / 2;        // keys of a tile per wave
    constexpr int XCH = DB * 4 + 2;      // floats per lane handed over at the end: O^T, m, l
    static_assert(2 * XCH * 64 * 4 <= 2 * TILEB, "two hand-overs fit one buffer");
    __shared__ __attribute__((aligned(16))) char lds_b0[2 * TILEB];
    __shared__ __attribute__((aligned(16))) char lds_b1[2 * TILEB];
    lds_char* const buf0 = (lds_char*)lds_b0;
    lds_char* const buf1 = (lds_char*)lds_b1;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qblk = wv >> 1, kh = wv & 1;  // query block, key half
    const int n16 = lane & 15, g = lane >> 4;
    const int n_qt = (p.S + QT256 - 1) / QT256;
    const int rank = int(blockIdx.x) / p.Hq;
    const int hq = int(blockIdx.x) - rank * p.Hq;
    const int qt = n_qt - 1 - rank;
    const int hkv = hq / p.G;
    const int qabs0 = p.n_cached - p.S;
    const int q0 = qt * QT256 + qblk * QW256;
    const int n_cached = p.n_cached;

    // Q^T operands: lane -> query q0 + n16, dims 32ks + 8g..+7 (a query past
    // the chunk loads the last row: its column stays finite and is not written)
    bf16x8_t qb[KS];
    {
        const int s = min(q0 + n16, p.S - 1);
        const uint16_t* qrow = p.q + int64_t(hq) * p.q_head_stride + int64_t(s) * p.q_tok_stride;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qb[ks] = as_bf16x8(*reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * g));
    }
    float m = -INFINITY, l = 0.0f;
    // nm = -m (0 while m = -inf); th = the raw score above which the scaled
    // score exceeds m + 8 (-inf while m = -inf)
    float nm = 0.0f, th = -INFINITY;
    f32x4_t acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int wg_last = min(qt * QT256 + QT256, p.S) - 1;
    const int kv_end = p.causal ? min(qabs0 + wg_last + 1, n_cached) : n_cached;
    const int n_tiles = (kv_end + KT256 - 1) / KT256;
    const bool wave_has_rows = q0 < p.S;
    // keys below wave_lim are visible to every query of the wave, keys at or
    // past wave_end to none of them
    const int wave_lim = p.causal ? min(qabs0 + q0 + 1, n_cached) : n_cached;
    const int wave_end = !wave_has_rows ? 0 : p.causal ? min(qabs0 + min(q0 + QW256, p.S), n_cached) : n_cached;

    // ---- staging: wave w moves kind w % 2 (K, V) of page w / 2 of each tile
    const bool paged = p.k_ids != nullptr;
    const int kind = wv & 1, pg = wv >> 1;
    const int32_t* const my_ids = kind ? p.v_ids : p.k_ids;
    const int64_t head_off = int64_t(hkv) * (p.kv_head_stride ? p.kv_head_stride : D);
    const uint16_t* const src = (kind ? p.v_pool : p.k_pool) + head_off;
    const int64_t kv_row = p.kv_row, page_elems = p.page_elems;
    const int kv_row_bytes = int(kv_row) * 2;
    // lane i <- the id of this wave's page of tile t0 + i
    auto load_ids = [&](int t0) -> int {
        const int page = 4 * (t0 + lane) + pg;
        return page * kPage < kv_end ? my_ids[page] : 0;
    };
    // instruction e fills rows 2e, 2e+1 of the page: lane -> row 2e + lane/32,
    // position lane%32 <- chunk 16 (p/16) + ((p%16) ^ swz(row))
    uint32_t dma_off[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int row = 2 * e + (lane >> 5), pos = lane & 31;
        const int chunk = 16 * (pos >> 4) + ((pos & 15) ^ swz(row));
        dma_off[e] = uint32_t(row * kv_row_bytes + 16 * chunk);
    }
    const int dst0 = kind * TILEB + pg * (kPage * ROWB);
    // The buffer resource of a page spans exactly its rows below kv_end, so
    // rows past the causal limit, the cache end or the table read as zeros:
    // their keys are masked and their zero values meet zero probabilities.
    auto issue_tile = [&](int t, int ids, lds_char* buf) {
        const int tok_page = t * KT256 + kPage * pg;
        const int valid = min(max(kv_end - tok_page, 0), kPage);
        const uint32_t span = uint32_t(__builtin_amdgcn_readfirstlane(valid > 0 ? (valid - 1) * kv_row_bytes + ROWB : 0));
        const int64_t base = paged ? int64_t(__builtin_amdgcn_readlane(ids, t & (IDS_BLOCK - 1))) * page_elems
                                   : int64_t(tok_page) * kv_row;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)(src + base), 0, span, kBufferFlags);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(buf + (dst0 + e * 1024)),
                                                     16, dma_off[e], 0, 0, 0);
    };

    // ---- this wave's 32 keys of one tile against its 16 queries (buf: K at
    // 0, V at TILEB).  masked: the keys reach past the first query of the wave
    // or past the cache end.
    const float c = fmaxf(p.scale_log2, __FLT_MIN__);  // > 0: masked -inf scores give exactly 0
    const float inv_c = 1.0f / c;                       // may be inf (then no row grows after its first tile)
    auto compute_tile = [&](int t, const lds_char* buf, bool masked) {
        const int tok0 = t * KT256 + KH * kh;  // first key of the half
        const int r0 = KH * kh;                // its first LDS row (a multiple of 16)
        f32x4_t s[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int row = r0 + 16 * kb + n16;
                const int pos = 16 * (ks >> 2) + ((4 * (ks & 3) + g) ^ swz(n16));
                const u32x4_t a = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
                    buf + (row * ROWB + pos * 16));
                s[kb] = mfma16x16x32(__builtin_bit_cast(bf16x8_t, a), qb[ks], s[kb]);
            }
        if (masked) {
            __asm__ volatile("");  // keep a branch: full tiles carry no selects
            const int qpos = qabs0 + q0 + n16;
            const int lim = p.causal ? min(qpos + 1, n_cached) : n_cached;
            const int rel = lim - tok0 - 4 * g;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[kb][i] = (16 * kb + i < rel) ? s[kb][i] : -INFINITY;
        }
        // raw row max, IEEE maximum (NaN-propagating: v_maximum3_f32, no quieting)
        float mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(s[0][0], s[0][1]),
                                                 __builtin_elementwise_maximum(s[0][2], s[0][3]));
        mx = __builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(__builtin_elementwise_maximum(s[1][0], s[1][1]),
                                                                             __builtin_elementwise_maximum(s[1][2], s[1][3])));
        if (__any(mx > th)) {  // lazy rescale, as in the D = 128 kernel
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const bool grow = mx > th;
            const float mn = grow ? mx * c : m;
            const float alpha = grow ? exp2_fast(m - mn) : 1.0f;
            l *= alpha;
            m = mn;
            nm = grow ? -mn : nm;
            th = grow ? (mn + 8.0f) * inv_c : th;
#pragma unroll
            for (int db = 0; db < DB; ++db) acc[db] *= alpha;
        }
        float e[2][4];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) e[kb][i] = exp2_fast(__builtin_fmaf(s[kb][i], c, nm));
        l += ((e[0][0] + e[0][1]) + (e[0][2] + e[0][3])) + ((e[1][0] + e[1][1]) + (e[1][2] + e[1][3]));
        const bf16x8_t pb = __builtin_bit_cast(
            bf16x8_t, u32x4_t{bf16_pair_rne(e[0][0], e[0][1]), bf16_pair_rne(e[0][2], e[0][3]),
                              bf16_pair_rne(e[1][0], e[1][1]), bf16_pair_rne(e[1][2], e[1][3])});
        // V^T from two transposing reads per 16 dims: rows r0 + 4g + n16/4 and
        // + 16, dims 16db + 4(n16%4)..+3 (chunk 2db + (n16%4)/2, half n16%2);
        // one integer offset per read (see the D = 128 kernel)
        const int row0 = r0 + 4 * g + (n16 >> 2), row1 = row0 + 16;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int chunk = 2 * db + ((n16 & 3) >> 1), half = (n16 & 1) * 8;
            const int pos = 16 * (chunk >> 4) + ((chunk & 15) ^ swz(row0 & 15));
            const int off0 = TILEB + row0 * ROWB + pos * 16 + half;
            const int off1 = TILEB + row1 * ROWB + pos * 16 + half;  // row1 % 16 == row0 % 16
            const s16x4_t lo = ds_read_tr(buf + off0);
            const s16x4_t hi = ds_read_tr(buf + off1);
            const s16x4_t a8[2] = {lo, hi};
            acc[db] = mfma16x16x32(__builtin_bit_cast(bf16x8_t, a8), pb, acc[db]);
        }
    };

    // ---- pipeline: one barrier per tile, two buffers.  Step t waits for its
    // own loads of tile t, meets the other waves (tile t complete in LDS;
    // everybody done with tile t-1), starts tile t+1 into the other buffer,
    // then computes its half of tile t.  Every step issues the same 8 loads
    // per wave; a tile past the last one has no rows below kv_end and reads
    // as zeros.  Page ids arrive IDS_BLOCK tiles per load; the rare reload
    // drains the loads in flight.
    int ids = paged ? load_ids(0) : 0;
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // q and ids landed
    issue_tile(0, ids, buf0);
    auto step = [&](int t, const lds_char* cur, lds_char* nxt) {
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        tile_barrier();
        if (((t + 1) & (IDS_BLOCK - 1)) == 0 && t + 1 < n_tiles) {
            if (paged) ids = load_ids(t + 1);
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        }
        issue_tile(t + 1, ids, nxt);
        const int tok0 = t * KT256 + KH * kh;
        if (tok0 < wave_end) compute_tile(t, cur, tok0 + KH > wave_lim);
    };
    for (int t = 0; t < n_tiles; t += 2) {
        step(t, buf0, buf1);
        step(t + 1, buf1, buf0);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // the trailing (empty) loads have landed: LDS is free

    // ---- merge the two key halves of each query block: the key-half-1 wave
    // stores (O^T, m, l) as [value][lane] floats, the key-half-0 wave combines
    // m = max(m0, m1), O = O0 2^(m0-m) + O1 2^(m1-m), l likewise (a half that
    // saw no key has m = -inf, weight 0) and writes the output.
    __syncthreads();  // every wave is done with the tiles
    lds_float* const xch = (lds_float*)((qblk >> 1) == 0 ? buf0 : buf1) + (qblk & 1) * XCH * 64 + lane;
    if (kh == 1) {
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) xch[(db * 4 + i) * 64] = acc[db][i];
        xch[(DB * 4) * 64] = m;
        xch[(DB * 4 + 1) * 64] = l;
    }
    __syncthreads();
    if (kh == 1 || !wave_has_rows) return;
    const float m1 = xch[(DB * 4) * 64], l1 = xch[(DB * 4 + 1) * 64];
    const float mt = fmaxf(m, m1);
    const float a0 = mt == -INFINITY ? 0.0f : exp2_fast(m - mt), a1 = mt == -INFINITY ? 0.0f : exp2_fast(m1 - mt);
    float lt = l * a0 + l1 * a1;
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    const float inv = 1.0f / lt;
    const int s = q0 + n16;
    if (s >= p.S) return;
    uint16_t* orow = p.out + int64_t(hq) * p.o_head_stride + int64_t(s) * p.o_tok_stride;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (acc[db][i] * a0 + xch[(db * 4 + i) * 64] * a1) * inv;
        uint2 w;
        w.x = bf16_pair_out(o[0], o[1]);
        w.y = bf16_pair_out(o[2], o[3]);
        *reinterpret_cast<uint2*>(orow + 16 * db + 4 * g) = w;
    }
}

}  // namespace

int launch_paged_prefill(const AttnParams& p, int head_dim, hipStream_t stream) {
    if (head_dim != 128 && head_dim != 256) return fail(GENLLM_ERR_UNSUPPORTED, "paged prefill: head_dim must be 128 or 256");
    if (p.S <= 0 || p.n_pages <= 0) return GENLLM_OK;
    if (head_dim == 256) {
        const int64_t n_qt = (p.S + QT256 - 1) / QT256;
        hipLaunchKernelGGL(paged_prefill_d256_kernel, dim3(unsigned(n_qt * p.Hq)), dim3(WAVES256 * 64), 0, stream, p);
        GENLLM_LAUNCH_CHECK("paged_prefill_d256_kernel");
        return GENLLM_OK;
    }
    const int64_t n_pairs = ((p.S + QT - 1) / QT + 1) / 2;
    hipLaunchKernelGGL(paged_prefill_kernel<128>, dim3(unsigned(n_pairs * p.Hq)), dim3(WAVES * 64), 0, stream, p);
    GENLLM_LAUNCH_CHECK("paged_prefill_kernel");
    return GENLLM_OK;
}

}  // namespace genllm
