// paged_prefill.hip -- causal paged FlashAttention on bf16 MFMA (gfx950).
//
// Same result as the attention loop of PagedAttentionImpl<CPU>::execute
// (src/backend/cpu/attention.cpp:148-215) for a chunk of S queries: query s sits
// at q_abs = n_cached - S + s and attends keys 0..q_abs (causal, :164-181),
// kv head = q head / groups (:158).
//
// Grid: query tiles of 64 rows x Hq workgroups of 8 waves: the long half of
// the query tiles from the last down, then the short half from the first up;
// q heads placed so that those of one kv head share an XCD.
// Wave w = qb + 4 kh owns query block qb (16 queries) of the tile and key
// half kh (32 keys) of every key tile of 64 tokens (4 pages), so the two key
// halves of a query block share a SIMD (waves w and w + 4; measured 30.9
// against 31.5 us at config 4 and 47.4 against 48.1 us at head_dim 256 with
// the halves of two query blocks paired instead); the two halves of a query
// block are merged through LDS at the end.  At
// head_dim 128 a workgroup holds 64 KB of LDS and at most 128 VGPRs per lane,
// so two workgroups share a CU (4 waves per SIMD: one workgroup's barrier
// waits and dependent chains are filled by the other's work); the grid's
// order puts a long and a short query tile on each CU.  At head_dim 256 (128
// KB) one workgroup runs per CU.
// Key tiles are staged in two LDS buffers (one tile in flight while the other
// is computed), K and V each as [token][dim] rows whose 16-byte chunks are
// swizzled per 256-byte half: chunk c of row r sits at position
// 16 (c / 16) + ((c % 16) ^ swz(r % 16)), with swz(r) = 2 ((r % 8) ^ 4 (r / 8))
// + r / 8.
// Wave w < 4 moves the K rows, then the V rows of page w of every tile
// straight from HBM into LDS with 16-byte buffer loads in LDS mode (lane i's
// 16 bytes land at base + 16 i), so a tile costs no registers, no VALU and no
// LDS store instructions; one buffer resource per
// page (base = the page of this kv head, size = the bytes its rows below the
// key limit span) bounds every load.  Waves 4-7 issue no loads.
// Per tile and wave:
//   S^T = K Q^T  (v_mfma_f32_16x16x32_bf16 x 2 D/32; A = K from LDS: lane l ->
//        key l%16, dims 32ks+8(l/16)..; B = Q^T held in registers).
//        D[key][q] lands in lane q%16 + 16*(key/4), register key%4: every
//        lane holds 4 keys of ONE query row per 16-key block, so the online
//        softmax state (m, l) of a row is per lane.
//   O^T += V^T P^T  (v_mfma_f32_16x16x32_bf16 x D/16, full rate: 32 keys; B =
//        P^T is the lane's own 8 exponentials; A = V^T from two
//        ds_read_b64_tr_b16 per 16 dims).  O^T[dim][q] belongs to the lane's
//        own query column, so the rescale by 2^(m_old-m_new) stays lane-local.
// Causal masking is applied only to the key halves that reach past the first
// query of the wave (the diagonal) or past the cache end.
#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

namespace {

constexpr int KT = 64;          // keys per tile (4 pages)
constexpr int QW = 16;          // queries per wave (one 16-column block of O^T)
constexpr int WAVES = 8;        // query block (4) x key half (2)
constexpr int QT = 4 * QW;      // queries per query tile
constexpr int IDS_BLOCK = 64;   // tiles whose page ids one vector load brings

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) float lds_float;

// two fp32 -> packed bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t bf16_pair_rne(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// chunk-position swizzle of a 256-byte LDS row, bijective on r % 16.  The
// K reads (16 rows, one chunk each) hit 16 distinct positions.  A transposing
// V read takes 32 bytes (one chunk pair) of each of 16 rows, and the LDS
// serves it in two halves, lanes 0-15 with 32-47 (rows 0-3 and 8-11 of the
// 16) and lanes 16-31 with 48-63 (rows 4-7 and 12-15): the XOR with 4 (r / 8)
// puts the chunk pairs of rows r and r + 8 in different halves of the row,
// so each half of the read covers all 64 banks once (PMC: 2 conflict cycles
// per transposing read without it, none with it; config 4 34.3 -> 33.3 us)
__device__ __forceinline__ constexpr int swz(int r) { return (((r & 7) ^ ((r >> 1) & 4)) << 1) | ((r >> 3) & 1); }

__device__ __forceinline__ s16x4_t ds_read_tr(const lds_char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<__attribute__((address_space(3))) s16x4_t*>(const_cast<lds_char*>(p)));
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

// The key half kh (keys KT t + KH kh .. + KH - 1 of every key tile t) below
// wave_end, for query q0 + n16 (lane n16 + 16 g), formed the reference's way:
// per query over the keys it sees, in fp32, one key after another.  res: the
// O^T values of the lane's dims 16 db + 4 g + i, then m (log2 units) and l
// (the row's, in lane g = 0; 0 elsewhere, as the hand-over adds the four
// lanes).  Called only by waves whose tiled state came out NaN or infinite.
template <int D, bool F16>
__device__ __forceinline__ void prefill_exact_half(const AttnParams& p, int hq, int q0, int kh, int wave_end,
                                                   int n_tiles, float* res) {
    using E = Elem<F16>;
    constexpr int KS = D / 32, DB = D / 16, KH = KT / 2;
    const int lane = threadIdx.x & 63, n16 = lane & 15, g = lane >> 4;
    const int n_cached = p.n_cached, qabs0 = p.n_cached - p.S;
    const int lim = p.causal ? min(qabs0 + q0 + n16 + 1, n_cached) : n_cached;
    const int hkv = hq / p.G;
    const int64_t head_off = int64_t(hkv) * (p.kv_head_stride ? p.kv_head_stride : D);
    const bool paged = p.k_ids != nullptr;
    const uint16_t* const qrow = p.q + int64_t(hq) * p.q_head_stride + int64_t(min(q0 + n16, p.S - 1)) * p.q_tok_stride;
    const float c = fmaxf(p.scale_log2, __FLT_MIN__);
    float m = -INFINITY, l = 0.0f;
    f32x4_t acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    for (int t = 0; t < n_tiles; ++t) {
        for (int j = 0; j < KH; ++j) {
            const int tok = t * KT + KH * kh + j;
            if (tok >= wave_end) break;  // wave-uniform
            const int64_t in_page = int64_t(tok % kPage) * p.kv_row;
            const int64_t krow = paged ? int64_t(p.k_ids[tok / kPage]) * p.page_elems + in_page : int64_t(tok) * p.kv_row;
            const int64_t vrow = paged ? int64_t(p.v_ids[tok / kPage]) * p.page_elems + in_page : int64_t(tok) * p.kv_row;
            float sp = 0.0f;  // this lane's dims 32 ks + 8 g .. + 7, then the row's four lanes
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const uint4 qq = *reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * g);
                const uint4 kk = *reinterpret_cast<const uint4*>(p.k_pool + head_off + krow + 32 * ks + 8 * g);
                const uint32_t qw[4] = {qq.x, qq.y, qq.z, qq.w}, kw[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
                for (int w2 = 0; w2 < 4; ++w2) {
                    sp = __builtin_fmaf(E::lo(qw[w2]), E::lo(kw[w2]), sp);
                    sp = __builtin_fmaf(E::hi(qw[w2]), E::hi(kw[w2]), sp);
                }
            }
            sp += __shfl_xor(sp, 16);
            sp += __shfl_xor(sp, 32);
            const bool vis = tok < lim;
            const float x = sp * c;
            const float mn = vis ? __builtin_fmaxf(m, x) : m;
            const float alpha = m == -INFINITY ? 0.0f : exp2_fast(m - mn);
            const float pk = exp2_fast(x - mn);
            l = vis ? __builtin_fmaf(l, alpha, pk) : l;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const uint2 u = *reinterpret_cast<const uint2*>(p.v_pool + head_off + vrow + 16 * db + 4 * g);
                const float v4[4] = {E::lo(u.x), E::hi(u.x), E::lo(u.y), E::hi(u.y)};
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[db][i] = vis ? __builtin_fmaf(pk, v4[i], acc[db][i] * alpha) : acc[db][i];
            }
            m = mn;
        }
    }
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) res[4 * db + i] = acc[db][i];
    res[4 * DB] = m;
    res[4 * DB + 1] = g == 0 ? l : 0.0f;
}

template <int D, bool F16>
__device__ __forceinline__ void prefill_tiles(const AttnParams& p) {
    using E = Elem<F16>;
    constexpr int KS = D / 32, DB = D / 16;
    constexpr int ROWB = D * 2;       // bytes per token row (256 or 512)
    constexpr int TILEB = KT * ROWB;  // bytes of K (or V) per tile
    constexpr int KH = KT / 2;        // keys of a tile per wave
    constexpr int XCH = DB * 4 + 2;   // floats per lane handed over at the end: O^T, m, l
    static_assert(2 * XCH * 64 * 4 <= 2 * TILEB, "two hand-overs fit one buffer");
    __shared__ __attribute__((aligned(16))) char lds_b0[2 * TILEB];
    __shared__ __attribute__((aligned(16))) char lds_b1[2 * TILEB];
    lds_char* const buf0 = (lds_char*)lds_b0;
    lds_char* const buf1 = (lds_char*)lds_b1;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qblk = wv & 3, kh = wv >> 2;  // query block, key half (waves w and w + 4 share a SIMD)
    const int n16 = lane & 15, g = lane >> 4;
    const int n_qt = (p.S + QT - 1) / QT;
    const int rank = int(blockIdx.x) / p.Hq;
    const int slot = int(blockIdx.x) - rank * p.Hq;
    // Workgroup i runs on XCD i % 8.  With Hq a multiple of 8, slot 8j + x
    // takes q head x Hq/8 + j, so XCD x holds q heads [x Hq/8, (x+1) Hq/8) and
    // the q heads of one kv head read its tiles through one L2 (config 4:
    // FETCH_SIZE 16.2 against 24.2 MiB per launch, the algorithmic q and K/V
    // bytes against 1.5x; 30.32-30.41 against 30.44-30.56 us, A/B on one box)
    const int hq = (p.Hq & 7) == 0 ? (slot & 7) * (p.Hq >> 3) + (slot >> 3) : slot;
    // the first half of the grid runs the query tiles with the most keys, from
    // the last tile down; the second half the others from the first tile up,
    // so that workgroups i and i + half the grid -- the two a CU holds when
    // every workgroup is resident (head_dim 128: 512 workgroups of two per
    // CU at 16 heads) -- carry n_qt + 1 key tiles between them (A/B at config
    // 4: 34.5-34.7 against 36.0-36.2 us with the second half running down too)
    const int half = (n_qt + 1) / 2;
    const int qt = rank < half ? n_qt - 1 - rank : rank - half;
    const int hkv = hq / p.G;
    const int qabs0 = p.n_cached - p.S;
    const int q0 = qt * QT + qblk * QW;
    const int n_cached = p.n_cached;

    // Q^T operands: lane -> query q0 + n16, dims 32ks + 8g..+7 (a query past
    // the chunk loads the last row: its column stays finite and is not written)
    uint4 qb[KS];  // raw 16-bit elements
    {
        const int s = min(q0 + n16, p.S - 1);
        const uint16_t* qrow = p.q + int64_t(hq) * p.q_head_stride + int64_t(s) * p.q_tok_stride;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) qb[ks] = *reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * g);
    }
    float m = -INFINITY, l = 0.0f;
    // nm = -m (0 while m = -inf); th = the raw score above which the scaled
    // score exceeds m + 8 (-inf while m = -inf)
    float nm = 0.0f, th = -INFINITY;
    f32x4_t acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int wg_last = min(qt * QT + QT, p.S) - 1;
    const int kv_end = p.causal ? min(qabs0 + wg_last + 1, n_cached) : n_cached;
    const int n_tiles = (kv_end + KT - 1) / KT;
    const bool wave_has_rows = q0 < p.S;
    // keys below wave_lim are visible to every query of the wave, keys at or
    // past wave_end to none of them
    const int wave_lim = p.causal ? min(qabs0 + q0 + 1, n_cached) : n_cached;
    const int wave_end = !wave_has_rows ? 0 : p.causal ? min(qabs0 + min(q0 + QW, p.S), n_cached) : n_cached;

    // ---- staging: wave w < 4 moves page w of each tile, its K rows, then its
    // V rows; waves 4-7 issue no tile loads.  Waves 4-7 share their SIMDs
    // with waves 0-3 and reach their S^T MFMAs after them, so the step waits
    // for them: keeping the loads' issue off their path measured 31.3 against
    // 31.5 us at config 4 and 48.9 against 50.2 us at head_dim 256 (A/B on one
    // box; the mirror split, waves 4-7 loading, 32.2 and 50.7).  Every K row
    // of the tile is requested before any V row (needed first): 30.6 against
    // 30.9 us at config 4, 47.0 against 47.3 at head_dim 256, against one
    // kind per wave over two pages.
    const bool paged = p.k_ids != nullptr;
    const int pg = wv & 3;  // this wave's page of the tile (waves 0-3)
    const bool dma_wave = wv < 4;
    const int64_t head_off = int64_t(hkv) * (p.kv_head_stride ? p.kv_head_stride : D);
    const int64_t kv_row = p.kv_row, page_elems = p.page_elems;
    const int kv_row_bytes = int(kv_row) * 2;
    // lane i <- the K (kindx 0) or V (1) id of page pg of tile t0 + i
    auto load_ids = [&](int t0, int kindx) -> int {
        const int page = 4 * (t0 + lane) + pg;
        return page * kPage < kv_end ? (kindx ? p.v_ids : p.k_ids)[page] : 0;
    };
    // instruction e fills rows RPI e .. RPI e + RPI-1 of the page (4 rows of
    // 256 B at D = 128, 2 of 512 B at D = 256): lane -> row RPI e + lane/LPR,
    // position p = lane % LPR <- chunk 16 (p/16) + ((p%16) ^ swz(row))
    constexpr int LPR = ROWB / 16, RPI = 64 / LPR, NI = kPage / RPI;  // lanes per row, rows per load, loads per page
    uint32_t dma_off[NI];
#pragma unroll
    for (int e = 0; e < NI; ++e) {
        const int row = RPI * e + lane / LPR, pos = lane % LPR;
        const int chunk = 16 * (pos >> 4) + ((pos & 15) ^ swz(row));
        dma_off[e] = uint32_t(row * kv_row_bytes + 16 * chunk);
    }

    // The buffer resource of a page spans exactly its rows below kv_end, so
    // rows past the causal limit, the cache end or the table read as zeros:
    // their keys are masked and their zero values meet zero probabilities.
    auto issue_page = [&](int t, int ids, lds_char* buf, int kindx) {  // K (0) or V (1) rows of page pg of tile t
        const uint16_t* const src = (kindx ? p.v_pool : p.k_pool) + head_off;
        const int tok_page = t * KT + kPage * pg;
        const int valid = min(max(kv_end - tok_page, 0), kPage);
        const uint32_t span = uint32_t(__builtin_amdgcn_readfirstlane(valid > 0 ? (valid - 1) * kv_row_bytes + ROWB : 0));
        const int64_t base = paged ? int64_t(__builtin_amdgcn_readlane(ids, t & (IDS_BLOCK - 1))) * page_elems
                                   : int64_t(tok_page) * kv_row;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)(src + base), 0, span, kBufferFlags);
#pragma unroll
        for (int e = 0; e < NI; ++e)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                r, (__attribute__((address_space(3))) void*)(buf + (kindx * TILEB + pg * (kPage * ROWB) + e * 1024)), 16,
                dma_off[e], 0, 0, 0);
    };
    auto issue_tile = [&](int t, int ids0, int ids1, lds_char* buf) {  // ids0, ids1: K and V ids of page pg
        if (dma_wave) {
            issue_page(t, ids0, buf, 0);
            issue_page(t, ids1, buf, 1);
        }
    };

    // ---- this wave's 32 keys of one tile against its 16 queries (buf: K at
    // 0, V at TILEB).  masked: the keys reach past the first query of the wave
    // or past the cache end.
    const float c = fmaxf(p.scale_log2, __FLT_MIN__);  // > 0: masked -inf scores give exactly 0
    const float inv_c = 1.0f / c;                       // may be inf (then no row grows after its first tile)
    auto compute_tile = [&](int t, const lds_char* buf, bool masked, auto&& after_s) {
        const int tok0 = t * KT + KH * kh;  // first key of the half
        const int r0 = KH * kh;             // its first LDS row (a multiple of 16)
        f32x4_t s[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int row = r0 + 16 * kb + n16;
                const int pos = 16 * (ks >> 2) + ((4 * (ks & 3) + g) ^ swz(n16));
                const u32x4_t a = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
                    buf + (row * ROWB + pos * 16));
                s[kb] = E::mma32(__builtin_bit_cast(uint4, a), qb[ks], s[kb]);
            }
        after_s();
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
        const uint4 pb = make_uint4(E::pack_p(e[0][0], e[0][1]), E::pack_p(e[0][2], e[0][3]),
                                    E::pack_p(e[1][0], e[1][1]), E::pack_p(e[1][2], e[1][3]));
        // V^T from two transposing reads per 16 dims: rows r0 + 4g + n16/4 and
        // + 16, dims 16db + 4(n16%4)..+3 (chunk 2db + (n16%4)/2, half n16%2);
        // each read's LDS offset is one integer added to the buffer base, which
        // lets the compiler tell these reads from the loads streaming into the
        // other buffer
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
            acc[db] = E::mma32(__builtin_bit_cast(uint4, a8), pb, acc[db]);
        }
    };

    // ---- pipeline: one barrier per tile, two buffers.  Step t waits for its
    // own loads of tile t, meets the other waves (tile t complete in LDS;
    // everybody done with tile t-1), starts tile t+1 into the other buffer,
    // then computes its half of tile t.  Every step issues the same 8 loads
    // in each of waves 0-3; a tile past the last one has no rows below kv_end and reads
    // as zeros.  Page ids arrive IDS_BLOCK tiles per load; the rare reload
    // drains the loads in flight.
    int ids0 = paged && dma_wave ? load_ids(0, 0) : 0;
    int ids1 = paged && dma_wave ? load_ids(0, 1) : 0;
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // q and ids landed
    issue_tile(0, ids0, ids1, buf0);
    auto step = [&](int t, const lds_char* cur, lds_char* nxt) {
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        tile_barrier();
        if (((t + 1) & (IDS_BLOCK - 1)) == 0 && t + 1 < n_tiles) {
            if (paged && dma_wave) {
                ids0 = load_ids(t + 1, 0);
                ids1 = load_ids(t + 1, 1);
            }
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        }
        // At head_dim 256 the next tile's V rows are requested after this
        // tile's S^T MFMAs: the K reads right after the barrier then share the
        // LDS with half the incoming rows, and the longer step still hides the
        // V rows' latency (46.6-46.9 against 48.1-48.2 us at 2048 tokens; at
        // head_dim 128 the step is too short: 32.6 against 30.4 us; A/B on
        // one box).
        constexpr bool late_v = D == 256;
        if (late_v) {
            if (dma_wave) issue_page(t + 1, ids0, nxt, 0);
        } else {
            issue_tile(t + 1, ids0, ids1, nxt);
        }
        auto issue_v = [&]() {
            if (late_v && dma_wave) issue_page(t + 1, ids1, nxt, 1);
        };
        const int tok0 = t * KT + KH * kh;
        if (tok0 < wave_end)
            compute_tile(t, cur, tok0 + KH > wave_lim, issue_v);
        else
            issue_v();
    };
    for (int t = 0; t < n_tiles; t += 2) {
        step(t, buf0, buf1);
        step(t + 1, buf1, buf0);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // the trailing (empty) loads have landed: LDS is free

    // Keys of a masked half that a query may not see meet a zero probability
    // in the P.V MFMA, and 0 x NaN is NaN: a NaN or infinite V row there would
    // reach queries the reference never lets it reach.  A wave whose state
    // came out NaN or infinite (only ever with such inputs) forms its key half
    // again from the pools, in fp32, visiting for each query only the keys it
    // sees, as the reference's loop does.  The check is one sum of the state
    // (a NaN or an infinity in it makes the sum non-finite); measured at
    // config 4, 30.85-30.93 against 30.65-30.80 us (A/B on one box, two passes;
    // checking each value instead cost 0.3-0.4 us).
    {
        float tsum = l;  // NaN or infinite when any of the state is
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) tsum += acc[db][i];
        if (__any(!(fabsf(tsum) <= __FLT_MAX__))) {
            float res[DB * 4 + 2];
            prefill_exact_half<D, F16>(p, hq, q0, kh, wave_end, n_tiles, res);
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[db][i] = res[4 * db + i];
            m = res[4 * DB];
            l = res[4 * DB + 1];
        }
    }

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
        if constexpr (F16) {
            w.x = pack2(E::out(o[0]), E::out(o[1]));
            w.y = pack2(E::out(o[2]), E::out(o[3]));
        } else {
            w.x = bf16_pair_out(o[0], o[1]);
            w.y = bf16_pair_out(o[2], o[3]);
        }
        *reinterpret_cast<uint2*>(orow + 16 * db + 4 * g) = w;
    }
}

// D = 128: 64 KB of LDS and at most 128 VGPRs, so two workgroups share a CU
// (4 waves per SIMD: at config 4 36.2 us, against 41.9 us for the earlier
// form of one 128 KB, 196-VGPR workgroup per CU running two query tiles of
// 2 x 32 queries, A/B on one box); D = 256: 128 KB, one workgroup per CU.
template <bool F16>
__global__ __launch_bounds__(WAVES * 64, 2) void paged_prefill_d128_kernel(AttnParams p) { prefill_tiles<128, F16>(p); }
template <bool F16>
__global__ __launch_bounds__(WAVES * 64) void paged_prefill_d256_kernel(AttnParams p) { prefill_tiles<256, F16>(p); }

}  // namespace

int launch_paged_prefill(const AttnParams& p, int head_dim, hipStream_t stream) {
    if (head_dim != 128 && head_dim != 256) return fail(GENLLM_ERR_UNSUPPORTED, "paged prefill: head_dim must be 128 or 256");
    if (p.S <= 0 || p.n_pages <= 0) return GENLLM_OK;
    const dim3 grid(unsigned(int64_t((p.S + QT - 1) / QT) * p.Hq)), block(WAVES * 64);
    if (head_dim == 128)
        hipLaunchKernelGGL(p.f16 ? paged_prefill_d128_kernel<true> : paged_prefill_d128_kernel<false>, grid, block, 0,
                           stream, p);
    else
        hipLaunchKernelGGL(p.f16 ? paged_prefill_d256_kernel<true> : paged_prefill_d256_kernel<false>, grid, block, 0,
                           stream, p);
    GENLLM_LAUNCH_CHECK("paged_prefill kernel");
    return GENLLM_OK;
}

}  // namespace genllm
