// paged_prefill.hip -- causal paged FlashAttention on bf16 MFMA (gfx950).
//
// Same result as the attention loop of PagedAttentionImpl<CPU>::execute
// (src/backend/cpu/attention.cpp:148-215) for a chunk of S queries: query s sits
// at q_abs = n_cached - S + s and attends keys 0..q_abs (causal, :164-181),
// kv head = q head / groups (:158).
//
// Grid: query tiles of 64 x Hq workgroups of 4 waves.  The tile's queries
// form two groups of 32 (two 16-row MFMA blocks each); each group is served
// by two waves that split every key tile between them (wave 2qg + kh takes
// keys 32kh..32kh+31 of each tile), and the two partial softmax states are
// merged through LDS at the end.  A wave thus reads half a tile from LDS for
// 32 queries: LDS read bandwidth, not the MFMA rate, bounds this loop.
// Key tiles of 64 tokens (4 pages) are staged in LDS double-buffered, K and V
// each as [token][dim] rows of 256 B whose 16-byte chunks are XOR-swizzled
// (chunk c of row r at position c ^ swz(r % 16), swz(r) = 2 (r % 8) + r / 8),
// which keeps both the K operand reads and the transposing V reads free of LDS
// bank conflicts.  Wave w moves page w of every tile, K and V, straight from
// HBM into LDS with 16-byte buffer loads in LDS mode (lane i's 16 bytes land
// at base + 16 i), so a tile costs no registers, no VALU and no LDS store
// instructions; one buffer resource per page (base = the page of this kv
// head, size = the bytes its 16 rows span) bounds every load.
// Per tile and wave, with v_mfma_f32_16x16x32_bf16:
//   S^T = K Q^T  (A = K from LDS: lane l -> token l%16 of a 16-block, dims
//        32ks+8(l/16)..; B = Q^T held in registers).  D[tok][q] lands in lane
//        q%16 + 16*(tok%16/4), register tok%4: every lane holds 8 keys of ONE
//        query row per query block, so the online softmax state (m, l) of a
//        row is per lane.
//   O^T += V^T P^T  (B = P^T from the lane's own S^T registers after exp2 and
//        bf16 packing -- the 8 keys of lane group g are {4g+i, 16+4g+i}, i<4;
//        A = V^T from two ds_read_b64_tr_b16 of those two 4-key groups: in each
//        16-lane group, lane 4j+q points at V[key0+j][dim0+4q..+3] and lane i
//        receives V[key0+0..3][dim0+i]).  O^T[dim][q] again belongs to the
//        lane's own query, so the rescale by 2^(m_old-m_new) is lane-local.
// Causal masking is applied only to the tiles that reach past the first
// query of the wave (the diagonal) or past the cache end.
#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

namespace {

constexpr int KT = 64;      // keys per tile (4 pages)
constexpr int WAVES = 4;    // one page of each tile per wave
constexpr int QW = 32;      // queries per wave (two 16-row blocks)
constexpr int QT = 2 * QW;  // queries per workgroup: two groups of two waves
constexpr int KH = KT / 2;  // keys of a tile per wave

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
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

__device__ __forceinline__ s16x4_t ds_read_tr(const lds_char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        reinterpret_cast<__attribute__((address_space(3))) s16x4_t*>(const_cast<lds_char*>(p)));
}

template <int D>
__global__ __launch_bounds__(WAVES * 64) void paged_prefill_kernel(AttnParams p) {
    static_assert(D == 128, "prefill kernel: head_dim 128");
    constexpr int KS = D / 32;        // k-steps of the S^T product
    constexpr int DB = D / 16;        // 16-dim blocks of O^T
    constexpr int ROWB = D * 2;       // bytes per token row (16 chunks of 16 B)
    constexpr int TILEB = KT * ROWB;  // bytes of a K (or V) tile
    static_assert(ROWB == 16 * 16, "16 chunks per row: the swizzle acts on r % 16");
    constexpr int XCH = 2 * DB * 4 + 4;  // floats per lane handed over at the end: O^T, m, l
    static_assert(XCH * 64 * 4 <= 2 * TILEB, "hand-over fits one buffer");

    // [buffer 0: K, V][buffer 1: K, V], separate arrays so that the compiler
    // sees the tile being loaded and the tile being read as distinct memory
    __shared__ __attribute__((aligned(16))) char lds_b0[2 * TILEB];
    __shared__ __attribute__((aligned(16))) char lds_b1[2 * TILEB];
    lds_char* const buf0 = (lds_char*)lds_b0;
    lds_char* const buf1 = (lds_char*)lds_b1;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS bases go to scalar registers
    const int qg = wv >> 1, kh = wv & 1;                      // query group, key half
    const int n16 = lane & 15, g = lane >> 4;
    // Grid order pairs heavy and light causal tiles: the first half of the
    // workgroups takes query tiles from the last (most keys) downwards, the
    // second half from the first upwards, so workgroups b and b + half --
    // resident together when the dispatcher deals them out round-robin -- sum
    // to the same work.
    const int n_qt = (p.S + QT - 1) / QT;
    const int rank = int(blockIdx.x) / p.Hq;
    const int hq = int(blockIdx.x) - rank * p.Hq;
    const int heavy = (n_qt + 1) / 2;
    const int qt = rank < heavy ? n_qt - 1 - rank : rank - heavy;
    const int hkv = hq / p.G;
    const int qabs0 = p.n_cached - p.S;  // absolute position of query 0
    const int q0 = qt * QT + qg * QW;    // first query of this wave's group

    // Q^T operands (B), block b: lane -> query q0 + 16b + n16, dims 32ks +
    // 8g..+7.  Loads are unconditional (row clamped), zeroed after.
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

    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
    f32x4_t acc[2][DB];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int db = 0; db < DB; ++db) acc[b][db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int wg_last = min(qt * QT + QT, p.S) - 1;
    const int kv_end = p.causal ? min(qabs0 + wg_last + 1, p.n_cached) : p.n_cached;
    const int n_tiles = (kv_end + KT - 1) / KT;
    const bool wave_has_rows = q0 < p.S;
    const int w_last_abs = qabs0 + min(q0 + QW, p.S) - 1;
    // keys below wave_lim are visible to every query of the wave
    const int wave_lim = p.causal ? min(qabs0 + q0 + 1, p.n_cached) : p.n_cached;

    // ---- tile staging.  Lanes 0..3 hold the K ids of the tile's 4 pages,
    // lanes 4..7 the V ids; wave w loads page w.
    const int32_t* const k_ids = p.k_ids;
    const int32_t* const v_ids = p.v_ids;
    const bool paged = k_ids != nullptr;
    const int64_t head_off = int64_t(hkv) * (p.kv_head_stride ? p.kv_head_stride : D);
    const uint16_t* const k_src = p.k_pool + head_off;
    const uint16_t* const v_src = p.v_pool + head_off;
    const int64_t kv_row = p.kv_row, page_elems = p.page_elems;
    const int n_cached = p.n_cached;
    auto load_ids = [&](int tile) -> int {
        const int page = 4 * tile + (lane & 3);
        int id = 0;
        if (lane < 8 && page * kPage < kv_end) id = !paged ? page : lane < 4 ? k_ids[page] : v_ids[page];
        return id;
    };
    // Lane byte offsets inside a page, the same for every tile: instruction e
    // fills rows 4e..4e+3, lane -> row 4e + lane/16 (rows start on page
    // boundaries, so row % 16 is that slot), position lane%16 <- chunk
    // (lane%16) ^ swz(slot).
    const int kv_row_bytes = int(kv_row) * 2;
    uint32_t dma_off[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int slot = 4 * e + (lane >> 4);
        dma_off[e] = uint32_t(slot * kv_row_bytes + 16 * ((lane & 15) ^ swz(slot)));
    }
    // Paged: the page of id k starts at k * page_elems; its 16 rows of this kv
    // head span 15 kv_row + D elements.  Head-major tensor: the "page" starts
    // at its first token and holds the rows still below n_cached -- the buffer
    // returns zeros past them.
    const uint32_t page_span = uint32_t(15 * kv_row_bytes + ROWB);
    auto issue_tile = [&](int tile, int ids, lds_char* buf) {
        const int tok_page = tile * KT + kPage * wv;  // first token of this wave's page
        int64_t kbase, vbase;
        uint32_t span;
        if (paged) {
            kbase = int64_t(__builtin_amdgcn_readlane(ids, wv)) * page_elems;
            vbase = int64_t(__builtin_amdgcn_readlane(ids, 4 + wv)) * page_elems;
            span = page_span;
        } else {
            kbase = vbase = int64_t(tok_page) * kv_row;
            // (readfirstlane: the value is uniform, keep it in a scalar register
            // so the buffer resource needs no per-lane loop)
            span = uint32_t(__builtin_amdgcn_readfirstlane(max(min(n_cached - tok_page, kPage), 0) * kv_row_bytes));
        }
        const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc((void*)(k_src + kbase), 0, span, kBufferFlags);
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc((void*)(v_src + vbase), 0, span, kBufferFlags);
        const int dst0 = wv * (kPage * ROWB);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (__attribute__((address_space(3))) void*)(buf + (dst0 + e * 1024)),
                                                     16, dma_off[e], 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (__attribute__((address_space(3))) void*)(buf + (TILEB + dst0 + e * 1024)),
                                                     16, dma_off[e], 0, 0, 0);
        }
    };
    // V rows at or past kv_end of the tile hold no key (or one no query here
    // may see); they are zeroed so that their zero probabilities never meet
    // a non-finite value.  Each wave clears rows of its own page, after its
    // own loads of them have landed.
    auto clear_tail = [&](int tile, lds_char* buf) {
        const int first = tile * KT + kPage * wv;
        if (first + kPage <= kv_end) return;  // wave-uniform
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int slot = 4 * e + (lane >> 4);  // the row lane's 16 bytes landed in: base + 16 lane
            if (first + slot >= kv_end)
                *reinterpret_cast<__attribute__((address_space(3))) u32x4_t*>(
                    buf + (TILEB + wv * (kPage * ROWB) + e * 1024 + 16 * lane)) = u32x4_t{0u, 0u, 0u, 0u};
        }
    };

    // ---- this wave's half of one tile from LDS (buf: K at 0, V at TILEB).
    // masked: the half reaches past the first query of the wave or past the
    // cache end.
    auto compute_tile = [&](int t, const lds_char* buf, bool masked) {
        const int tok0 = t * KT + KH * kh;  // first key of the half
        const int r0 = KH * kh;             // its first LDS row (a multiple of 16)
        // S^T = K Q^T: s[kb][b] = keys 16kb.. of the half x query block b
        f32x4_t s[2][2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int b = 0; b < 2; ++b) s[kb][b] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int row = r0 + 16 * kb + n16;
                const int pos = (4 * ks + g) ^ swz(n16);  // row % 16 == n16
                const u32x4_t a = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
                    buf + (row * ROWB + pos * 16));
#pragma unroll
                for (int b = 0; b < 2; ++b) s[kb][b] = mfma16x16x32(__builtin_bit_cast(bf16x8_t, a), qb[b][ks], s[kb][b]);
            }

        // online softmax, per lane = per query row of each block.
        // The scale (>= 0, checked by the host) is raised to at least FLT_MIN,
        // so that a masked score of -inf gives exp2(-inf * c - m) = 0 without a
        // select; at scale 0 every weight stays exp2(~0) = 1.
        const float c = fmaxf(p.scale_log2, __FLT_MIN__);
        if (masked) {
            // wave-uniform; the empty asm keeps this a branch of its own
            // instead of selects on every tile.  A key is visible to a query
            // when kpos < lim (lim = n_cached, or q_abs + 1 when causal); the
            // lane's keys are tok0 + 16kb + 4g + i.
            __asm__ volatile("");
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int qpos = qabs0 + q0 + 16 * b + n16;
                const int lim = p.causal ? min(qpos + 1, n_cached) : n_cached;
                const int rel = lim - tok0 - 4 * g;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[kb][b][i] = (16 * kb + i < rel) ? s[kb][b][i] : -INFINITY;
            }
        }
        // max over raw scores (c > 0), then p = exp2(s * scale*log2e - m), one fma.
        // Lazy rescale: a row's reference max only moves (and its l, O^T are
        // rescaled) when the tile max exceeds it by more than 2^8, so p <= 256;
        // a lane's own keys decide whether any row may grow, and the row max
        // (two cross-lane steps) is formed only then.
        float mx[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            float mr = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i) mr = fmaxf(mr, s[kb][b][i]);
            mx[b] = mr * c;
        }
        if (__any(mx[0] > m[0] + 8.0f || mx[1] > m[1] + 8.0f)) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                float r = fmaxf(mx[b], __shfl_xor(mx[b], 16));
                r = fmaxf(r, __shfl_xor(r, 32));
                const bool grow = r > m[b] + 8.0f;
                const float mn = grow ? r : m[b];
                const float alpha = grow ? exp2_fast(m[b] - mn) : 1.0f;
                l[b] *= alpha;
                m[b] = mn;
#pragma unroll
                for (int db = 0; db < DB; ++db) acc[b][db] *= alpha;
            }
        }
        bf16x8_t pb[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const float mu = m[b] == -INFINITY ? 0.0f : m[b];
            float sum = 0.0f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e = exp2_fast(__builtin_fmaf(s[kb][b][i], c, -mu));  // masked: exactly 0
                    s[kb][b][i] = e;
                    sum += e;
                }
            l[b] += sum;
            uint4 u;
            u.x = bf16_pair_rne(s[0][b][0], s[0][b][1]);
            u.y = bf16_pair_rne(s[0][b][2], s[0][b][3]);
            u.z = bf16_pair_rne(s[1][b][0], s[1][b][1]);
            u.w = bf16_pair_rne(s[1][b][2], s[1][b][3]);
            pb[b] = as_bf16x8(u);
        }

        // O^T += V^T P^T.  This lane's source address for the transposing
        // reads: row key0 + n16/4, dims 16db + 4(n16%4)..+3 (chunk 2db +
        // (n16%4)/2, half n16%2).  The byte offsets are formed as one integer
        // and applied to the buffer in a single step: the compiler attributes
        // an LDS access to its array (and so can tell it apart from the loads
        // still streaming into the other buffer, without waiting for them) only
        // through a short chain of pointer arithmetic.
        const int row0 = r0 + 4 * g + (n16 >> 2), row1 = row0 + 16;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const int chunk = 2 * db + ((n16 & 3) >> 1), half = (n16 & 1) * 8;
            const int off0 = TILEB + row0 * ROWB + ((chunk ^ swz(row0 & 15)) * 16) + half;
            const int off1 = TILEB + row1 * ROWB + ((chunk ^ swz(row1 & 15)) * 16) + half;
            const s16x4_t lo = ds_read_tr(buf + off0);
            const s16x4_t hi = ds_read_tr(buf + off1);
            const s16x4_t a8[2] = {lo, hi};
            const bf16x8_t va = __builtin_bit_cast(bf16x8_t, a8);
#pragma unroll
            for (int b = 0; b < 2; ++b) acc[b][db] = mfma16x16x32(va, pb[b], acc[b][db]);
        }
    };

    // ---- pipeline: one barrier per tile, two LDS buffers.  Iteration t waits
    // for its own loads of tile t, clears the tail, meets the other waves (tile
    // t complete in LDS; everybody done reading tile t-1), starts tile t+1 into
    // the other buffer, fetches the ids of tile t+2, then computes its half of
    // tile t.
    int ids_next = 0;
    if (n_tiles > 0) {
        const int ids0 = load_ids(0);
        if (n_tiles > 1) ids_next = load_ids(1);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // q and ids landed on every path
        issue_tile(0, ids0, buf0);
    }
    auto step = [&](int t, lds_char* cur, lds_char* nxt) {
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        clear_tail(t, cur);
        __syncthreads();
        if (t + 1 < n_tiles) {
            issue_tile(t + 1, ids_next, nxt);
            if (t + 2 < n_tiles) ids_next = load_ids(t + 2);
        }
        // masked unless every key of the half is visible to every query of the wave
        const int tok0 = t * KT + KH * kh;
        if (wave_has_rows && !(p.causal && tok0 > w_last_abs)) compute_tile(t, cur, tok0 + KH > wave_lim);
    };
    for (int t = 0; t < n_tiles; t += 2) {
        step(t, buf0, buf1);
        if (t + 1 < n_tiles) step(t + 1, buf1, buf0);
    }

    // ---- merge the two key halves of each query group.  The key-half-1 wave
    // stores (O^T, m, l) as [value][lane] floats in the buffer of its group;
    // the key-half-0 wave combines: m = max(m0, m1), O = O0 2^(m0-m) +
    // O1 2^(m1-m), l likewise (a half that saw no key has m = -inf, weight 0).
    __syncthreads();  // every wave is done with the tiles
    lds_float* const xch = (lds_float*)(qg == 0 ? buf0 : buf1);
    if (kh == 1) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) xch[((b * DB + db) * 4 + i) * 64 + lane] = acc[b][db][i];
            xch[(2 * DB * 4 + b) * 64 + lane] = m[b];
            xch[(2 * DB * 4 + 2 + b) * 64 + lane] = l[b];
        }
    }
    __syncthreads();
    if (kh == 1 || !wave_has_rows) return;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const float m1 = xch[(2 * DB * 4 + b) * 64 + lane];
        const float l1 = xch[(2 * DB * 4 + 2 + b) * 64 + lane];
        const float mt = fmaxf(m[b], m1);
        const float a0 = exp2_fast(m[b] - mt), a1 = exp2_fast(m1 - mt);
        float lt = l[b] * a0 + l1 * a1;
        lt += __shfl_xor(lt, 16);
        lt += __shfl_xor(lt, 32);
        const float inv = 1.0f / lt;
        const int s = q0 + 16 * b + n16;
        if (s < p.S) {
            uint16_t* orow = p.out + int64_t(hq) * p.o_head_stride + int64_t(s) * p.o_tok_stride;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                float o[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[i] = (acc[b][db][i] * a0 + xch[((b * DB + db) * 4 + i) * 64 + lane] * a1) * inv;
                uint2 w;
                w.x = pack2(f32_to_bf16_ref(o[0]), f32_to_bf16_ref(o[1]));
                w.y = pack2(f32_to_bf16_ref(o[2]), f32_to_bf16_ref(o[3]));
                *reinterpret_cast<uint2*>(orow + 16 * db + 4 * g) = w;
            }
        }
    }
}

// ---------------------------------------------------------------- D = 256
// Qwen3.5's head_dim (Qwen35.hpp:14-16).  A token row is 512 B (32 chunks of
// 16 B); both 256-byte halves carry the swizzle above (chunk c of row r at
// position 16 (c / 16) + ((c % 16) ^ swz(r % 16))).  Two query blocks per wave
// would need 128 accumulator registers here, so each wave owns one 16-query
// block and every key of the tile; key tiles are 32 tokens (2 pages), double
// buffered in 64 KB of LDS (two workgroups per CU).  Wave w moves the K
// (w even) or V (w odd) rows of page w / 2 of each tile.
constexpr int KT256 = 32;
constexpr int QW256 = 16;
constexpr int QT256 = QW256 * WAVES;

__global__ __launch_bounds__(WAVES * 64) void paged_prefill_d256_kernel(AttnParams p) {
    constexpr int D = 256;
    constexpr int KS = D / 32, DB = D / 16;
    constexpr int ROWB = D * 2;          // 512 bytes per token row
    constexpr int TILEB = KT256 * ROWB;  // 16 KB of K (or V) per tile
    __shared__ __attribute__((aligned(16))) char lds_b0[2 * TILEB];
    __shared__ __attribute__((aligned(16))) char lds_b1[2 * TILEB];
    lds_char* const buf0 = (lds_char*)lds_b0;
    lds_char* const buf1 = (lds_char*)lds_b1;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n16 = lane & 15, g = lane >> 4;
    const int n_qt = (p.S + QT256 - 1) / QT256;
    const int rank = int(blockIdx.x) / p.Hq;
    const int hq = int(blockIdx.x) - rank * p.Hq;
    const int heavy = (n_qt + 1) / 2;
    const int qt = rank < heavy ? n_qt - 1 - rank : rank - heavy;  // heavy and light tiles paired
    const int hkv = hq / p.G;
    const int qabs0 = p.n_cached - p.S;
    const int q0 = qt * QT256 + wv * QW256;

    bf16x8_t qb[KS];
    {
        const int s = q0 + n16;
        const bool ok = s < p.S;
        const uint16_t* qrow = p.q + int64_t(hq) * p.q_head_stride + int64_t(ok ? s : p.S - 1) * p.q_tok_stride;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint4 u = *reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * g);
            if (!ok) u = make_uint4(0, 0, 0, 0);
            qb[ks] = as_bf16x8(u);
        }
    }
    float m = -INFINITY, l = 0.0f;
    f32x4_t acc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int wg_last = min(qt * QT256 + QT256, p.S) - 1;
    const int kv_end = p.causal ? min(qabs0 + wg_last + 1, p.n_cached) : p.n_cached;
    const int n_tiles = (kv_end + KT256 - 1) / KT256;
    const bool wave_has_rows = q0 < p.S;
    const int w_last_abs = qabs0 + min(q0 + QW256, p.S) - 1;
    const int wave_lim = p.causal ? min(qabs0 + q0 + 1, p.n_cached) : p.n_cached;

    // ---- staging: wave w moves kind w % 2 (K, V) of page w / 2 of each tile;
    // lanes 0..1 hold the tile's two K ids, lanes 2..3 the V ids
    const int32_t* const k_ids = p.k_ids;
    const int32_t* const v_ids = p.v_ids;
    const bool paged = k_ids != nullptr;
    const int64_t head_off = int64_t(hkv) * (p.kv_head_stride ? p.kv_head_stride : D);
    const int kind = wv & 1, pg = wv >> 1;
    const uint16_t* const src = (kind ? p.v_pool : p.k_pool) + head_off;
    const int64_t kv_row = p.kv_row, page_elems = p.page_elems;
    const int n_cached = p.n_cached;
    auto load_ids = [&](int tile) -> int {
        const int page = 2 * tile + (lane & 1);
        int id = 0;
        if (lane < 4 && page * kPage < kv_end) id = !paged ? page : lane < 2 ? k_ids[page] : v_ids[page];
        return id;
    };
    // instruction e fills rows 2e, 2e+1 of the page: lane -> row 2e + lane/32,
    // position lane%32 <- chunk 16 (p/16) + ((p%16) ^ swz(row))
    const int kv_row_bytes = int(kv_row) * 2;
    uint32_t dma_off[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int row = 2 * e + (lane >> 5), pos = lane & 31;
        const int chunk = 16 * (pos >> 4) + ((pos & 15) ^ swz(row));
        dma_off[e] = uint32_t(row * kv_row_bytes + 16 * chunk);
    }
    const uint32_t page_span = uint32_t(15 * kv_row_bytes + ROWB);
    const int dst0 = kind * TILEB + pg * (kPage * ROWB);
    auto issue_tile = [&](int tile, int ids, lds_char* buf) {
        const int tok_page = tile * KT256 + kPage * pg;
        int64_t base;
        uint32_t span;
        if (paged) {
            base = int64_t(__builtin_amdgcn_readlane(ids, 2 * kind + pg)) * page_elems;
            span = page_span;
        } else {
            base = int64_t(tok_page) * kv_row;
            span = uint32_t(__builtin_amdgcn_readfirstlane(max(min(n_cached - tok_page, kPage), 0) * kv_row_bytes));
        }
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)(src + base), 0, span, kBufferFlags);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(buf + (dst0 + e * 1024)),
                                                     16, dma_off[e], 0, 0, 0);
    };
    // V rows at or past kv_end are zeroed by the wave that loaded them
    auto clear_tail = [&](int tile, lds_char* buf) {
        if (kind == 0) return;
        const int first = tile * KT256 + kPage * pg;
        if (first + kPage <= kv_end) return;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int row = 2 * e + (lane >> 5);
            if (first + row >= kv_end)
                *reinterpret_cast<__attribute__((address_space(3))) u32x4_t*>(buf + (dst0 + e * 1024 + 16 * lane)) =
                    u32x4_t{0u, 0u, 0u, 0u};
        }
    };

    auto compute_tile = [&](int t, const lds_char* buf, bool masked) {
        const int tok0 = t * KT256;
        f32x4_t s[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int row = 16 * kb + n16;
                const int pos = 16 * (ks >> 2) + ((4 * (ks & 3) + g) ^ swz(n16));
                const u32x4_t a = *reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(
                    buf + (row * ROWB + pos * 16));
                s[kb] = mfma16x16x32(__builtin_bit_cast(bf16x8_t, a), qb[ks], s[kb]);
            }
        const float c = fmaxf(p.scale_log2, __FLT_MIN__);  // > 0: masked -inf scores give exactly 0
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
        float mr = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) mr = fmaxf(mr, s[kb][i]);
        float mx = mr * c;
        if (__any(mx > m + 8.0f)) {  // lazy rescale, as in the D = 128 kernel
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const bool grow = mx > m + 8.0f;
            const float mn = grow ? mx : m;
            const float alpha = grow ? exp2_fast(m - mn) : 1.0f;
            l *= alpha;
            m = mn;
#pragma unroll
            for (int db = 0; db < DB; ++db) acc[db] *= alpha;
        }
        const float mu = m == -INFINITY ? 0.0f : m;
        float sum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = exp2_fast(__builtin_fmaf(s[kb][i], c, -mu));
                s[kb][i] = e;
                sum += e;
            }
        l += sum;
        uint4 u;
        u.x = bf16_pair_rne(s[0][0], s[0][1]);
        u.y = bf16_pair_rne(s[0][2], s[0][3]);
        u.z = bf16_pair_rne(s[1][0], s[1][1]);
        u.w = bf16_pair_rne(s[1][2], s[1][3]);
        const bf16x8_t pb = as_bf16x8(u);
        // V^T from two transposing reads per 16 dims: rows 4g + n16/4 and + 16,
        // dims 16db + 4(n16%4)..+3 (chunk 2db + (n16%4)/2, half n16%2); one
        // integer offset per read (see the D = 128 kernel)
        const int row0 = 4 * g + (n16 >> 2), row1 = row0 + 16;
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

    int ids_next = 0;
    if (n_tiles > 0) {
        const int ids0 = load_ids(0);
        if (n_tiles > 1) ids_next = load_ids(1);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        issue_tile(0, ids0, buf0);
    }
    auto step = [&](int t, lds_char* cur, lds_char* nxt) {
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        clear_tail(t, cur);
        __syncthreads();
        if (t + 1 < n_tiles) {
            issue_tile(t + 1, ids_next, nxt);
            if (t + 2 < n_tiles) ids_next = load_ids(t + 2);
        }
        const int tok0 = t * KT256;
        if (wave_has_rows && !(p.causal && tok0 > w_last_abs)) compute_tile(t, cur, tok0 + KT256 > wave_lim);
    };
    for (int t = 0; t < n_tiles; t += 2) {
        step(t, buf0, buf1);
        if (t + 1 < n_tiles) step(t + 1, buf1, buf0);
    }

    if (!wave_has_rows) return;
    float lt = l;
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    const float inv = 1.0f / lt;
    const int s = q0 + n16;
    if (s >= p.S) return;
    uint16_t* orow = p.out + int64_t(hq) * p.o_head_stride + int64_t(s) * p.o_tok_stride;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        uint2 w;
        w.x = pack2(f32_to_bf16_ref(acc[db][0] * inv), f32_to_bf16_ref(acc[db][1] * inv));
        w.y = pack2(f32_to_bf16_ref(acc[db][2] * inv), f32_to_bf16_ref(acc[db][3] * inv));
        *reinterpret_cast<uint2*>(orow + 16 * db + 4 * g) = w;
    }
}

}  // namespace

int launch_paged_prefill(const AttnParams& p, int head_dim, hipStream_t stream) {
    if (head_dim != 128 && head_dim != 256) return fail(GENLLM_ERR_UNSUPPORTED, "paged prefill: head_dim must be 128 or 256");
    if (p.S <= 0 || p.n_pages <= 0) return GENLLM_OK;
    if (head_dim == 256) {
        const int64_t n_qt = (p.S + QT256 - 1) / QT256;
        hipLaunchKernelGGL(paged_prefill_d256_kernel, dim3(unsigned(n_qt * p.Hq)), dim3(WAVES * 64), 0, stream, p);
        GENLLM_LAUNCH_CHECK("paged_prefill_d256_kernel");
        return GENLLM_OK;
    }
    const int64_t n_qt = (p.S + QT - 1) / QT;
    hipLaunchKernelGGL(paged_prefill_kernel<128>, dim3(unsigned(n_qt * p.Hq)), dim3(WAVES * 64), 0, stream, p);
    GENLLM_LAUNCH_CHECK("paged_prefill_kernel");
    return GENLLM_OK;
}

}  // namespace genllm
