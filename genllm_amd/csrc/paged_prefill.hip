// paged_prefill.hip -- causal paged FlashAttention on bf16 MFMA (gfx950).
//
// Same result as the attention loop of PagedAttentionImpl<CPU>::execute
// (src/backend/cpu/attention.cpp:148-215) for a chunk of S queries: query s sits
// at q_abs = n_cached - S + s and attends keys 0..q_abs (causal, :164-181),
// kv head = q head / groups (:158).
//
// Grid: query tiles x Hq workgroups of WAVES x 64 threads.  A workgroup owns
// QW*WAVES consecutive queries of one q head; wave w owns QW = 16*NB of them
// (NB 16-row MFMA blocks).  K/V tiles of 64 tokens (4 pages) are gathered through the
// block table into LDS:
//   K  as [token][dim]  (row pad 16 B),
//   V  transposed as [dim][token] (row pad 8 B) -- pairs of tokens are packed
//      into dwords so the transpose is plain ds_write_b32.
// Per tile and wave, with v_mfma_f32_16x16x32_bf16:
//   S^T = K Q^T  (A = K from LDS: lane l -> token l%16 of a 16-block, dims
//        32ks+8(l/16)..; B = Q^T held in registers).  D[tok][q] lands in lane
//        q%16 + 16*(tok%16/4), register tok%4: every lane holds 16 keys of ONE
//        query row per 16-query block, so the online softmax state (m, l) of a
//        row is per lane and the row max needs only two cross-lane shuffles.
//   O^T += V^T P^T  (A = V^T from LDS, two 8-byte reads; B = P^T taken from the
//        lane's own S^T registers after exp2 and bf16 packing -- the 8 keys of
//        lane group g for k-step kt are {32kt+4g+i, 32kt+16+4g+i}, i<4, and
//        the V^T reads use the same 8 keys).  O^T[dim][q] again belongs to the
//        lane's own query, so the rescale by 2^(m_old-m_new) is lane-local.
#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

namespace {

constexpr int KT = 64;  // keys per tile (4 pages)
// 16-row query blocks per wave: 1 keeps a wave at 184 registers, so two
// workgroups (8 waves) share a CU and the grid's heavy/light pairing applies.
constexpr int kPrefillBlocks = 1;

__device__ __forceinline__ uint32_t bf16_pair_rne(float lo, float hi) {
    const __bf16 a = static_cast<__bf16>(lo), b = static_cast<__bf16>(hi);
    return uint32_t(__builtin_bit_cast(uint16_t, a)) | (uint32_t(__builtin_bit_cast(uint16_t, b)) << 16);
}

template <int D, int WAVES, int NB>
__global__ __launch_bounds__(WAVES * 64) void paged_prefill_kernel(AttnParams p) {
    static_assert(D == 128, "prefill kernel: head_dim 128");
    constexpr int KS = D / 32;     // k-steps of the S^T product
    constexpr int DB = D / 16;     // 16-dim blocks of O^T
    constexpr int KROW = D + 8;    // K tile row stride (elements)
    constexpr int VROW = KT + 4;   // V^T tile row stride (elements)
    constexpr int NT = WAVES * 64;
    constexpr int QW = 16 * NB;  // queries per wave: NB blocks of 16 rows
    constexpr int QT = QW * WAVES;

    __shared__ __attribute__((aligned(16))) uint16_t k_lds[2 * KT * KROW];  // two buffers
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[2 * D * VROW];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
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
    const int qabs0 = p.n_cached - p.S;   // absolute position of query 0
    const int q0 = qt * QT + wv * QW;     // first query of this wave

    // Q^T operands (B): lane -> query q0 + 16nb + n16, dims 32ks + 8g..+7
    bf16x8_t qb[NB][KS];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        // unconditional loads (row clamped into the chunk), zeroed after: a
        // load under a branch keeps the compiler from proving it complete later
        const int s = q0 + 16 * nb + n16;
        const bool ok = s < p.S;
        const uint16_t* qrow = p.q + int64_t(hq) * p.q_head_stride + int64_t(ok ? s : p.S - 1) * p.q_tok_stride;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint4 u = *reinterpret_cast<const uint4*>(qrow + 32 * ks + 8 * g);
            if (!ok) u = make_uint4(0, 0, 0, 0);
            qb[nb][ks] = as_bf16x8(u);
        }
    }

    float m[NB], l[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) m[nb] = -INFINITY, l[nb] = 0.0f;
    f32x4_t acc[DB][NB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[db][nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int wg_last = min(qt * QT + QT, p.S) - 1;
    const int kv_end = p.causal ? min(qabs0 + wg_last + 1, p.n_cached) : p.n_cached;
    const int n_tiles = (kv_end + KT - 1) / KT;
    const bool wave_has_rows = q0 < p.S;
    const int w_last_abs = qabs0 + min(q0 + QW, p.S) - 1;
    const int w_first_abs = qabs0 + q0;

    // Pipeline (one barrier per tile, two LDS buffers):
    //   iteration t: store tile t+1 (already in registers) into buffer (t+1)&1,
    //   request tile t+2 from HBM into registers using its block-table entries
    //   (fetched one iteration earlier), fetch the entries of tile t+3, then
    //   compute tile t from buffer t&1.
    // Thread -> data: K chunk e of a tile is token 16e + tid/16 (page e of the
    // tile), dims 8*(tid%16)..+7; V task e is the token pair 2*(tid%32), +1
    // (page (tid%32)/8), dims 8*(tid/32 + 8e)..+7.  Lanes 0..3 of every wave
    // hold the tile's 4 K page ids, lanes 4..7 its 4 V page ids.
    constexpr int KCH = KT * (D / 8) / NT;          // 16-byte K chunks per thread
    constexpr int VTK = (KT / 2) * (D / 8) / NT;    // V token-pair tasks per thread
    static_assert(KCH * NT == KT * (D / 8) && VTK * NT == (KT / 2) * (D / 8), "tile split");
    static_assert(NT % (KT / 2) == 0 && (NT / (D / 8)) * KCH == KT && KCH == KT / kPage, "thread map");
    uint4 kreg[KCH], va[VTK], vb[VTK];
    // in-page element offsets are the same for every tile (tiles start on page boundaries)
    const int tp = tid & (KT / 2 - 1);
    const int64_t head_off = int64_t(hkv) * (p.kv_head_stride ? p.kv_head_stride : D);
    const uint16_t* kbase = p.k_pool + (tid >> 4) * p.kv_row + head_off + 8 * (tid & 15);
    const uint16_t* vbase = p.v_pool + ((2 * tp) % kPage) * p.kv_row + head_off + 8 * (tid >> 5);
    // kernel arguments used inside the lambdas, read once into registers
    const int32_t* const k_ids = p.k_ids;
    const int32_t* const v_ids = p.v_ids;
    const bool paged = k_ids != nullptr;
    auto load_ids = [&](int tile) -> int {
        const int page = 4 * tile + (lane & 3);
        int id = 0;
        if (lane < 8 && page * kPage < kv_end) id = !paged ? page : lane < 4 ? k_ids[page] : v_ids[page];
        return id;
    };
    auto load_tile = [&](int tile, int ids) {
        const int tok0 = tile * KT;
        const int64_t vid = __shfl(ids, 4 + (tp >> 3));
        if (tok0 + KT <= p.n_cached) {  // whole tile cached: no per-load conditions
#pragma unroll
            for (int e = 0; e < KCH; ++e)
                kreg[e] = *reinterpret_cast<const uint4*>(kbase + int64_t(__builtin_amdgcn_readlane(ids, e)) *
                                                                      p.page_elems);
#pragma unroll
            for (int e = 0; e < VTK; ++e) {
                const uint16_t* src = vbase + vid * p.page_elems + 8 * (NT / 32) * e;
                va[e] = *reinterpret_cast<const uint4*>(src);
                vb[e] = *reinterpret_cast<const uint4*>(src + p.kv_row);
            }
            return;
        }
#pragma unroll
        for (int e = 0; e < KCH; ++e) {
            const int pos = tok0 + 16 * e + (tid >> 4);
            const int64_t id = __builtin_amdgcn_readlane(ids, e);
            kreg[e] = make_uint4(0, 0, 0, 0);
            if (pos < p.n_cached) kreg[e] = *reinterpret_cast<const uint4*>(kbase + id * p.page_elems);
        }
        const int pos = tok0 + 2 * tp;
#pragma unroll
        for (int e = 0; e < VTK; ++e) {
            const uint16_t* src = vbase + vid * p.page_elems + 8 * (NT / 32) * e;
            va[e] = make_uint4(0, 0, 0, 0);
            vb[e] = make_uint4(0, 0, 0, 0);
            if (pos < p.n_cached) va[e] = *reinterpret_cast<const uint4*>(src);
            if (pos + 1 < p.n_cached) vb[e] = *reinterpret_cast<const uint4*>(src + p.kv_row);
        }
    };
    auto store_tile = [&](int buf) {
        uint16_t* kl = k_lds + buf * (KT * KROW);
        uint16_t* vl = v_lds + buf * (D * VROW);
#pragma unroll
        for (int e = 0; e < KCH; ++e) {
            const int tt = 16 * e + (tid >> 4), ch = tid & 15;
            *reinterpret_cast<uint4*>(&kl[tt * KROW + 8 * ch]) = kreg[e];
        }
        // V transposed: the dword at V^T[d][2tp] packs tokens 2tp (low) and 2tp+1 (high)
#pragma unroll
        for (int e = 0; e < VTK; ++e) {
            const int ch = (tid >> 5) + (NT / 32) * e;
            const uint32_t av[4] = {va[e].x, va[e].y, va[e].z, va[e].w};
            const uint32_t bv[4] = {vb[e].x, vb[e].y, vb[e].z, vb[e].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t* row0 = reinterpret_cast<uint32_t*>(&vl[(8 * ch + 2 * q) * VROW + 2 * tp]);
                uint32_t* row1 = reinterpret_cast<uint32_t*>(&vl[(8 * ch + 2 * q + 1) * VROW + 2 * tp]);
                *row0 = __builtin_amdgcn_perm(bv[q], av[q], 0x05040100u);  // low halves
                *row1 = __builtin_amdgcn_perm(bv[q], av[q], 0x07060302u);  // high halves
            }
        }
    };

    int ids_next = 0;
    if (n_tiles > 0) load_tile(0, load_ids(0));
    // Q and tile 0 have landed on every path.  Without this unconditional
    // wait the compiler cannot prove that the Q loads completed before the
    // loop and waits for all outstanding loads (the prefetched tiles too) at
    // the first use of Q in every iteration.
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    if (n_tiles > 0) {
        store_tile(0);
        if (n_tiles > 1) load_tile(1, load_ids(1));
        if (n_tiles > 2) ids_next = load_ids(2);
    }
    for (int t = 0; t < n_tiles; ++t) {
        const int tok0 = t * KT;
        __syncthreads();  // tile t is in LDS; nobody still reads buffer (t+1)&1
        if (t + 1 < n_tiles) store_tile((t + 1) & 1);
        if (t + 2 < n_tiles) {
            load_tile(t + 2, ids_next);
            if (t + 3 < n_tiles) ids_next = load_ids(t + 3);
        }
        if (!wave_has_rows || (p.causal && tok0 > w_last_abs)) continue;
        const uint16_t* k_cur = k_lds + (t & 1) * (KT * KROW);
        const uint16_t* v_cur = v_lds + (t & 1) * (D * VROW);

        // ---- S^T = K Q^T
        f32x4_t s[4][NB];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) s[mb][nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                const bf16x8_t a =
                    as_bf16x8(*reinterpret_cast<const uint4*>(&k_cur[(16 * mb + n16) * KROW + 32 * ks + 8 * g]));
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) s[mb][nb] = mfma16x16x32(a, qb[nb][ks], s[mb][nb]);
            }

        // ---- online softmax, per lane = per query row
        const bool need_mask = (p.causal && tok0 + KT - 1 > w_first_abs) || tok0 + KT > p.n_cached;
        // Lazy rescale: a row's reference max m only moves (and its l, O^T are
        // rescaled) when the tile max exceeds it by more than 2^8, so p <= 256.
        // max over raw scores (scale >= 0), then p = exp2(s * scale*log2e - m), one fma
        const float c = p.scale_log2;
        float mx[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int qpos = qabs0 + q0 + 16 * nb + n16;
            float mr = -INFINITY;
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (need_mask) {
                        const int kpos = tok0 + 16 * mb + 4 * g + i;
                        if (kpos >= p.n_cached || (p.causal && kpos > qpos)) s[mb][nb][i] = -INFINITY;
                    }
                    mr = fmaxf(mr, s[mb][nb][i]);
                }
            mx[nb] = mr == -INFINITY ? -INFINITY : mr * c;  // this lane's 16 keys
        }
        // A lane's own keys decide whether any row may grow; the row max (two
        // cross-lane steps) is formed only then.
        bool any_lane = false;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) any_lane = any_lane || mx[nb] > m[nb] + 8.0f;
        if (__any(any_lane)) {
            float alpha[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                mx[nb] = fmaxf(mx[nb], __shfl_xor(mx[nb], 16));
                mx[nb] = fmaxf(mx[nb], __shfl_xor(mx[nb], 32));
                const bool grow = mx[nb] > m[nb] + 8.0f;
                const float mn = grow ? mx[nb] : m[nb];
                alpha[nb] = grow ? exp2_fast(m[nb] - mn) : 1.0f;
                l[nb] *= alpha[nb];
                m[nb] = mn;
            }
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) acc[db][nb] *= alpha[nb];
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const float mu = m[nb] == -INFINITY ? 0.0f : m[nb];
            float sum = 0.0f;
#pragma unroll
            for (int mb = 0; mb < 4; ++mb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float e = exp2_fast(__builtin_fmaf(s[mb][nb][i], c, -mu));
                    if (need_mask && s[mb][nb][i] == -INFINITY) e = 0.0f;  // also when scale == 0
                    s[mb][nb][i] = e;
                    sum += e;
                }
            l[nb] += sum;
        }

        // ---- O^T += V^T P^T
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            bf16x8_t pb[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const f32x4_t& x0 = s[2 * kt][nb];
                const f32x4_t& x1 = s[2 * kt + 1][nb];
                uint4 u;
                u.x = bf16_pair_rne(x0[0], x0[1]);
                u.y = bf16_pair_rne(x0[2], x0[3]);
                u.z = bf16_pair_rne(x1[0], x1[1]);
                u.w = bf16_pair_rne(x1[2], x1[3]);
                pb[nb] = as_bf16x8(u);
            }
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const uint16_t* vr = &v_cur[(16 * db + n16) * VROW + 32 * kt + 4 * g];
                const uint2 lo = *reinterpret_cast<const uint2*>(vr);
                const uint2 hi = *reinterpret_cast<const uint2*>(vr + 16);
                const bf16x8_t a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) acc[db][nb] = mfma16x16x32(a, pb[nb], acc[db][nb]);
            }
        }
    }

    if (!wave_has_rows) return;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        float lt = l[nb];
        lt += __shfl_xor(lt, 16);
        lt += __shfl_xor(lt, 32);
        const float inv = 1.0f / lt;
        const int s = q0 + 16 * nb + n16;
        if (s >= p.S) continue;
        uint16_t* orow = p.out + int64_t(hq) * p.o_head_stride + int64_t(s) * p.o_tok_stride;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const f32x4_t& a = acc[db][nb];
            uint2 w;
            w.x = pack2(f32_to_bf16_ref(a[0] * inv), f32_to_bf16_ref(a[1] * inv));
            w.y = pack2(f32_to_bf16_ref(a[2] * inv), f32_to_bf16_ref(a[3] * inv));
            *reinterpret_cast<uint2*>(orow + 16 * db + 4 * g) = w;
        }
    }
}

}  // namespace

int launch_paged_prefill(const AttnParams& p, int head_dim, hipStream_t stream) {
    if (head_dim != 128) return fail(GENLLM_ERR_UNSUPPORTED, "paged prefill: head_dim must be 128");
    if (p.S <= 0 || p.n_pages <= 0) return GENLLM_OK;
    constexpr int WAVES = 4, NB = kPrefillBlocks;
    const int64_t n_qt = (p.S + 16 * NB * WAVES - 1) / (16 * NB * WAVES);
    hipLaunchKernelGGL((paged_prefill_kernel<128, WAVES, NB>), dim3(unsigned(n_qt * p.Hq)), dim3(WAVES * 64), 0, stream,
                       p);
    GENLLM_LAUNCH_CHECK("paged_prefill_kernel");
    return GENLLM_OK;
}

}  // namespace genllm
