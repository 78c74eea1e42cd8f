// kv_cache.hip -- host side of the path: the kv_cache memory pool, the
// PagedAttentionManager / BlockPool state machine, and the C ABI entry points.
//
// Reference: include/core/page_attention.h:9-90, src/core/page_attention.cpp:25-216,
// src/core/pools.cpp:17-48 (bump allocator), src/backend/cpu/attention.cpp:123-216
// and src/backend/cuda/attention.cu:491-580 (the op).  Differences, by design:
//   * the device page table lives in HBM (allocated once, at reserve_layer)
//     and is updated incrementally (the CUDA op mallocs, copies and frees it
//     on every call);
//   * the K/V append is one kernel (the CUDA path issues 2*S*Hkv memcpys);
//   * a pool without free pages is an error that leaves the layer unchanged
//     (the reference breaks out of the loop but still advances num_cached).
#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace genllm {

// ------------------------------------------------------------------ errors
static thread_local std::string t_error;
void set_error(const std::string& msg) { t_error = msg; }
int fail(int code, const std::string& msg) {
    t_error = msg;
    return code;
}
int hip_fail(hipError_t e, const char* what) {
    return fail(GENLLM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

int device_cu_count() {
    // per device, resolved once (a decode call reads one atomic, no lock)
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (dev < 0 || dev >= 64) {
        int n = 0;
        return hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

// -------------------------------------------------------------- BlockPool
// page_attention.h:11-45 / page_attention.cpp:25-64
struct BlockPool {
    int32_t capacity = 0;    // 0 = unbounded
    int32_t num_blocks = 0;  // ids handed out so far (high-water mark)
    std::vector<int32_t> free_list;

    int32_t alloc() {
        if (!free_list.empty()) {
            const int32_t id = free_list.back();
            free_list.pop_back();
            return id;
        }
        if (capacity > 0 && num_blocks >= capacity) return -1;
        return num_blocks++;
    }
    // alloc() that reports whether the id came off the free list, so that
    // unalloc() can revert it: undone in reverse allocation order, the pool
    // is restored exactly (free-list order included).
    int32_t alloc(bool& from_free) {
        from_free = !free_list.empty();
        return alloc();
    }
    void unalloc(int32_t id, bool from_free) {
        if (from_free)
            free_list.push_back(id);
        else
            --num_blocks;
    }
    void free(int32_t id) {
        if (id >= 0 && id < num_blocks) free_list.push_back(id);
    }
    void reset() {
        free_list.clear();
        for (int32_t i = 0; i < num_blocks; ++i) free_list.push_back(i);
    }
    int64_t available() const {
        return int64_t(free_list.size()) + (capacity > 0 ? int64_t(capacity - num_blocks) : int64_t(INT32_MAX));
    }
};

// page_attention.h:57-66 plus the device-side resources of the layer
struct LayerState {
    bool active = false;
    int32_t num_cached = 0;
    int32_t n_kv_heads = 0, head_dim = 0, dtype = 0;
    BlockPool k_pool, v_pool;
    std::vector<int32_t> k_ids, v_ids;  // page table
    uint16_t* k_base = nullptr;
    uint16_t* v_base = nullptr;
    // Device page table: its own allocation (2 * max_blocks int32), outside
    // the kv_cache pool, so that the pool holds exactly the K and V pools the
    // scheduler sizes it for (scheduler.cpp:62-79).
    int32_t* d_k_ids = nullptr;
    int32_t* d_v_ids = nullptr;
    // Pinned host staging of the table ([max_blocks] K ids, then [max_blocks]
    // V ids): new entries are written here once and uploaded asynchronously,
    // so an append never waits on a pageable copy.  An entry is rewritten only
    // after reset / set_page_table, which first drain pending uploads.
    int32_t* h_ids = nullptr;
    int32_t max_blocks = 0;
    size_t block_bytes = 0;
    // Device-position decode (graph-capturable steps): the control block
    // {pos, limit, arrivals, error} follows the device page table.  Between
    // genllm_kv_stage_decode and genllm_kv_sync_decode the device owns the
    // position; num_cached and the tables then describe the end of the staged
    // window, and stage_k / stage_v list the blocks staging handed out (in
    // allocation order, with their free-list origin) so that the unused ones
    // can be given back exactly.
    int32_t* d_step = nullptr;
    bool staged = false;
    int32_t stage_num_cached = 0;
    size_t stage_table_size = 0;
    std::vector<std::pair<int32_t, bool>> stage_k, stage_v;
};

}  // namespace genllm

using namespace genllm;

struct genllm_kv {
    int32_t device = 0;
    char* base = nullptr;  // kv_cache MemoryPool buffer
    size_t capacity = 0, cursor = 0;
    std::map<int32_t, LayerState> layers;
    // Split-K decode workspace (arrival counters, then per-split partials),
    // sized by reserve_layer for the largest reserved layer and zero-filled
    // there; the op path never allocates, frees or synchronises.
    void* ws = nullptr;
    size_t ws_bytes = 0;
    std::vector<void*> pinned;     // every h_ids buffer, freed at destroy
    std::vector<void*> tables;     // every device page table, freed at destroy
    bool uploads_pending = false;  // async table uploads from h_ids may be in flight
};

namespace {

size_t elem_size(int32_t dtype) {
    switch (dtype) {
        case 0: return 4;   // F32
        case 1: return 2;   // F16
        case 30: return 2;  // BF16
        default: return 0;
    }
}

// MemoryPool::allocate (pools.cpp:17-48): aligned bump allocation.
int pool_allocate(genllm_kv* kv, size_t size, size_t align, void** out) {
    const size_t at = (kv->cursor + align - 1) & ~(align - 1);
    if (at + size > kv->capacity)
        return fail(GENLLM_ERR_NO_MEMORY, "kv_cache pool: out of memory, need " + std::to_string(size) +
                                              " bytes, remaining " + std::to_string(kv->capacity - std::min(at, kv->capacity)));
    *out = kv->base + at;
    kv->cursor = at + size;
    return GENLLM_OK;
}

int64_t pages_opened(int32_t num_cached, int32_t count) {
    // positions g in [num_cached, num_cached+count) with g % 16 == 0
    return (int64_t(num_cached) + count + kPage - 1) / kPage - (int64_t(num_cached) + kPage - 1) / kPage;
}

// What one append_pages call changed, so that a failure after it (a kernel
// launch error) can restore the layer exactly.
struct AppendUndo {
    int32_t num_cached = 0;
    size_t table_size = 0;
    std::vector<std::pair<int32_t, bool>> k, v;  // ids handed out, and whether from the free list
};

// append_kv_pages (page_attention.cpp:141-162) on the host state, in closed
// form: the positions g in [num_cached, num_cached + count) with g % 16 == 0
// are the page indices first .. first + need - 1; each takes one K and one V
// block, and enters the table only past its end (as the reference pushes).
// Every check runs before the state changes, so an error leaves the layer
// as it was.  New entries go to the device table either through `upd` (the
// next kernel writes them; when given and large enough) or with async copies
// on `stream` from the layer's pinned staging.
template <typename Upd = TableUpdate>
int append_pages(genllm_kv* kv, LayerState& s, int32_t count, hipStream_t stream, Upd* upd = nullptr,
                 AppendUndo* undo = nullptr) {
    constexpr size_t kCap = sizeof(Upd::k) / sizeof(int32_t);
    if (upd) *upd = Upd{};
    if (undo) {
        undo->num_cached = s.num_cached;
        undo->table_size = s.k_ids.size();
        undo->k.clear();
        undo->v.clear();
    }
    if (!s.active || count <= 0) return GENLLM_OK;
    if (int64_t(s.num_cached) + count > int64_t(INT32_MAX) - kPage)
        return fail(GENLLM_ERR_INVALID, "append_kv_pages: position overflow");
    const int64_t first = (int64_t(s.num_cached) + kPage - 1) / kPage;
    const int64_t need = pages_opened(s.num_cached, count);
    if (need > s.k_pool.available() || need > s.v_pool.available())
        return fail(GENLLM_ERR_POOL_FULL, "append_kv_pages: block pool exhausted (" + std::to_string(need) +
                                              " pages needed)");
    const size_t old_size = s.k_ids.size();
    if (need > 0 && first > int64_t(old_size))
        return fail(GENLLM_ERR_INVALID, "append_kv_pages: page table shorter than num_cached");
    const size_t new_size = std::max<size_t>(old_size, size_t(first + need));
    if (s.d_k_ids && new_size > size_t(s.max_blocks))
        return fail(GENLLM_ERR_POOL_FULL, "append_kv_pages: page table longer than max_blocks");
    for (int64_t i = 0; i < need; ++i) {
        bool kf = false, vf = false;
        const int32_t k = s.k_pool.alloc(kf);
        const int32_t v = s.v_pool.alloc(vf);
        if (undo) {
            undo->k.emplace_back(k, kf);
            undo->v.emplace_back(v, vf);
        }
        if (first + i >= int64_t(s.k_ids.size())) {
            s.k_ids.push_back(k);
            s.v_ids.push_back(v);
        }
    }
    s.num_cached += count;
    if (new_size > old_size && s.d_k_ids) {
        const size_t n = new_size - old_size;
        if (upd && n <= kCap) {
            upd->first = int32_t(old_size);
            upd->count = int32_t(n);
            for (size_t i = 0; i < n; ++i) {
                upd->k[i] = s.k_ids[old_size + i];
                upd->v[i] = s.v_ids[old_size + i];
            }
        } else {
            int32_t* hk = s.h_ids + old_size;
            int32_t* hv = s.h_ids + s.max_blocks + old_size;
            std::copy(s.k_ids.begin() + old_size, s.k_ids.end(), hk);
            std::copy(s.v_ids.begin() + old_size, s.v_ids.end(), hv);
            kv->uploads_pending = true;
            GENLLM_HIP_TRY(hipMemcpyAsync(s.d_k_ids + old_size, hk, n * sizeof(int32_t), hipMemcpyHostToDevice, stream));
            GENLLM_HIP_TRY(hipMemcpyAsync(s.d_v_ids + old_size, hv, n * sizeof(int32_t), hipMemcpyHostToDevice, stream));
        }
    }
    return GENLLM_OK;
}

// Restores the layer to its state before the append_pages call `u` recorded.
void undo_append(LayerState& s, const AppendUndo& u) {
    for (size_t i = u.k.size(); i-- > 0;) {
        s.k_pool.unalloc(u.k[i].first, u.k[i].second);
        s.v_pool.unalloc(u.v[i].first, u.v[i].second);
    }
    s.k_ids.resize(u.table_size);
    s.v_ids.resize(u.table_size);
    s.num_cached = u.num_cached;
}

// Per-thread undo record (its vectors keep their capacity across calls).
thread_local AppendUndo t_undo;

LayerState* active_layer(genllm_kv* kv, int32_t layer) {
    auto it = kv->layers.find(layer);
    if (it == kv->layers.end() || !it->second.active) return nullptr;
    return &it->second;
}

// Host-driven changes of a layer whose position the device owns would break
// the exact rewind of genllm_kv_sync_decode: they are refused until then.
int refuse_staged(const LayerState& s, const char* what) {
    return s.staged ? fail(GENLLM_ERR_INVALID, std::string(what) +
                                                   ": the layer is staged for device-position decode "
                                                   "(call genllm_kv_sync_decode first)")
                    : GENLLM_OK;
}

// Writes the device-position control block: limit always; when `enter`,
// also the position, with the arrival counter and the error flag cleared.
// A kernel, not a memset or copy, so it needs no host buffer to outlive it.
__global__ void set_step_kernel(int32_t* ctl, int32_t pos, int32_t limit, int32_t enter) {
    if (threadIdx.x != 0) return;
    if (enter) {
        ctl[kStepPos] = pos;
        ctl[kStepArrivals] = 0;
        ctl[kStepError] = 0;
    }
    ctl[kStepLimit] = limit;
}

// Split-K workspace of the manager, grown at set-up only (reserve_layer) to
// the largest decode plan any reserved layer can make: 16 rows per kv head
// (the decode kernel's limit) and as many splits as the layer's max_blocks
// allow.  The new buffer is zero-filled: its arrival counters must start at
// zero, and the kernels leave them at zero.
int reserve_workspace(genllm_kv* kv, size_t need) {
    if (need <= kv->ws_bytes) return GENLLM_OK;
    GENLLM_HIP_TRY(hipSetDevice(kv->device));
    if (kv->ws) {
        GENLLM_HIP_TRY(hipDeviceSynchronize());  // the old buffer may still be in use
        GENLLM_HIP_TRY(hipFree(kv->ws));
        kv->ws = nullptr;
        kv->ws_bytes = 0;
    }
    GENLLM_HIP_TRY(hipMalloc(&kv->ws, need));
    kv->ws_bytes = need;
    GENLLM_HIP_TRY(hipMemset(kv->ws, 0, need));
    return GENLLM_OK;
}

// Waits for async table uploads that read the pinned staging.
int drain_uploads(genllm_kv* kv) {
    if (!kv->uploads_pending) return GENLLM_OK;
    GENLLM_HIP_TRY(hipSetDevice(kv->device));
    GENLLM_HIP_TRY(hipDeviceSynchronize());
    kv->uploads_pending = false;
    return GENLLM_OK;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int check_attn_args(const AttnParams& p, int head_dim) {
    if (!p.q || !p.out || !p.k_pool || !p.v_pool || !p.k_ids || !p.v_ids)
        return fail(GENLLM_ERR_INVALID, "paged attention: null pointer");
    if (head_dim != 128 && head_dim != 256)
        return fail(GENLLM_ERR_UNSUPPORTED, "paged attention requires head_dim 128 or 256");
    if (p.Hkv <= 0 || p.Hq <= 0 || p.Hq % p.Hkv != 0)
        return fail(GENLLM_ERR_INVALID, "paged attention: n_q_heads must be a multiple of n_kv_heads");
    if (p.S <= 0 || p.n_cached < p.S || p.n_pages < (p.n_cached + kPage - 1) / kPage)
        return fail(GENLLM_ERR_INVALID, "paged attention: need 0 < seq_len <= n_cached <= 16 * n_pages");
    // OpFactory::Attention replaces a negative scale by 1/sqrt(head_dim) (op_factory.hpp:467),
    // so the op never sees one; the kernels rely on scale >= 0.
    if (!(p.scale_log2 >= 0.0f) || p.scale_log2 == INFINITY)
        return fail(GENLLM_ERR_INVALID, "paged attention: scale must be finite and >= 0");
    if (!aligned(p.q, 16) || !aligned(p.k_pool, 16) || !aligned(p.v_pool, 16) || !aligned(p.out, 8) ||
        (p.q_head_stride % 8) || (p.q_tok_stride % 8) || (p.o_head_stride % 4) || (p.o_tok_stride % 4))
        return fail(GENLLM_ERR_INVALID, "paged attention: q/pools must be 16-byte aligned, strides multiples of 8");
    return GENLLM_OK;
}

// Short query chunks (<= 16 rows per kv head) take the split-K decode kernel
// on the manager's workspace (reserve_layer sized it for every plan a reserved
// layer can make); longer chunks take the MFMA prefill kernel.  Checks and the
// split plan come first, so a caller can run them before changing any state.
int prepare_attention(AttnParams& p, int head_dim, genllm_kv* kv) {
    if (int rc = check_attn_args(p, head_dim)) return rc;
    if (p.G * p.S <= 16) return decode_plan(p, head_dim, kv->ws_bytes, kv->ws);
    return GENLLM_OK;
}

int launch_attention(const AttnParams& p, int head_dim, hipStream_t stream) {
    if (p.G * p.S <= 16) return launch_paged_decode(p, head_dim, stream);
    return launch_paged_prefill(p, head_dim, stream);
}

}  // namespace

// ====================================================================== C ABI

extern "C" const char* genllm_last_error(void) { return t_error.c_str(); }

extern "C" int genllm_kv_create(int32_t device, size_t kv_pool_bytes, genllm_kv** out) {
    if (!out) return fail(GENLLM_ERR_INVALID, "kv_create: null out");
    *out = nullptr;
    GENLLM_HIP_TRY(hipSetDevice(device));
    genllm_kv* kv = new genllm_kv;
    kv->device = device;
    kv->capacity = kv_pool_bytes;
    if (kv_pool_bytes > 0) {
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, kv_pool_bytes);
        if (e != hipSuccess) {
            delete kv;
            return fail(GENLLM_ERR_NO_MEMORY, std::string("kv_create: hipMalloc failed: ") + hipGetErrorString(e));
        }
        // pools start zeroed, as the reference's CPU pools (resource_cpu.cpp:43)
        e = hipMemset(p, 0, kv_pool_bytes);
        if (e != hipSuccess) {
            (void)hipFree(p);
            delete kv;
            return hip_fail(e, "kv_create: hipMemset");
        }
        kv->base = static_cast<char*>(p);
    }
    *out = kv;
    return GENLLM_OK;
}

extern "C" int genllm_kv_destroy(genllm_kv* kv) {
    if (!kv) return GENLLM_OK;
    (void)hipSetDevice(kv->device);
    (void)hipDeviceSynchronize();
    if (kv->base) (void)hipFree(kv->base);
    if (kv->ws) (void)hipFree(kv->ws);
    for (void* t : kv->tables) (void)hipFree(t);
    for (void* h : kv->pinned) (void)hipHostFree(h);
    delete kv;
    return GENLLM_OK;
}

extern "C" int genllm_kv_init_layer(genllm_kv* kv, int32_t layer, int32_t n_kv_heads, int32_t head_dim,
                                    int32_t dtype) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "init_layer: null kv");
    if (n_kv_heads <= 0 || head_dim <= 0 || elem_size(dtype) == 0)
        return fail(GENLLM_ERR_INVALID, "init_layer: bad n_kv_heads/head_dim/dtype");
    LayerState& s = kv->layers[layer];
    s.n_kv_heads = n_kv_heads;
    s.head_dim = head_dim;
    s.dtype = dtype;
    s.active = true;
    s.num_cached = 0;
    s.staged = false;
    return GENLLM_OK;
}

extern "C" int genllm_kv_reserve_layer(genllm_kv* kv, int32_t layer, int32_t max_blocks) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "reserve_layer: null kv");
    if (max_blocks <= 0) return fail(GENLLM_ERR_INVALID, "reserve_layer: max_blocks must be > 0");
    LayerState& s = kv->layers[layer];
    if (!s.active || !kv->base) return GENLLM_OK;  // page_attention.cpp:84
    const size_t bb = size_t(kPage) * s.n_kv_heads * s.head_dim * elem_size(s.dtype);
    const size_t total = size_t(max_blocks) * bb;
    // The pool holds exactly the K and V pools (2 * max_blocks * block_bytes,
    // the scheduler's sizing, scheduler.cpp:62-79 and 371); the device page
    // table, its pinned staging and the decode workspace are allocated
    // separately, once, here.
    // The decode workspace grows (a new buffer) only while no layer is staged:
    // a captured device-position step holds the current buffer's address.
    // Checked first, so that a refusal changes nothing.
    const int rows = 16;  // decode kernel limit: (query, q-head) rows per kv head
    const size_t ws_need = decode_workspace_bytes(rows * s.n_kv_heads, s.n_kv_heads, 1, s.head_dim, max_blocks);
    if (ws_need > kv->ws_bytes)
        for (const auto& kvp : kv->layers)
            if (kvp.second.active && kvp.second.staged)
                return fail(GENLLM_ERR_INVALID,
                            "reserve_layer: this layer needs a larger decode workspace, which cannot be replaced "
                            "while layer " + std::to_string(kvp.first) + " is staged (reserve every layer first)");
    const size_t cursor0 = kv->cursor;
    void *kp, *vp;
    if (int rc = pool_allocate(kv, total, 256, &kp)) return rc;
    if (int rc = pool_allocate(kv, total, 256, &vp)) {
        kv->cursor = cursor0;
        return rc;
    }
    GENLLM_HIP_TRY(hipSetDevice(kv->device));
    void* table = nullptr;
    void* staging = nullptr;
    const size_t table_bytes = (size_t(max_blocks) * 2 + kStepInts) * sizeof(int32_t);
    hipError_t e = hipMalloc(&table, table_bytes);
    if (e == hipSuccess) e = hipMemset(table, 0, table_bytes);
    if (e == hipSuccess) e = hipHostMalloc(&staging, size_t(max_blocks) * 2 * sizeof(int32_t), hipHostMallocDefault);
    if (e != hipSuccess) {
        if (table) (void)hipFree(table);
        kv->cursor = cursor0;
        return hip_fail(e, "reserve_layer: page table allocation");
    }
    if (int rc = reserve_workspace(kv, ws_need)) {  // nothing of this call is kept
        (void)hipFree(table);
        (void)hipHostFree(staging);
        kv->cursor = cursor0;
        return rc;
    }
    kv->tables.push_back(table);
    kv->pinned.push_back(staging);
    s.h_ids = static_cast<int32_t*>(staging);
    s.k_base = static_cast<uint16_t*>(kp);
    s.v_base = static_cast<uint16_t*>(vp);
    s.d_k_ids = static_cast<int32_t*>(table);
    s.d_v_ids = static_cast<int32_t*>(table) + max_blocks;
    s.d_step = static_cast<int32_t*>(table) + 2 * size_t(max_blocks);
    s.staged = false;
    s.block_bytes = bb;
    s.max_blocks = max_blocks;
    s.k_pool = BlockPool{};
    s.v_pool = BlockPool{};
    s.k_pool.capacity = max_blocks;
    s.v_pool.capacity = max_blocks;
    return GENLLM_OK;
}

extern "C" int genllm_kv_is_active(genllm_kv* kv, int32_t layer, int32_t* active) {
    if (!kv || !active) return fail(GENLLM_ERR_INVALID, "is_active: null pointer");
    *active = active_layer(kv, layer) != nullptr;
    return GENLLM_OK;
}

extern "C" int genllm_kv_append_pages(genllm_kv* kv, int32_t layer, int32_t count, void* stream) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "append_pages: null kv");
    LayerState& s = kv->layers[layer];
    if (int rc = refuse_staged(s, "append_pages")) return rc;
    return append_pages<TableUpdate>(kv, s, count, as_stream(stream), nullptr);
}

extern "C" int genllm_kv_reset(genllm_kv* kv) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "reset: null kv");
    if (int rc = drain_uploads(kv)) return rc;  // staged entries are about to be reused
    for (auto& [id, s] : kv->layers) {
        s.num_cached = 0;
        s.k_ids.clear();
        s.v_ids.clear();
        s.k_pool.reset();
        s.v_pool.reset();
        s.staged = false;  // the device position is re-uploaded by the next staging
        s.stage_k.clear();
        s.stage_v.clear();
    }
    return GENLLM_OK;
}

extern "C" int genllm_kv_layer_info(genllm_kv* kv, int32_t layer, genllm_layer_info* out) {
    if (!kv || !out) return fail(GENLLM_ERR_INVALID, "layer_info: null pointer");
    std::memset(out, 0, sizeof *out);
    auto it = kv->layers.find(layer);
    if (it == kv->layers.end()) return GENLLM_OK;
    const LayerState& s = it->second;
    out->active = s.active;
    out->num_cached = s.num_cached;
    out->num_pages = int32_t(s.k_ids.size());
    out->n_kv_heads = s.n_kv_heads;
    out->head_dim = s.head_dim;
    out->dtype = s.dtype;
    out->max_blocks = s.max_blocks;
    out->k_num_blocks = s.k_pool.num_blocks;
    out->k_num_free = int32_t(s.k_pool.free_list.size());
    out->v_num_blocks = s.v_pool.num_blocks;
    out->v_num_free = int32_t(s.v_pool.free_list.size());
    out->k_pool = s.k_base;
    out->v_pool = s.v_base;
    out->k_ids = s.d_k_ids;
    out->v_ids = s.d_v_ids;
    out->block_bytes = s.block_bytes;
    return GENLLM_OK;
}

extern "C" int genllm_kv_page_table(genllm_kv* kv, int32_t layer, int32_t* k_ids, int32_t* v_ids, int32_t cap,
                                    int32_t* n) {
    if (!kv || !n) return fail(GENLLM_ERR_INVALID, "page_table: null pointer");
    auto it = kv->layers.find(layer);
    *n = 0;
    if (it == kv->layers.end()) return GENLLM_OK;
    const LayerState& s = it->second;
    *n = int32_t(s.k_ids.size());
    for (int32_t i = 0; i < *n && i < cap; ++i) {
        if (k_ids) k_ids[i] = s.k_ids[i];
        if (v_ids) v_ids[i] = s.v_ids[i];
    }
    return GENLLM_OK;
}

extern "C" int genllm_kv_set_page_table(genllm_kv* kv, int32_t layer, const int32_t* k_ids, const int32_t* v_ids,
                                        int32_t n, int32_t num_cached, void* stream) {
    if (!kv || (n > 0 && (!k_ids || !v_ids))) return fail(GENLLM_ERR_INVALID, "set_page_table: null pointer");
    LayerState* s = active_layer(kv, layer);
    if (!s) return fail(GENLLM_ERR_INVALID, "set_page_table: layer not active");
    if (int rc = refuse_staged(*s, "set_page_table")) return rc;
    if (n < 0 || num_cached < 0 || (s->max_blocks > 0 && n > s->max_blocks) || int64_t(num_cached) > int64_t(n) * kPage)
        return fail(GENLLM_ERR_INVALID, "set_page_table: bad length or num_cached");
    for (int32_t i = 0; i < n; ++i)
        if (k_ids[i] < 0 || k_ids[i] >= s->k_pool.num_blocks || v_ids[i] < 0 || v_ids[i] >= s->v_pool.num_blocks)
            return fail(GENLLM_ERR_INVALID, "set_page_table: id was never handed out by its pool");
    if (int rc = drain_uploads(kv)) return rc;  // later appends rewrite staged entries
    s->k_ids.assign(k_ids, k_ids + n);
    s->v_ids.assign(v_ids, v_ids + n);
    s->num_cached = num_cached;
    if (n > 0 && s->d_k_ids) {
        GENLLM_HIP_TRY(hipMemcpyAsync(s->d_k_ids, s->k_ids.data(), size_t(n) * 4, hipMemcpyHostToDevice,
                                      as_stream(stream)));
        GENLLM_HIP_TRY(hipMemcpyAsync(s->d_v_ids, s->v_ids.data(), size_t(n) * 4, hipMemcpyHostToDevice,
                                      as_stream(stream)));
        GENLLM_HIP_TRY(hipStreamSynchronize(as_stream(stream)));  // host vectors may be reassigned next
    }
    return GENLLM_OK;
}

extern "C" int genllm_kv_block_alloc(genllm_kv* kv, int32_t layer, int32_t which, int32_t* id) {
    if (!kv || !id) return fail(GENLLM_ERR_INVALID, "block_alloc: null pointer");
    LayerState& s = kv->layers[layer];
    if (int rc = refuse_staged(s, "block_alloc")) return rc;
    *id = (which ? s.v_pool : s.k_pool).alloc();
    return GENLLM_OK;
}

extern "C" int genllm_kv_block_free(genllm_kv* kv, int32_t layer, int32_t which, int32_t id) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "block_free: null kv");
    LayerState& s = kv->layers[layer];
    if (int rc = refuse_staged(s, "block_free")) return rc;
    (which ? s.v_pool : s.k_pool).free(id);
    return GENLLM_OK;
}

// ------------------------------------------------------------------ the op
namespace {

// Argument checks of the op and its attention parameters for a layer holding
// n_after tokens once this call's seq_len tokens are appended.
int op_params(const LayerState& s, const void* q, const void* k, const void* v, void* out, int32_t batch,
              int32_t n_q_heads, int32_t seq_len, int32_t head_dim, int32_t n_kv_heads, int32_t n_kv_groups,
              float scale, int32_t causal, int32_t n_after, AttnParams& p) {
    if (head_dim != 128 && head_dim != 256)
        return fail(GENLLM_ERR_UNSUPPORTED, "paged_attention requires head_dim 128 or 256");
    if (batch < 1) return fail(GENLLM_ERR_INVALID, "paged_attention: batch must be >= 1");
    if (s.dtype != GENLLM_DTYPE_BF16 && s.dtype != GENLLM_DTYPE_F16)
        return fail(GENLLM_ERR_UNSUPPORTED, "paged_attention: layer dtype must be bf16 or f16");
    if (s.head_dim != head_dim || s.n_kv_heads != n_kv_heads)
        return fail(GENLLM_ERR_INVALID, "paged_attention: tensor shape differs from the layer's pools");
    if (n_kv_groups <= 0 || n_q_heads != n_kv_heads * n_kv_groups)
        return fail(GENLLM_ERR_INVALID, "paged_attention: n_q_heads must equal n_kv_heads * n_kv_groups");
    if (!q || !k || !v || !out) return fail(GENLLM_ERR_INVALID, "paged_attention: null tensor");
    if (!s.k_base) return fail(GENLLM_ERR_INVALID, "paged_attention: layer has no reserved pools");
    if (!aligned(k, 16) || !aligned(v, 16))
        return fail(GENLLM_ERR_INVALID, "paged_attention: k/v must be 16-byte aligned");
    p = AttnParams{};
    p.q = static_cast<const uint16_t*>(q);
    p.q_head_stride = int64_t(seq_len) * head_dim;
    p.q_tok_stride = head_dim;
    p.out = static_cast<uint16_t*>(out);
    p.o_head_stride = int64_t(seq_len) * head_dim;
    p.o_tok_stride = head_dim;
    p.k_pool = s.k_base;
    p.v_pool = s.v_base;
    p.k_ids = s.d_k_ids;
    p.v_ids = s.d_v_ids;
    p.n_cached = n_after;
    p.n_pages = (n_after + kPage - 1) / kPage;
    p.S = seq_len;
    p.Hq = n_q_heads;
    p.Hkv = n_kv_heads;
    p.G = n_kv_groups;
    p.scale_log2 = scale * kLog2e;
    p.causal = causal != 0;
    p.f16 = s.dtype == GENLLM_DTYPE_F16;
    p.page_elems = int64_t(kPage) * n_kv_heads * head_dim;
    p.kv_row = int64_t(n_kv_heads) * head_dim;
    return GENLLM_OK;
}

// The decode kernel's fused append: new rows (head-major [Hkv][S][D]) come
// from k / v and are written to the pools by the waves that read their pages.
void fuse_append(AttnParams& p, const LayerState& s, const void* k, const void* v, int32_t seq_len,
                 int32_t head_dim, int32_t new_from) {
    p.k_new = static_cast<const uint16_t*>(k);
    p.v_new = static_cast<const uint16_t*>(v);
    p.new_head_stride = int64_t(seq_len) * head_dim;
    p.new_tok_stride = head_dim;
    p.new_from = new_from;
    p.k_pool_w = s.k_base;
    p.v_pool_w = s.v_base;
    p.k_ids_w = s.d_k_ids;
    p.v_ids_w = s.d_v_ids;
}

}  // namespace

extern "C" int genllm_paged_attention(genllm_kv* kv, int32_t layer, const void* q, const void* k, const void* v,
                                      void* out, int32_t batch, int32_t n_q_heads, int32_t seq_len,
                                      int32_t head_dim, int32_t n_kv_heads, int32_t n_kv_groups, float scale,
                                      int32_t causal, void* stream) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "paged_attention: null kv");
    LayerState* s = active_layer(kv, layer);
    if (!s) return GENLLM_OK;  // attention.cpp:127: inactive layer, nothing written
    if (int rc = refuse_staged(*s, "paged_attention")) return rc;
    if (seq_len <= 0) {
        AttnParams unused;
        return op_params(*s, q, k, v, out, batch, n_q_heads, 1, head_dim, n_kv_heads, n_kv_groups, scale, causal,
                         1, unused);
    }
    hipStream_t st = as_stream(stream);
    const int32_t pos0 = s->num_cached;
    if (int64_t(pos0) + seq_len > int64_t(INT32_MAX) - kPage)
        return fail(GENLLM_ERR_INVALID, "paged_attention: position overflow");
    const int32_t n_after = pos0 + seq_len;
    const bool fuse = int64_t(n_kv_groups) * seq_len <= 16;

    // 0. attention arguments and split plan for the state after the append,
    // checked before anything changes: an error leaves the layer as it was
    AttnParams p;
    if (int rc = op_params(*s, q, k, v, out, batch, n_q_heads, seq_len, head_dim, n_kv_heads, n_kv_groups, scale,
                           causal, n_after, p))
        return rc;
    if (int rc = prepare_attention(p, head_dim, kv)) return rc;

    // 1. append (append_kv_from_tensor, attention.cpp:146): head-major [Hkv][S][D].
    // Short chunks (the decode kernel's range) append inside the attention
    // kernel itself: the wave that reads a page takes the new rows from k/v and
    // writes them to their slots, so no separate launch is needed.
    AppendParams ap;
    AppendUndo& undo = t_undo;
    if (int rc = append_pages(kv, *s, seq_len, st, &ap.upd, &undo)) return rc;
    ap.k = static_cast<const uint16_t*>(k);
    ap.v = static_cast<const uint16_t*>(v);
    ap.k_tok_stride = ap.v_tok_stride = head_dim;
    ap.k_head_stride = ap.v_head_stride = int64_t(seq_len) * head_dim;
    ap.S = seq_len;
    ap.Hkv = n_kv_heads;
    ap.pos0 = pos0;
    ap.nkv_tasks = (n_kv_heads + 7) / 8;
    ap.k_pool = s->k_base;
    ap.v_pool = s->v_base;
    ap.page_elems = int64_t(kPage) * n_kv_heads * head_dim;
    ap.k_ids = s->d_k_ids;
    ap.v_ids = s->d_v_ids;
    ap.max_blocks = s->max_blocks;
    if (!fuse) {
        if (int rc = launch_kv_append(ap, head_dim, st)) {
            undo_append(*s, undo);
            return rc;
        }
    }

    // 2. attend over all cached tokens
    if (fuse) {
        fuse_append(p, *s, k, v, seq_len, head_dim, pos0);
        // seq_len <= 16 opens at most 2 pages, which fit the launch arguments
        // (append_pages put them in ap.upd, as it holds up to 256)
        static_assert(sizeof(p.upd.k) / sizeof(int32_t) >= 2, "decode step opens up to 2 pages");
        p.upd.first = ap.upd.first;
        p.upd.count = ap.upd.count;
        for (int32_t i = 0; i < ap.upd.count; ++i) {
            p.upd.k[i] = ap.upd.k[i];
            p.upd.v[i] = ap.upd.v[i];
        }
    }
    if (int rc = launch_attention(p, head_dim, st)) {
        if (fuse) undo_append(*s, undo);  // nothing ran: the fused append is part of this launch
        return rc;
    }
    // 3. batch entries after the first attend over the same cache
    // (attention.cpp:156: the loop over b reads one page table; the append
    // above took the first entry's K/V rows, as append_kv_from_tensor reads
    // K->data for n_kv_heads x seq_len rows): attention only, after the first
    // entry's launch has written the new rows and page ids.
    if (batch > 1) {
        AttnParams pb = p;
        pb.k_new = pb.v_new = nullptr;
        pb.new_from = INT32_MAX;
        pb.upd.count = 0;
        const int64_t entry = int64_t(n_q_heads) * seq_len * head_dim;
        for (int32_t b = 1; b < batch; ++b) {
            pb.q = p.q + b * entry;
            pb.out = p.out + b * entry;
            if (int rc = launch_attention(pb, head_dim, st)) return rc;
        }
    }
    return GENLLM_OK;
}

// ------------------------------------------------ device-position decode
// The reference's decode loop (src/core/executor.cpp:227-236) advances the
// position every step, and each step's append opens a page whenever the
// position crosses a multiple of 16 (append_kv_pages, page_attention.cpp:
// 141-162).  For a step captured once into a HIP graph and replayed, both
// move to the device: staging opens, ahead of time and in the order the steps
// would, the pages of a window of future tokens; the step reads the position
// from the layer's control block and its last workgroup advances it; sync
// reads it back and returns the staged pages no step reached.

extern "C" int genllm_kv_stage_decode(genllm_kv* kv, int32_t layer, int32_t n_tokens, void* stream) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "stage_decode: null kv");
    LayerState* s = active_layer(kv, layer);
    if (!s) return fail(GENLLM_ERR_INVALID, "stage_decode: layer not active");
    if (!s->d_step) return fail(GENLLM_ERR_INVALID, "stage_decode: layer has no reserved pools");
    if (n_tokens < 0) return fail(GENLLM_ERR_INVALID, "stage_decode: n_tokens must be >= 0");
    hipStream_t st = as_stream(stream);
    const bool enter = !s->staged;
    const int32_t pos = s->num_cached;
    const size_t table0 = s->k_ids.size();
    AppendUndo& undo = t_undo;
    if (int rc = append_pages(kv, *s, n_tokens, st, static_cast<TableUpdate*>(nullptr), &undo)) return rc;
    GENLLM_HIP_TRY(hipSetDevice(kv->device));
    hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(64), 0, st, s->d_step, pos, s->num_cached, int32_t(enter));
    if (hipError_t e = hipGetLastError(); e != hipSuccess) {
        undo_append(*s, undo);
        return hip_fail(e, "stage_decode: set_step_kernel");
    }
    if (enter) {
        s->staged = true;
        s->stage_num_cached = pos;
        s->stage_table_size = table0;
        s->stage_k.clear();
        s->stage_v.clear();
    }
    s->stage_k.insert(s->stage_k.end(), undo.k.begin(), undo.k.end());
    s->stage_v.insert(s->stage_v.end(), undo.v.begin(), undo.v.end());
    return GENLLM_OK;
}

extern "C" int genllm_kv_sync_decode(genllm_kv* kv, int32_t layer, void* stream, int32_t* num_cached) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "sync_decode: null kv");
    LayerState* s = active_layer(kv, layer);
    if (!s) return fail(GENLLM_ERR_INVALID, "sync_decode: layer not active");
    if (!s->staged) {
        if (num_cached) *num_cached = s->num_cached;
        return GENLLM_OK;
    }
    hipStream_t st = as_stream(stream);
    GENLLM_HIP_TRY(hipSetDevice(kv->device));
    int32_t ctl[kStepInts] = {};
    GENLLM_HIP_TRY(hipMemcpyAsync(ctl, s->d_step, sizeof ctl, hipMemcpyDeviceToHost, st));
    GENLLM_HIP_TRY(hipStreamSynchronize(st));
    const int32_t pos = ctl[kStepPos];
    if (pos < s->stage_num_cached || pos > s->num_cached)
        return fail(GENLLM_ERR_INVALID, "sync_decode: device position " + std::to_string(pos) +
                                             " outside the staged window [" + std::to_string(s->stage_num_cached) +
                                             ", " + std::to_string(s->num_cached) + "]");
    // Staging handed out one K and one V block per page the window opens, in
    // position order.  The steps that ran used the first `used`; the rest go
    // back in reverse order, which restores the pools exactly, and the table
    // keeps the entries the reference's appends up to `pos` would have pushed.
    const int64_t used = pages_opened(s->stage_num_cached, pos - s->stage_num_cached);
    for (size_t i = s->stage_k.size(); i-- > size_t(used);) {
        s->k_pool.unalloc(s->stage_k[i].first, s->stage_k[i].second);
        s->v_pool.unalloc(s->stage_v[i].first, s->stage_v[i].second);
    }
    const size_t first = size_t((int64_t(s->stage_num_cached) + kPage - 1) / kPage);
    const size_t keep = std::max(s->stage_table_size, first + size_t(used));
    if (keep < s->k_ids.size()) {
        s->k_ids.resize(keep);
        s->v_ids.resize(keep);
    }
    s->num_cached = pos;
    s->staged = false;
    s->stage_k.clear();
    s->stage_v.clear();
    if (num_cached) *num_cached = pos;
    hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(64), 0, st, s->d_step, pos, pos, 1);
    GENLLM_LAUNCH_CHECK("set_step_kernel");
    if (ctl[kStepError])
        return fail(GENLLM_ERR_POOL_FULL, "decode step: a step at position " + std::to_string(pos) +
                                              " would pass the staged window; it and the steps after it did "
                                              "nothing (the layer now holds " + std::to_string(pos) + " tokens)");
    return GENLLM_OK;
}

extern "C" int genllm_paged_attention_step(genllm_kv* kv, int32_t layer, const void* q, const void* k,
                                           const void* v, void* out, int32_t batch, int32_t n_q_heads,
                                           int32_t seq_len, int32_t head_dim, int32_t n_kv_heads,
                                           int32_t n_kv_groups, float scale, int32_t causal, void* stream) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "paged_attention_step: null kv");
    LayerState* s = active_layer(kv, layer);
    if (!s) return GENLLM_OK;  // attention.cpp:127
    if (!s->staged) return fail(GENLLM_ERR_INVALID, "paged_attention_step: layer not staged (genllm_kv_stage_decode)");
    if (seq_len <= 0 || int64_t(n_kv_groups) * seq_len > 16)
        return fail(GENLLM_ERR_UNSUPPORTED, "paged_attention_step: seq_len * n_kv_groups must be in [1, 16]");
    if (batch != 1) return fail(GENLLM_ERR_UNSUPPORTED, "paged_attention_step: batch must be 1");
    // Planned for the end of the staged window: the grid covers every page a
    // step inside it can reach; splits past a step's last page are empty.
    const int32_t window_end = std::max(s->num_cached, seq_len);
    AttnParams p;
    if (int rc = op_params(*s, q, k, v, out, batch, n_q_heads, seq_len, head_dim, n_kv_heads, n_kv_groups, scale,
                           causal, window_end, p))
        return rc;
    p.step = s->d_step;
    if (int rc = prepare_attention(p, head_dim, kv)) return rc;
    fuse_append(p, *s, k, v, seq_len, head_dim, 0);
    return launch_attention(p, head_dim, as_stream(stream));
}


extern "C" int genllm_qk_norm_rope_append(genllm_kv* kv, int32_t layer, int32_t seq_len, const void* k,
                                          int64_t k_tok_stride, int64_t k_head_stride, const void* v,
                                          int64_t v_tok_stride, int64_t v_head_stride, const float* gamma_k,
                                          const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                          int32_t n_q_heads, const float* gamma_q, void* q_out,
                                          int64_t qo_tok_stride, int64_t qo_head_stride, float eps,
                                          const float* cos_tab, const float* sin_tab, int32_t rope_dim,
                                          int64_t rope_pos0, void* stream) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "qk_norm_rope_append: null kv");
    LayerState* s = active_layer(kv, layer);
    if (!s) return GENLLM_OK;
    if (int rc = refuse_staged(*s, "qk_norm_rope_append")) return rc;
    if (!s->k_base) return fail(GENLLM_ERR_INVALID, "qk_norm_rope_append: layer has no reserved pools");
    const int D = s->head_dim;
    if (D != 64 && D != 128 && D != 256) return fail(GENLLM_ERR_UNSUPPORTED, "qk_norm_rope_append: head_dim");
    if (s->dtype != GENLLM_DTYPE_BF16) return fail(GENLLM_ERR_UNSUPPORTED, "qk_norm_rope_append: bf16 only");
    if (seq_len <= 0) return GENLLM_OK;
    if (!k || !v) return fail(GENLLM_ERR_INVALID, "qk_norm_rope_append: null k/v");
    if ((cos_tab == nullptr) != (sin_tab == nullptr))
        return fail(GENLLM_ERR_INVALID, "qk_norm_rope_append: cos and sin tables go together");
    if (cos_tab && (rope_dim <= 0 || rope_dim > D || rope_dim % 64))
        return fail(GENLLM_ERR_UNSUPPORTED, "qk_norm_rope_append: rope_dim must be a multiple of 64, at most head_dim");
    if (q && (!q_out || n_q_heads <= 0)) return fail(GENLLM_ERR_INVALID, "qk_norm_rope_append: q needs q_out");
    if (!aligned(k, 8) || !aligned(v, 16) || (k_tok_stride % 4) || (k_head_stride % 4) || (v_tok_stride % 8) ||
        (v_head_stride % 8) || (q && (!aligned(q, 8) || !aligned(q_out, 8) || (q_tok_stride % 4) ||
                                      (q_head_stride % 4) || (qo_tok_stride % 4) || (qo_head_stride % 4))) ||
        (gamma_k && !aligned(gamma_k, 16)) || (gamma_q && !aligned(gamma_q, 16)) ||
        (cos_tab && (!aligned(cos_tab, 16) || !aligned(sin_tab, 16))))
        return fail(GENLLM_ERR_INVALID, "qk_norm_rope_append: misaligned pointer or stride");
    hipStream_t st = as_stream(stream);
    AppendParams ap;
    const int32_t pos0 = s->num_cached;
    AppendUndo& undo = t_undo;
    if (int rc = append_pages(kv, *s, seq_len, st, &ap.upd, &undo)) return rc;
    ap.k = static_cast<const uint16_t*>(k);
    ap.k_tok_stride = k_tok_stride;
    ap.k_head_stride = k_head_stride;
    ap.v = static_cast<const uint16_t*>(v);
    ap.v_tok_stride = v_tok_stride;
    ap.v_head_stride = v_head_stride;
    ap.q = static_cast<const uint16_t*>(q);
    ap.q_tok_stride = q_tok_stride;
    ap.q_head_stride = q_head_stride;
    ap.q_out = static_cast<uint16_t*>(q_out);
    ap.qo_tok_stride = qo_tok_stride;
    ap.qo_head_stride = qo_head_stride;
    ap.gamma_k = gamma_k;
    ap.gamma_q = gamma_q;
    ap.eps = eps;
    ap.cos_tab = cos_tab;
    ap.sin_tab = sin_tab;
    ap.rope_stride = cos_tab ? rope_dim : D;
    ap.rope_dim = cos_tab ? rope_dim : D;
    ap.rope_pos0 = rope_pos0;
    ap.S = seq_len;
    ap.Hkv = s->n_kv_heads;
    ap.Hq = q ? n_q_heads : 0;
    ap.pos0 = pos0;
    ap.nq_tasks = q ? (n_q_heads + 7) / 8 : 0;
    ap.nkv_tasks = (s->n_kv_heads + 7) / 8;
    ap.k_pool = s->k_base;
    ap.v_pool = s->v_base;
    ap.page_elems = int64_t(kPage) * s->n_kv_heads * D;
    ap.k_ids = s->d_k_ids;
    ap.v_ids = s->d_v_ids;
    ap.max_blocks = s->max_blocks;
    if (int rc = launch_kv_append(ap, D, st)) {
        undo_append(*s, undo);
        return rc;
    }
    return GENLLM_OK;
}

// ---------------------------------------------------------- stateless ops
extern "C" int genllm_rms_norm(void* out, const void* x, const float* w, int64_t rows, int32_t hidden, float eps,
                               void* stream) {
    if (!out || !x || !w || hidden <= 0) return fail(GENLLM_ERR_INVALID, "rms_norm: bad arguments");
    return launch_rms_norm(static_cast<uint16_t*>(out), static_cast<const uint16_t*>(x), w, rows, hidden, eps,
                           as_stream(stream));
}

extern "C" int genllm_apply_rope(void* out, const void* x, const float* cos_tab, const float* sin_tab,
                                 int32_t n_heads, int32_t seq_len, int32_t head_dim, int32_t rope_dim,
                                 int64_t start_pos, void* stream) {
    if (!out || !x || !cos_tab || !sin_tab || head_dim <= 0 || head_dim % 2 || start_pos < 0 || rope_dim <= 0 ||
        rope_dim % 2 || rope_dim > head_dim)
        return fail(GENLLM_ERR_INVALID, "apply_rope: bad arguments");
    return launch_apply_rope(static_cast<uint16_t*>(out), static_cast<const uint16_t*>(x), cos_tab, sin_tab,
                             n_heads, seq_len, head_dim, rope_dim, start_pos, as_stream(stream));
}

// ApplyRopeImpl for a device-position decode step: as genllm_apply_rope with
// start_pos = the staged layer's device position (read when the kernel runs).
extern "C" int genllm_apply_rope_step(genllm_kv* kv, int32_t layer, void* out, const void* x, const float* cos_tab,
                                      const float* sin_tab, int32_t n_heads, int32_t seq_len, int32_t head_dim,
                                      int32_t rope_dim, int32_t max_seq, void* stream) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "apply_rope_step: null kv");
    LayerState* s = active_layer(kv, layer);
    if (!s || !s->staged) return fail(GENLLM_ERR_INVALID, "apply_rope_step: layer not staged (genllm_kv_stage_decode)");
    if (!out || !x || !cos_tab || !sin_tab || head_dim <= 0 || head_dim % 2 || rope_dim <= 0 || rope_dim % 2 ||
        rope_dim > head_dim || max_seq <= 0)
        return fail(GENLLM_ERR_INVALID, "apply_rope_step: bad arguments");
    return launch_apply_rope(static_cast<uint16_t*>(out), static_cast<const uint16_t*>(x), cos_tab, sin_tab,
                             n_heads, seq_len, head_dim, rope_dim, 0, as_stream(stream), s->d_step, max_seq);
}

extern "C" int genllm_rope_cache(float* dst, float theta, int32_t head_dim, int32_t max_seq, int32_t is_cos) {
    // RopeCacheImpl<CPU> (rope.cpp:121-148): double-precision angles, each value
    // stored at i and i + head_dim/2.
    if (!dst || head_dim <= 0 || head_dim % 2 || max_seq < 0) return fail(GENLLM_ERR_INVALID, "rope_cache: bad args");
    const int half = head_dim / 2;
    std::vector<double> inv(half);
    for (int i = 0; i < half; ++i) inv[i] = 1.0 / std::pow(double(theta), (2.0 * double(i)) / double(head_dim));
    for (int s = 0; s < max_seq; ++s) {
        for (int i = 0; i < half; ++i) {
            const double a = double(s) * inv[i];
            const float val = is_cos ? float(std::cos(a)) : float(std::sin(a));
            dst[size_t(s) * head_dim + i] = val;
            dst[size_t(s) * head_dim + i + half] = val;
        }
    }
    return GENLLM_OK;
}

// append_kv_from_pos (page_attention.cpp:164-203) as a manager call: the
// pages of positions [global_pos, global_pos + count) are opened by the rule
// of append_kv_pages (a block from each pool at every position that is a
// multiple of 16, entered into the table only past its end), the rows are
// written by the scatter kernel, and num_cached = max(num_cached,
// global_pos + count).  The source is head-major [Hkv][count][D] for every
// head (the reference reads head 0's row for all heads, :195 and :198).
// Checked before anything changes: every touched page must exist after the
// call (no gap past the table end, none not opened by this call), and both
// pools must hold the pages it opens.
extern "C" int genllm_kv_append_from_pos(genllm_kv* kv, int32_t layer, const void* k, const void* v,
                                         int32_t n_kv_heads, int32_t head_dim, int32_t dtype, int32_t global_pos,
                                         int32_t count, void* stream) {
    if (!kv) return fail(GENLLM_ERR_INVALID, "append_kv_from_pos: null kv");
    LayerState* s = active_layer(kv, layer);
    if (!s) return GENLLM_OK;  // page_attention.cpp:169: inactive layer
    if (int rc = refuse_staged(*s, "append_kv_from_pos")) return rc;
    if (count <= 0) return GENLLM_OK;
    if (!s->k_base) return fail(GENLLM_ERR_INVALID, "append_kv_from_pos: layer has no reserved pools");
    if (!k || !v) return fail(GENLLM_ERR_INVALID, "append_kv_from_pos: null k/v");
    if (dtype != s->dtype || elem_size(dtype) != 2 || n_kv_heads != s->n_kv_heads || head_dim != s->head_dim)
        return fail(GENLLM_ERR_INVALID, "append_kv_from_pos: tensor shape/dtype differs from the layer's pools");
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return fail(GENLLM_ERR_UNSUPPORTED, "append_kv_from_pos: head_dim must be 64, 128 or 256");
    if (!aligned(k, 16) || !aligned(v, 16))
        return fail(GENLLM_ERR_INVALID, "append_kv_from_pos: k/v must be 16-byte aligned");
    if (global_pos < 0 || int64_t(global_pos) + count > int64_t(INT32_MAX) - kPage)
        return fail(GENLLM_ERR_INVALID, "append_kv_from_pos: position out of range");
    const int64_t size = int64_t(s->k_ids.size());
    const int64_t first = (int64_t(global_pos) + kPage - 1) / kPage;  // first page this call opens
    const int64_t need = pages_opened(global_pos, count);
    const int64_t new_size = need > 0 ? std::max(size, first + need) : size;
    const int64_t last = (int64_t(global_pos) + count - 1) / kPage;  // last page written
    if ((need > 0 && first > size) || last >= new_size)
        return fail(GENLLM_ERR_INVALID, "append_kv_from_pos: positions " + std::to_string(global_pos) + ".." +
                                            std::to_string(int64_t(global_pos) + count - 1) +
                                            " reach pages the table does not hold and this call does not open");
    hipStream_t st = as_stream(stream);
    const int32_t saved = s->num_cached;
    AppendUndo& undo = t_undo;
    s->num_cached = global_pos;  // append_pages opens pages from its layer's num_cached
    if (int rc = append_pages(kv, *s, count, st, static_cast<TableUpdate*>(nullptr), &undo)) {
        s->num_cached = saved;
        return rc;
    }
    s->num_cached = std::max(saved, global_pos + count);
    AppendParams ap;
    ap.k = static_cast<const uint16_t*>(k);
    ap.v = static_cast<const uint16_t*>(v);
    ap.k_tok_stride = ap.v_tok_stride = head_dim;
    ap.k_head_stride = ap.v_head_stride = int64_t(count) * head_dim;
    ap.S = count;
    ap.Hkv = n_kv_heads;
    ap.pos0 = global_pos;
    ap.nkv_tasks = (n_kv_heads + 7) / 8;
    ap.k_pool = s->k_base;
    ap.v_pool = s->v_base;
    ap.page_elems = int64_t(kPage) * n_kv_heads * head_dim;
    ap.k_ids = s->d_k_ids;
    ap.v_ids = s->d_v_ids;
    ap.max_blocks = s->max_blocks;
    if (int rc = launch_kv_append(ap, head_dim, st)) {
        undo_append(*s, undo);
        s->num_cached = saved;
        return rc;
    }
    return GENLLM_OK;
}

extern "C" int genllm_kv_scatter(const void* k, int64_t k_tok_stride, int64_t k_head_stride, const void* v,
                                 int64_t v_tok_stride, int64_t v_head_stride, void* k_pool, void* v_pool,
                                 const int32_t* k_ids, const int32_t* v_ids, int32_t pos0, int32_t seq_len,
                                 int32_t n_kv_heads, int32_t head_dim, void* stream) {
    if (!k || !v || !k_pool || !v_pool || !k_ids || !v_ids || n_kv_heads <= 0 || pos0 < 0)
        return fail(GENLLM_ERR_INVALID, "kv_scatter: bad arguments");
    if (!aligned(k, 8) || !aligned(v, 16) || (k_tok_stride % 4) || (k_head_stride % 4) || (v_tok_stride % 8) ||
        (v_head_stride % 8))
        return fail(GENLLM_ERR_INVALID, "kv_scatter: misaligned pointer or stride");
    AppendParams ap;
    ap.k = static_cast<const uint16_t*>(k);
    ap.k_tok_stride = k_tok_stride;
    ap.k_head_stride = k_head_stride;
    ap.v = static_cast<const uint16_t*>(v);
    ap.v_tok_stride = v_tok_stride;
    ap.v_head_stride = v_head_stride;
    ap.S = seq_len;
    ap.Hkv = n_kv_heads;
    ap.pos0 = pos0;
    ap.nkv_tasks = (n_kv_heads + 7) / 8;
    ap.k_pool = static_cast<uint16_t*>(k_pool);
    ap.v_pool = static_cast<uint16_t*>(v_pool);
    ap.page_elems = int64_t(kPage) * n_kv_heads * head_dim;
    ap.k_ids = const_cast<int32_t*>(k_ids);
    ap.v_ids = const_cast<int32_t*>(v_ids);
    return launch_kv_append(ap, head_dim, as_stream(stream));
}

extern "C" int genllm_decode_tuning(int32_t pages_per_split, int32_t merge, int32_t heads_per_workgroup) {
    return set_decode_tuning(pages_per_split, merge, heads_per_workgroup);
}

extern "C" size_t genllm_paged_decode_workspace_bytes(int32_t n_q_heads, int32_t n_kv_heads, int32_t seq_len,
                                                      int32_t head_dim, int32_t max_pages) {
    return decode_workspace_bytes(n_q_heads, n_kv_heads, seq_len, head_dim, max_pages);
}

static AttnParams make_attn(const void* q, int64_t q_head_stride, int64_t q_tok_stride, void* out,
                            int64_t o_head_stride, int64_t o_tok_stride, const void* k_pool, const void* v_pool,
                            const int32_t* k_ids, const int32_t* v_ids, int32_t n_pages, int32_t n_cached,
                            int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, float scale,
                            int32_t causal) {
    AttnParams p;
    p.q = static_cast<const uint16_t*>(q);
    p.q_head_stride = q_head_stride;
    p.q_tok_stride = q_tok_stride;
    p.out = static_cast<uint16_t*>(out);
    p.o_head_stride = o_head_stride;
    p.o_tok_stride = o_tok_stride;
    p.k_pool = static_cast<const uint16_t*>(k_pool);
    p.v_pool = static_cast<const uint16_t*>(v_pool);
    p.k_ids = k_ids;
    p.v_ids = v_ids;
    p.n_pages = std::min(n_pages, (n_cached + kPage - 1) / kPage);
    p.n_cached = n_cached;
    p.S = seq_len;
    p.Hq = n_q_heads;
    p.Hkv = n_kv_heads;
    p.G = n_kv_heads > 0 ? n_q_heads / n_kv_heads : 0;
    p.scale_log2 = scale * kLog2e;
    p.causal = causal != 0;
    p.page_elems = int64_t(kPage) * n_kv_heads * head_dim;
    p.kv_row = int64_t(n_kv_heads) * head_dim;
    return p;
}

extern "C" int genllm_paged_decode(const void* q, int64_t q_head_stride, int64_t q_tok_stride, void* out,
                                   int64_t o_head_stride, int64_t o_tok_stride, const void* k_pool,
                                   const void* v_pool, const int32_t* k_ids, const int32_t* v_ids, int32_t n_pages,
                                   int32_t n_cached, int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads,
                                   int32_t head_dim, float scale, int32_t causal, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    AttnParams p = make_attn(q, q_head_stride, q_tok_stride, out, o_head_stride, o_tok_stride, k_pool, v_pool, k_ids,
                             v_ids, n_pages, n_cached, seq_len, n_q_heads, n_kv_heads, head_dim, scale, causal);
    if (int rc = check_attn_args(p, head_dim)) return rc;
    if (p.G * p.S > 16)
        return fail(GENLLM_ERR_INVALID, "paged_decode: seq_len * groups must be <= 16 (use paged_prefill)");
    if (int rc = decode_plan(p, head_dim, workspace_bytes, workspace)) return rc;
    return launch_paged_decode(p, head_dim, as_stream(stream));
}

extern "C" int genllm_paged_prefill(const void* q, int64_t q_head_stride, int64_t q_tok_stride, void* out,
                                    int64_t o_head_stride, int64_t o_tok_stride, const void* k_pool,
                                    const void* v_pool, const int32_t* k_ids, const int32_t* v_ids, int32_t n_pages,
                                    int32_t n_cached, int32_t seq_len, int32_t n_q_heads, int32_t n_kv_heads,
                                    int32_t head_dim, float scale, int32_t causal, void* stream) {
    AttnParams p = make_attn(q, q_head_stride, q_tok_stride, out, o_head_stride, o_tok_stride, k_pool, v_pool, k_ids,
                             v_ids, n_pages, n_cached, seq_len, n_q_heads, n_kv_heads, head_dim, scale, causal);
    if (int rc = check_attn_args(p, head_dim)) return rc;
    return launch_paged_prefill(p, head_dim, as_stream(stream));
}

// ------------------------------------------------ allocation-free decode
// Device scratch of genllm_paged_decode_noalloc: the arrival counters and the
// split partials that genllm_paged_decode takes from its caller's workspace.
// One copy per GPU the library runs on, held until the process ends.  In host
// code `scratch` is only a stand-in for the symbol: its device address on the
// current device comes from hipGetSymbolAddress (scratch_on_device).
static __device__ __align__(256) unsigned char scratch[GENLLM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};  // device address of `scratch`, per device

__global__ void zero_words_kernel(uint32_t* p, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

// The scratch of the current device: resolved once per device, with its
// arrival counters cleared by a small kernel on `stream` (no memset, so the
// call may be captured into a graph).
int scratch_on_device(hipStream_t stream, void** out) {
    int dev = 0;
    GENLLM_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(GENLLM_ERR_UNSUPPORTED, "paged_decode_noalloc: device id >= 64");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        GENLLM_HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) return fail(GENLLM_ERR_HIP, "paged_decode_noalloc: scratch has no device address");
        hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(256), 0, stream, static_cast<uint32_t*>(ptr),
                           int(kDecodeCounterBytes / sizeof(uint32_t)));
        GENLLM_LAUNCH_CHECK("zero_words_kernel");
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return GENLLM_OK;
}

}  // namespace

extern "C" int genllm_paged_decode_noalloc(const void* q, int64_t q_head_stride, int64_t q_tok_stride, void* out,
                                           int64_t o_head_stride, int64_t o_tok_stride, const void* k_pool,
                                           const void* v_pool, const int32_t* k_ids, const int32_t* v_ids,
                                           int32_t n_pages, int32_t n_cached, int32_t seq_len, int32_t n_q_heads,
                                           int32_t n_kv_heads, int32_t head_dim, float scale, int32_t causal,
                                           void* stream) {
    AttnParams p = make_attn(q, q_head_stride, q_tok_stride, out, o_head_stride, o_tok_stride, k_pool, v_pool, k_ids,
                             v_ids, n_pages, n_cached, seq_len, n_q_heads, n_kv_heads, head_dim, scale, causal);
    if (int rc = check_attn_args(p, head_dim)) return rc;
    if (p.G * p.S > 16)
        return fail(GENLLM_ERR_INVALID, "paged_decode_noalloc: seq_len * groups must be <= 16");
    void* ws = nullptr;
    if (int rc = scratch_on_device(as_stream(stream), &ws)) return rc;
    if (int rc = decode_plan(p, head_dim, SIZE_MAX, ws)) return rc;
    const size_t need = p.n_splits > 1 ? kDecodeCounterBytes + size_t(p.Hkv) * p.n_splits * size_t(p.G * p.S) *
                                                                 size_t(head_dim + 2) * sizeof(float)
                                       : 0;
    if (need > GENLLM_NOALLOC_SCRATCH_BYTES)
        return fail(GENLLM_ERR_INVALID, "paged_decode_noalloc: this launch needs " + std::to_string(need) +
                                            " bytes of scratch, more than its fixed " +
                                            std::to_string(size_t(GENLLM_NOALLOC_SCRATCH_BYTES)) +
                                            " (use genllm_paged_decode with a workspace)");
    return launch_paged_decode(p, head_dim, as_stream(stream));
}

// Non-paged attention (FlashAttentionImpl, attention.cpp:39-121): the prefill
// kernel reading K/V straight from the [B][Hkv][S][D] tensors -- page i of a
// head is rows 16i..16i+15 of that head, so no block table is involved.  Query
// s attends keys 0..s (causal) or all S keys; one launch per batch entry.
extern "C" int genllm_flash_attention(const void* q, const void* k, const void* v, void* out, int32_t batch,
                                      int32_t n_q_heads, int32_t seq_len, int32_t n_kv_heads, int32_t head_dim,
                                      int32_t n_kv_groups, float scale, int32_t causal, void* stream) {
    if (!q || !k || !v || !out) return fail(GENLLM_ERR_INVALID, "flash_attention: null tensor");
    if (head_dim != 128 && head_dim != 256)
        return fail(GENLLM_ERR_UNSUPPORTED, "flash_attention requires head_dim 128 or 256");
    if (batch < 0 || seq_len < 0 || n_kv_heads <= 0 || n_kv_groups <= 0 || n_q_heads != n_kv_heads * n_kv_groups)
        return fail(GENLLM_ERR_INVALID, "flash_attention: n_q_heads must equal n_kv_heads * n_kv_groups");
    if (!(scale >= 0.0f) || scale == INFINITY)
        return fail(GENLLM_ERR_INVALID, "flash_attention: scale must be finite and >= 0");
    if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 8))
        return fail(GENLLM_ERR_INVALID, "flash_attention: tensors must be 16-byte aligned");
    const int64_t D = head_dim, S = seq_len;
    for (int32_t b = 0; b < batch && seq_len > 0; ++b) {
        AttnParams p;
        p.q = static_cast<const uint16_t*>(q) + int64_t(b) * n_q_heads * S * D;
        p.q_head_stride = S * D;
        p.q_tok_stride = D;
        p.out = static_cast<uint16_t*>(out) + int64_t(b) * n_q_heads * S * D;
        p.o_head_stride = S * D;
        p.o_tok_stride = D;
        p.k_pool = static_cast<const uint16_t*>(k) + int64_t(b) * n_kv_heads * S * D;
        p.v_pool = static_cast<const uint16_t*>(v) + int64_t(b) * n_kv_heads * S * D;
        p.k_ids = p.v_ids = nullptr;
        p.n_pages = int32_t((S + kPage - 1) / kPage);
        p.n_cached = seq_len;
        p.S = seq_len;
        p.Hq = n_q_heads;
        p.Hkv = n_kv_heads;
        p.G = n_kv_groups;
        p.scale_log2 = scale * kLog2e;
        p.causal = causal != 0;
        p.page_elems = kPage * D;
        p.kv_row = D;
        p.kv_head_stride = S * D;
        if (int rc = launch_paged_prefill(p, head_dim, as_stream(stream))) return rc;
    }
    return GENLLM_OK;
}
