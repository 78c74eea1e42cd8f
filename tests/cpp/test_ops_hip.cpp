// test_ops_hip.cpp -- the HIP backend driven through the reference's operator
// interface (Tensor nodes -> kernel::dispatch -> ops::*Impl<Device::HIP>), in
// the spirit of the reference's tests/test_page_attention.cpp and
// tests/test_ops_cpu.cpp (same sequences, checked with check.hpp).  Results are checked against the CPU restatement in
// oracle/ (liboracle.so): page tables and K/V pages bit-exact, RMSNorm /
// RoPE / rope tables bit-exact, attention within max-abs <= 2^-7 * max|ref|
// and relative L2 <= 1e-2.  Needs one GPU.
#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <vector>

#include "genllm/kernels.hpp"
#include "genllm/manager.hpp"
#include "genllm/page_attention.hpp"
#include "genllm/tensor.hpp"
#include "genllm_paged.h"
#include "oracle.h"
#include "check.hpp"

namespace {

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    explicit DevBuf(size_t n) : bytes(n) {
        if (hipMalloc(&p, n ? n : 16) != hipSuccess) throw std::runtime_error("hipMalloc failed");
    }
    ~DevBuf() { (void)hipFree(p); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
};

template <typename T>
std::vector<T> to_host(const void* dev, size_t n) {
    std::vector<T> h(n);
    if (hipDeviceSynchronize() != hipSuccess || hipMemcpy(h.data(), dev, n * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
        throw std::runtime_error("device -> host copy failed");
    return h;
}

template <typename T>
void to_device(void* dev, const std::vector<T>& h) {
    if (hipMemcpy(dev, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
        throw std::runtime_error("host -> device copy failed");
}

// seeded N(0,1) bf16 on the device (libgenllm_hip's generator), plus a host copy
std::vector<uint16_t> fill_normal(DevBuf& b, uint64_t seed) {
    const size_t n = b.bytes / 2;
    if (genllm_fill_normal_bf16(b.p, n, seed, 0, nullptr) != GENLLM_OK) throw std::runtime_error(genllm_last_error());
    return to_host<uint16_t>(b.p, n);
}

Tensor make_tensor(void* data, std::array<int64_t, 4> dims, DataType dt = DataType::GGML_TYPE_BF16) {
    Tensor t;
    t.data = data;
    t.device = Device::HIP;
    t.dtype = dt;
    t.dims = dims;
    return t;
}

// max-abs <= 2^-7 * max|ref| and rel-L2 <= 1e-2 (bf16 output, fp32 accumulation)
bool attn_close(const std::vector<uint16_t>& got, const std::vector<uint16_t>& want, const char* what) {
    if (got.size() != want.size()) return false;
    double max_ref = 0, max_err = 0, num = 0, den = 0;
    for (size_t i = 0; i < got.size(); ++i) {
        const double a = or_bf16_to_f32(got[i]), b = or_bf16_to_f32(want[i]);
        if (!std::isfinite(a)) {
            std::printf("    %s: non-finite output at %zu\n", what, i);
            return false;
        }
        max_ref = std::max(max_ref, std::abs(b));
        max_err = std::max(max_err, std::abs(a - b));
        num += (a - b) * (a - b);
        den += b * b;
    }
    const double rel = den > 0 ? std::sqrt(num / den) : std::sqrt(num);
    const bool ok = max_err <= max_ref / 128.0 && rel <= 1e-2;
    std::printf("    %s: max_abs %.3g (bound %.3g) rel_l2 %.3g\n", what, max_err, max_ref / 128.0, rel);
    return ok;
}

// ---------------------------------------------------------------- enums
void test_device_enum(check::Context& c) {
    // tests/test_tensor.cpp:72-76, plus the HIP value
    CHECK_TRUE(c, static_cast<int>(Device::CPU) == 0, "cpu=0");
    CHECK_TRUE(c, static_cast<int>(Device::CUDA) == 1, "cuda=1");
    CHECK_TRUE(c, static_cast<int>(Device::HIP) == 2, "hip=2");
    CHECK_TRUE(c, static_cast<int>(Device::VULKAN) == 4, "vulkan=4");
    CHECK_TRUE(c, static_cast<int>(OperationType::OP_TYPE_PAGED_ATTN) == 24, "paged attn op id");
    CHECK_TRUE(c, static_cast<int>(DataType::GGML_TYPE_BF16) == 30, "bf16 id");
}

// ---------------------------------------------- tests/test_page_attention.cpp
void test_block_pool_alloc_free(check::Context& c) {
    PagedAttentionManager mgr(0, 64 << 20);
    mgr.init_layer(0, 8, 128, DataType::GGML_TYPE_BF16);
    mgr.reserve_layer(0, 100);
    BlockPool pool = mgr.get_layer(0).k_pool;
    CHECK_TRUE(c, pool.num_blocks() == 0, "initially 0 blocks");
    CHECK_TRUE(c, pool.num_free() == 0, "initially 0 free");
    const int32_t id = pool.alloc();
    CHECK_TRUE(c, id == 0, "first alloc returns 0");
    CHECK_TRUE(c, pool.num_blocks() == 1, "1 block after alloc");
    CHECK_TRUE(c, pool.alloc() == 1, "second alloc returns 1");
    pool.free(id);
    CHECK_TRUE(c, pool.num_free() == 1, "1 free after free");
    CHECK_TRUE(c, pool.alloc() == id, "reuse freed block");
    CHECK_TRUE(c, pool.num_free() == 0, "0 free after re-alloc");
    CHECK_TRUE(c, pool.block_data(1) == static_cast<char*>(pool.block_data(0)) + 16 * 8 * 128 * 2, "block stride");
    CHECK_TRUE(c, pool.block_data(2) == nullptr, "no data past num_blocks");
}

void test_block_pool_many_allocs(check::Context& c) {
    PagedAttentionManager mgr(0, 8 << 20);
    mgr.init_layer(0, 8, 128, DataType::GGML_TYPE_BF16);
    mgr.reserve_layer(0, 10);
    BlockPool pool = mgr.get_layer(0).v_pool;
    for (int i = 0; i < 10; i++) CHECK_TRUE(c, pool.alloc() >= 0, "alloc within capacity");
    CHECK_TRUE(c, pool.alloc() == -1, "beyond capacity returns -1");
}

void test_block_pool_reset(check::Context& c) {
    PagedAttentionManager mgr(0, 8 << 20);
    mgr.init_layer(0, 8, 128, DataType::GGML_TYPE_BF16);
    mgr.reserve_layer(0, 10);
    BlockPool pool = mgr.get_layer(0).k_pool;
    (void)pool.alloc();
    (void)pool.alloc();
    (void)pool.alloc();
    mgr.reset();
    CHECK_TRUE(c, pool.num_blocks() == 3, "reset keeps num_blocks");
    CHECK_TRUE(c, pool.num_free() == 3, "reset adds all back to free");
    CHECK_TRUE(c, pool.alloc() == 2, "free list [0,1,2] pops 2");
}

void test_page_table_append_kv(check::Context& c) {
    PagedAttentionManager mgr(0, 1 << 20);
    mgr.init_layer(0, 8, 128, DataType::GGML_TYPE_BF16);
    // held across the appends, as test_page_attention.cpp:53-61 holds it
    auto& layer = mgr.get_layer(0);
    CHECK_TRUE(c, layer.active, "layer active");
    CHECK_TRUE(c, layer.num_cached == 0, "initially 0 cached");
    mgr.append_kv_pages(0, 1);
    CHECK_TRUE(c, layer.num_cached == 1, "1 token cached");
    mgr.append_kv_pages(0, 31);
    CHECK_TRUE(c, layer.num_cached == 32, "32 tokens cached");
    CHECK_TRUE(c, layer.page_table.size() == 2, "2 pages (16+16)");
    CHECK_TRUE(c, &mgr.get_layer(0) == &layer, "one view per layer");
    mgr.reset();
    CHECK_TRUE(c, layer.num_cached == 0 && layer.page_table.empty(), "reset shows in the view");
}

// get_layer's reference is writable, as the reference's is: an in-place edit
// of page_table reaches the native table before the next call on the layer.
void test_get_layer_edit_in_place(check::Context& c) {
    PagedAttentionManager mgr(0, 4 << 20);
    mgr.init_layer(0, 8, 128, DataType::GGML_TYPE_BF16);
    mgr.reserve_layer(0, 8);
    auto& layer = mgr.get_layer(0);
    mgr.append_kv_pages(0, 32);
    CHECK_TRUE(c, layer.page_table.size() == 2, "2 pages");
    const PageEntry p0 = layer.page_table[0], p1 = layer.page_table[1];
    std::swap(layer.page_table[0], layer.page_table[1]);  // e.g. a permuted table, set in place
    mgr.append_kv_pages(0, 1);                           // commits the edit, then opens page 2
    CHECK_TRUE(c, layer.num_cached == 33 && layer.page_table.size() == 3, "append after the edit");
    CHECK_TRUE(c, layer.page_table[0].k_block_id == p1.k_block_id && layer.page_table[1].k_block_id == p0.k_block_id,
           "edit kept");
    std::vector<int32_t> k(3), v(3);
    int32_t n = 0;
    CHECK_TRUE(c, genllm_kv_page_table(mgr.handle(), 0, k.data(), v.data(), 3, &n) == 0 && n == 3, "native table");
    CHECK_TRUE(c, k[0] == p1.k_block_id && v[0] == p1.v_block_id && k[1] == p0.k_block_id, "native table holds the edit");
    layer.page_table[0].k_block_id = 1000;  // not a block the pool handed out
    bool threw = false;
    try {
        mgr.append_kv_pages(0, 1);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK_TRUE(c, threw, "an invalid edit is refused at commit");
    layer.page_table[0].k_block_id = p1.k_block_id;
    mgr.append_kv_pages(0, 1);
    CHECK_TRUE(c, layer.num_cached == 34, "usable again once the edit is valid");
}

void test_page_table_multi_layer(check::Context& c) {
    PagedAttentionManager mgr(0, 1 << 20);
    mgr.init_layer(0, 8, 128, DataType::GGML_TYPE_F16);
    mgr.init_layer(1, 4, 64, DataType::GGML_TYPE_F32);
    CHECK_TRUE(c, mgr.is_active(0), "layer 0 active");
    CHECK_TRUE(c, mgr.is_active(1), "layer 1 active");
    CHECK_TRUE(c, !mgr.is_active(2), "layer 2 not active");
    mgr.append_kv_pages(0, 5);
    mgr.append_kv_pages(1, 20);
    CHECK_TRUE(c, mgr.get_layer(0).num_cached == 5, "layer0 cached 5");
    CHECK_TRUE(c, mgr.get_layer(1).num_cached == 20, "layer1 cached 20");
    mgr.reset();
    CHECK_TRUE(c, mgr.get_layer(0).num_cached == 0, "after reset layer0 = 0");
    CHECK_TRUE(c, mgr.get_layer(1).page_table.empty(), "after reset page_table empty");
}

// ------------------------------------------- scheduler rules and the switch
void test_kv_cache_per_layer_switch(check::Context& c) {
    CHECK_TRUE(c, attention_op_type(0) == OperationType::OP_TYPE_FLASH_ATTN, "0 -> flash attention");
    CHECK_TRUE(c, attention_op_type(1) == OperationType::OP_TYPE_PAGED_ATTN, "1 -> paged attention");
    CHECK_TRUE(c, attention_op_type(4) == OperationType::OP_TYPE_PAGED_ATTN, ">1 -> paged attention");
    Tensor k = make_tensor(nullptr, {1, 8, 1, 128});
    Tensor paged = make_tensor(nullptr, {1, 32, 1, 128});
    paged.op_type = OperationType::OP_TYPE_PAGED_ATTN;
    paged.src[1] = &k;
    paged.layer_id = 0;
    Tensor flash = paged;
    flash.op_type = OperationType::OP_TYPE_FLASH_ATTN;
    flash.layer_id = 1;
    // scheduler.cpp:363-372: 2 * ceil(max_seq/16) * 16 * Hkv * D * elem
    CHECK_TRUE(c, kv_cache_bytes({&paged}, Device::HIP, 300, 1.0f) == size_t(2) * 19 * 16 * 8 * 128 * 2, "paged sizing");
    CHECK_TRUE(c, kv_cache_bytes({&flash}, Device::HIP, 300, 1.0f) == 0, "flash attention owns no pages");
    CHECK_TRUE(c, kv_cache_bytes({&paged}, Device::CPU, 300, 1.0f) == 0, "other device not counted");
}

// ------------------------------------- the op through the executor's switch
// A two-layer graph of PAGED_ATTN nodes: prefill chunk of `s0` tokens, then
// `steps` decode tokens, every call checked against or_paged_attention.
void run_paged_graph(check::Context& c, int32_t Hq, int32_t Hkv, int32_t s0, int steps, uint64_t seed) {
    const int32_t D = 128, G = Hq / Hkv, max_seq = 256, L = 2;
    const float scale = 1.0f / std::sqrt(float(D));
    MemoryManager mm;
    std::vector<Tensor> ks(L), nodes(L);
    std::vector<Tensor*> graph;
    for (int l = 0; l < L; ++l) {
        ks[l] = make_tensor(nullptr, {1, Hkv, 1, D});
        nodes[l] = make_tensor(nullptr, {1, Hq, 1, D});
        nodes[l].op_type = OperationType::OP_TYPE_PAGED_ATTN;
        nodes[l].src[1] = &ks[l];
        nodes[l].layer_id = l;
        graph.push_back(&nodes[l]);
    }
    // exactly the scheduler's sizing, no slack (scheduler.cpp:62-79, 371)
    const size_t bytes = kv_cache_bytes(graph, Device::HIP, max_seq);
    PagedAttentionManager& pam = mm.create_attention_manager(Device::HIP, 0, bytes);
    initialize_kv_cache(pam, graph, max_seq);

    or_manager* ref = or_mgr_create(1);
    for (int l = 0; l < L; ++l) {
        or_mgr_init_layer(ref, l, Hkv, D, OR_DTYPE_BF16);
        or_mgr_reserve_layer(ref, l, (max_seq + 15) / 16);
    }
    bool ok = true;
    const auto& live = pam.get_layer(L - 1);  // kept current by the PAGED_ATTN nodes themselves
    for (int step = 0; step <= steps && ok; ++step) {
        const int32_t S = step == 0 ? s0 : 1;
        for (int l = 0; l < L && ok; ++l) {
            DevBuf q(size_t(Hq) * S * D * 2), k(size_t(Hkv) * S * D * 2), v(size_t(Hkv) * S * D * 2),
                o(size_t(Hq) * S * D * 2);
            const uint64_t sd = seed + 1000 * step + 10 * l;
            auto hq = fill_normal(q, sd), hk = fill_normal(k, sd + 1), hv = fill_normal(v, sd + 2);
            Tensor Q = make_tensor(q.p, {1, Hq, S, D}), K = make_tensor(k.p, {1, Hkv, S, D}),
                   V = make_tensor(v.p, {1, Hkv, S, D});
            Tensor out = make_tensor(o.p, {1, Hq, S, D});
            out.op_type = OperationType::OP_TYPE_PAGED_ATTN;
            out.layer_id = l;
            out.src = {&Q, &K, &V, nullptr, nullptr, nullptr};
            out.op_params = {float(D), scale, 1.0f, float(G)};
            CHECK_TRUE(c, kernel::dispatch(&out, 0), "executor dispatches PAGED_ATTN");
            std::vector<uint16_t> want(size_t(Hq) * S * D);
            or_paged_attention(ref, l, hq.data(), hk.data(), hv.data(), want.data(), 1, Hq, S, D, Hkv, G, scale, 1);
            char what[96];
            std::snprintf(what, sizeof what, "Hq%d Hkv%d layer %d step %d (S=%d)", Hq, Hkv, l, step, S);
            ok = attn_close(to_host<uint16_t>(o.p, want.size()), want, what);
            // page placement: tables and pools bit-exact
            const auto st = pam.get_layer(l);
            std::vector<int32_t> rk(st.page_table.size()), rv(st.page_table.size());
            const int32_t n = or_mgr_get_page_table(ref, l, rk.data(), rv.data(), int32_t(rk.size()));
            CHECK_TRUE(c, n == int32_t(st.page_table.size()), "page table length");
            for (int32_t i = 0; i < n; ++i)
                CHECK_TRUE(c, st.page_table[i].k_block_id == rk[i] && st.page_table[i].v_block_id == rv[i], "page ids");
            CHECK_TRUE(c, st.num_cached == or_mgr_num_cached(ref, l), "num_cached");
            CHECK_TRUE(c, live.num_cached == or_mgr_num_cached(ref, L - 1), "held view follows the op");
        }
    }
    for (int l = 0; l < L && ok; ++l) {
        const auto st = pam.get_layer(l);
        const size_t pool_elems = size_t(st.k_pool.num_blocks()) * 16 * Hkv * D;
        const auto dk = to_host<uint16_t>(st.k_pool.block_data(0), pool_elems);
        const auto dv = to_host<uint16_t>(st.v_pool.block_data(0), pool_elems);
        CHECK_TRUE(c, std::memcmp(dk.data(), or_mgr_k_pool(ref, l), pool_elems * 2) == 0, "K pages bit-exact");
        CHECK_TRUE(c, std::memcmp(dv.data(), or_mgr_v_pool(ref, l), pool_elems * 2) == 0, "V pages bit-exact");
    }
    or_mgr_destroy(ref);
    CHECK_TRUE(c, ok, "attention within tolerance of the oracle");
}

// A decode loop captured into one HIP graph (the executor's loop,
// executor.cpp:227-236, without its per-step host bookkeeping): two layers'
// RoPE(q), RoPE(k) and PAGED_ATTN nodes, their op_params' start_pos left
// stale, dispatched once under stream capture with the layers staged, then
// replayed for 12 tokens across the page boundary at 32.  Every replay:
// RoPE'd q bit-exact and attention within tolerance of the oracle run with
// host positions; after sync_decode, num_cached and the tables equal the
// oracle's.
void test_decode_step_graph(check::Context& c) {
    const int32_t Hq = 32, Hkv = 8, D = 128, G = Hq / Hkv, L = 2, P = 26, steps = 12, max_seq = 128;
    const float scale = 1.0f / std::sqrt(float(D));
    MemoryManager mm;
    hipStream_t s = nullptr;
    CHECK_TRUE(c, hipStreamCreate(&s) == hipSuccess, "stream");
    std::vector<Tensor> ks(L), sizing(L);
    std::vector<Tensor*> graph;
    for (int l = 0; l < L; ++l) {
        ks[l] = make_tensor(nullptr, {1, Hkv, 1, D});
        sizing[l] = make_tensor(nullptr, {1, Hq, 1, D});
        sizing[l].op_type = OperationType::OP_TYPE_PAGED_ATTN;
        sizing[l].src[1] = &ks[l];
        sizing[l].layer_id = l;
        graph.push_back(&sizing[l]);
    }
    PagedAttentionManager& pam =
        mm.create_attention_manager(Device::HIP, 0, kv_cache_bytes(graph, Device::HIP, max_seq));
    initialize_kv_cache(pam, graph, max_seq);
    mm.set_stream(Device::HIP, 0, s);
    or_manager* ref = or_mgr_create(1);
    for (int l = 0; l < L; ++l) {
        or_mgr_init_layer(ref, l, Hkv, D, OR_DTYPE_BF16);
        or_mgr_reserve_layer(ref, l, (max_seq + 15) / 16);
    }
    bool ok = true;
    // the prompt, through the host-position op
    for (int l = 0; l < L; ++l) {
        DevBuf q(size_t(Hq) * P * D * 2), k(size_t(Hkv) * P * D * 2), v(size_t(Hkv) * P * D * 2),
            o(size_t(Hq) * P * D * 2);
        auto hq = fill_normal(q, 900 + l), hk = fill_normal(k, 910 + l), hv = fill_normal(v, 920 + l);
        Tensor Q = make_tensor(q.p, {1, Hq, P, D}), K = make_tensor(k.p, {1, Hkv, P, D}),
               V = make_tensor(v.p, {1, Hkv, P, D}), out = make_tensor(o.p, {1, Hq, P, D});
        out.op_type = OperationType::OP_TYPE_PAGED_ATTN;
        out.layer_id = l;
        out.src = {&Q, &K, &V, nullptr, nullptr, nullptr};
        out.op_params = {float(D), scale, 1.0f, float(G)};
        CHECK_TRUE(c, kernel::dispatch(&out, 0), "prompt");
        std::vector<uint16_t> want(size_t(Hq) * P * D);
        or_paged_attention(ref, l, hq.data(), hk.data(), hv.data(), want.data(), 1, Hq, P, D, Hkv, G, scale, 1);
    }
    CHECK_TRUE(c, hipStreamSynchronize(s) == hipSuccess, "prompt done");
    std::vector<float> hcos(size_t(max_seq) * D), hsin(size_t(max_seq) * D);
    or_rope_cache(hcos.data(), 1e6f, D, max_seq, 1);
    or_rope_cache(hsin.data(), 1e6f, D, max_seq, 0);
    DevBuf dcos(hcos.size() * 4), dsin(hsin.size() * 4);
    to_device(dcos.p, hcos);
    to_device(dsin.p, hsin);
    Tensor cos_t = make_tensor(dcos.p, {max_seq, D, 0, 0}, DataType::GGML_TYPE_F32),
           sin_t = make_tensor(dsin.p, {max_seq, D, 0, 0}, DataType::GGML_TYPE_F32);
    // fixed step buffers and nodes per layer
    struct Layer {
        std::unique_ptr<DevBuf> q, k, v, qr, kr, o;
        Tensor xq, xk, rq, rk, vv, attn;
    };
    std::vector<Layer> ly(L);
    for (int l = 0; l < L; ++l) {
        Layer& y = ly[l];
        y.q = std::make_unique<DevBuf>(size_t(Hq) * D * 2);
        y.qr = std::make_unique<DevBuf>(size_t(Hq) * D * 2);
        y.o = std::make_unique<DevBuf>(size_t(Hq) * D * 2);
        y.k = std::make_unique<DevBuf>(size_t(Hkv) * D * 2);
        y.kr = std::make_unique<DevBuf>(size_t(Hkv) * D * 2);
        y.v = std::make_unique<DevBuf>(size_t(Hkv) * D * 2);
        y.xq = make_tensor(y.q->p, {1, Hq, 1, D});
        y.xk = make_tensor(y.k->p, {1, Hkv, 1, D});
        y.vv = make_tensor(y.v->p, {1, Hkv, 1, D});
        for (auto [r, x, buf, H] : {std::tuple{&y.rq, &y.xq, y.qr.get(), Hq}, std::tuple{&y.rk, &y.xk, y.kr.get(), Hkv}}) {
            *r = make_tensor(buf->p, {1, H, 1, D});
            r->op_type = OperationType::OP_TYPE_APPLY_ROPE;
            r->src = {x, &cos_t, &sin_t, nullptr, nullptr, nullptr};
            r->op_params = {float(D), float(D), 0.0f, 0};  // start_pos stale: the device position rules
            r->layer_id = l;
        }
        y.attn = make_tensor(y.o->p, {1, Hq, 1, D});
        y.attn.op_type = OperationType::OP_TYPE_PAGED_ATTN;
        y.attn.layer_id = l;
        y.attn.src = {&y.rq, &y.rk, &y.vv, nullptr, nullptr, nullptr};
        y.attn.op_params = {float(D), scale, 1.0f, float(G)};
        pam.stage_decode(l, steps);
    }
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    CHECK_TRUE(c, hipStreamBeginCapture(s, hipStreamCaptureModeGlobal) == hipSuccess, "begin capture");
    for (int l = 0; l < L; ++l)
        for (Tensor* t : {&ly[l].rq, &ly[l].rk, &ly[l].attn}) kernel::dispatch(t, 0);
    CHECK_TRUE(c, hipStreamEndCapture(s, &g) == hipSuccess, "end capture");
    CHECK_TRUE(c, hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) == hipSuccess, "instantiate");
    for (int step = 0; step < steps && ok; ++step) {
        const int32_t pos = P + step;
        std::vector<std::vector<uint16_t>> hq(L), hk(L), hv(L);
        for (int l = 0; l < L; ++l) {
            hq[l] = fill_normal(*ly[l].q, 5000 + 10 * step + l);
            hk[l] = fill_normal(*ly[l].k, 6000 + 10 * step + l);
            hv[l] = fill_normal(*ly[l].v, 7000 + 10 * step + l);
        }
        CHECK_TRUE(c, hipGraphLaunch(ge, s) == hipSuccess, "replay");
        CHECK_TRUE(c, hipStreamSynchronize(s) == hipSuccess, "replay done");
        for (int l = 0; l < L && ok; ++l) {
            std::vector<uint16_t> qr(size_t(Hq) * D), kr(size_t(Hkv) * D), want(size_t(Hq) * D);
            or_apply_rope(qr.data(), hq[l].data(), hcos.data(), hsin.data(), Hq, 1, D, pos);
            or_apply_rope(kr.data(), hk[l].data(), hcos.data(), hsin.data(), Hkv, 1, D, pos);
            CHECK_TRUE(c, to_host<uint16_t>(ly[l].qr->p, qr.size()) == qr, "RoPE'd q at the device position bit-exact");
            or_paged_attention(ref, l, qr.data(), kr.data(), hv[l].data(), want.data(), 1, Hq, 1, D, Hkv, G, scale, 1);
            char what[80];
            std::snprintf(what, sizeof what, "replay %d layer %d position %d", step, l, pos);
            ok = attn_close(to_host<uint16_t>(ly[l].o->p, want.size()), want, what);
        }
    }
    for (int l = 0; l < L && ok; ++l) {
        CHECK_TRUE(c, pam.sync_decode(l) == P + steps && !pam.is_staged(l), "num_cached after sync");
        const auto st = pam.get_layer(l);
        std::vector<int32_t> rk(st.page_table.size()), rv(st.page_table.size());
        CHECK_TRUE(c, or_mgr_get_page_table(ref, l, rk.data(), rv.data(), int32_t(rk.size())) == int32_t(rk.size()),
               "page table length");
        for (size_t i = 0; i < rk.size(); ++i)
            CHECK_TRUE(c, st.page_table[i].k_block_id == rk[i] && st.page_table[i].v_block_id == rv[i], "page ids");
        CHECK_TRUE(c, st.num_cached == or_mgr_num_cached(ref, l), "num_cached");
    }
    (void)hipGraphExecDestroy(ge);
    (void)hipGraphDestroy(g);
    mm.set_stream(Device::HIP, 0, nullptr);
    (void)hipStreamDestroy(s);
    or_mgr_destroy(ref);
    CHECK_TRUE(c, ok, "attention within tolerance of the oracle");
}

void test_paged_attention_qwen06b(check::Context& c) { run_paged_graph(c, 16, 8, 40, 3, 0x5EED0001); }
void test_paged_attention_qwen4b(check::Context& c) { run_paged_graph(c, 32, 8, 33, 3, 0x5EED0003); }

void test_paged_attention_errors(check::Context& c) {
    MemoryManager mm;
    PagedAttentionManager& pam = mm.create_attention_manager(Device::HIP, 0, 8 << 20);
    pam.init_layer(0, 2, 64, DataType::GGML_TYPE_BF16);
    pam.reserve_layer(0, 8);
    DevBuf q(4 * 64 * 2), k(2 * 64 * 2), o(4 * 64 * 2);
    (void)fill_normal(q, 7);
    (void)fill_normal(k, 8);
    Tensor Q = make_tensor(q.p, {1, 4, 1, 64}), K = make_tensor(k.p, {1, 2, 1, 64});
    Tensor out = make_tensor(o.p, {1, 4, 1, 64});
    out.op_type = OperationType::OP_TYPE_PAGED_ATTN;
    out.src = {&Q, &K, &K, nullptr, nullptr, nullptr};
    out.op_params = {64.0f, 0.125f, 1.0f, 2.0f};
    out.layer_id = 0;
    bool threw = false;
    try {
        kernel::paged_attention(&out, 0);  // attention.cu:511 throws for head_dim != 128
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK_TRUE(c, threw, "head_dim 64 throws std::runtime_error");
    // inactive layer: silent return, output untouched (attention.cpp:127)
    std::vector<uint16_t> sentinel(4 * 64, 0x7777);
    to_device(o.p, sentinel);
    out.layer_id = 5;
    kernel::paged_attention(&out, 0);
    CHECK_TRUE(c, to_host<uint16_t>(o.p, sentinel.size()) == sentinel, "inactive layer leaves out untouched");
    // a CPU node never reaches the HIP backend
    out.device = Device::CPU;
    threw = false;
    try {
        kernel::paged_attention(&out, 0);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK_TRUE(c, threw, "dispatchOp throws for a device this library does not serve");
}

// ----------------------------------------------- FlashAttention (non-paged)
void run_flash(check::Context& c, int32_t B, int32_t Hq, int32_t Hkv, int32_t S, bool causal, uint64_t seed) {
    const int32_t D = 128, G = Hq / Hkv;
    const float scale = 1.0f / std::sqrt(float(D));
    DevBuf q(size_t(B) * Hq * S * D * 2), k(size_t(B) * Hkv * S * D * 2), v(size_t(B) * Hkv * S * D * 2),
        o(size_t(B) * Hq * S * D * 2);
    auto hq = fill_normal(q, seed), hk = fill_normal(k, seed + 1), hv = fill_normal(v, seed + 2);
    Tensor Q = make_tensor(q.p, {B, Hq, S, D}), K = make_tensor(k.p, {B, Hkv, S, D}),
           V = make_tensor(v.p, {B, Hkv, S, D});
    Tensor out = make_tensor(o.p, {B, Hq, S, D});
    out.op_type = OperationType::OP_TYPE_FLASH_ATTN;
    out.src = {&Q, &K, &V, nullptr, nullptr, nullptr};
    out.op_params = {float(D), scale, causal ? 1.0f : 0.0f, float(G)};
    CHECK_TRUE(c, kernel::dispatch(&out, 0), "executor dispatches FLASH_ATTN");
    std::vector<uint16_t> want(size_t(B) * Hq * S * D);
    or_flash_attention(hq.data(), hk.data(), hv.data(), want.data(), B, Hq, S, Hkv, D, G, scale, causal);
    char what[96];
    std::snprintf(what, sizeof what, "flash B%d Hq%d Hkv%d S%d causal %d", B, Hq, Hkv, S, int(causal));
    CHECK_TRUE(c, attn_close(to_host<uint16_t>(o.p, want.size()), want, what), "flash attention within tolerance");
}

void test_flash_attention_causal(check::Context& c) { run_flash(c, 2, 8, 2, 77, true, 11); }
void test_flash_attention_full(check::Context& c) { run_flash(c, 1, 16, 8, 130, false, 12); }
void test_flash_attention_one_token(check::Context& c) { run_flash(c, 1, 4, 4, 1, true, 13); }

// ----------------------------------------------------- RMSNorm, RoPE, tables
void test_rms_norm_rope_nodes(check::Context& c) {
    const int32_t H = 5, S = 9, D = 128, max_seq = 64;
    const int64_t start = 7;
    MemoryManager mm;
    DevBuf x(size_t(H) * S * D * 2), y(size_t(H) * S * D * 2), r(size_t(H) * S * D * 2), w(D * 4);
    DevBuf cs(size_t(max_seq) * D * 4), sn(size_t(max_seq) * D * 4);
    auto hx = fill_normal(x, 21);
    std::vector<float> gamma(D);
    for (int i = 0; i < D; ++i) gamma[i] = 0.5f + float(i) / D;
    to_device(w.p, gamma);

    Tensor X = make_tensor(x.p, {1, H, S, D}), W = make_tensor(w.p, {D, 0, 0, 0}, DataType::GGML_TYPE_F32);
    Tensor norm = make_tensor(y.p, {1, H, S, D});
    norm.op_type = OperationType::OP_TYPE_RMS_NORM;
    norm.src = {&X, &W, nullptr, nullptr, nullptr, nullptr};
    norm.op_params = {1e-6f, 0, 0, 0};
    Tensor cos_t = make_tensor(cs.p, {max_seq, D, 0, 0}, DataType::GGML_TYPE_F32),
           sin_t = make_tensor(sn.p, {max_seq, D, 0, 0}, DataType::GGML_TYPE_F32);
    cos_t.op_type = sin_t.op_type = OperationType::OP_TYPE_ROPE_CACHE;
    cos_t.op_params = sin_t.op_params = {1e6f, float(D), float(max_seq), 0};
    cos_t.name = "rope_cos";
    sin_t.name = "rope_sin";
    Tensor rope = make_tensor(r.p, {1, H, S, D});
    rope.op_type = OperationType::OP_TYPE_APPLY_ROPE;
    rope.src = {&norm, &cos_t, &sin_t, nullptr, nullptr, nullptr};
    rope.op_params = {float(D), float(D), float(start), 0};
    for (Tensor* t : {&norm, &cos_t, &sin_t, &rope}) CHECK_TRUE(c, kernel::dispatch(t, 0), "dispatched");

    std::vector<float> rc(size_t(max_seq) * D), rs(size_t(max_seq) * D);
    or_rope_cache(rc.data(), 1e6f, D, max_seq, 1);
    or_rope_cache(rs.data(), 1e6f, D, max_seq, 0);
    CHECK_TRUE(c, to_host<float>(cs.p, rc.size()) == rc, "cos table bit-exact");
    CHECK_TRUE(c, to_host<float>(sn.p, rs.size()) == rs, "sin table bit-exact");
    std::vector<uint16_t> yn(hx.size()), yr(hx.size());
    or_rms_norm(yn.data(), hx.data(), gamma.data(), size_t(H) * S, D, 1e-6f);
    CHECK_TRUE(c, to_host<uint16_t>(y.p, yn.size()) == yn, "rms_norm bit-exact");
    or_apply_rope(yr.data(), yn.data(), rc.data(), rs.data(), H, S, D, start);
    CHECK_TRUE(c, to_host<uint16_t>(r.p, yr.size()) == yr, "apply_rope bit-exact");
}

// ------------------------------------------------------------------- Linear
// LINEAR node (linear.cpp:325-345): decode-sized M bit-exact against the
// oracle's restatement of the reference's summation order; a prefill-sized M
// through the GEMM path within one bf16 rounding of it.
void run_linear(check::Context& c, int64_t M, int64_t common, int64_t cols, bool with_bias, uint64_t seed, bool exact) {
    MemoryManager mm;
    DevBuf x(size_t(M * common * 2)), w(size_t(cols * common * 2)), b(size_t(cols * 2)), o(size_t(M * cols * 2));
    auto hx = fill_normal(x, seed), hw = fill_normal(w, seed + 1), hb = fill_normal(b, seed + 2);
    Tensor X = make_tensor(x.p, {1, M, common, 0}), W = make_tensor(w.p, {cols, common, 0, 0}),
           Bv = make_tensor(b.p, {cols, 0, 0, 0});
    Tensor out = make_tensor(o.p, {1, M, cols, 0});
    out.op_type = OperationType::OP_TYPE_LINEAR;
    out.src = {&X, &W, with_bias ? &Bv : nullptr, nullptr, nullptr, nullptr};
    out.op_params = {1.0f, 0, 0, 0};  // transpose_w
    const size_t ws = op_workspace_bytes({&out}, Device::HIP, M);
    if (ws > 0) {
        // the op never allocates: without the reserved workspace it refuses
        bool threw = false;
        try {
            kernel::dispatch(&out, 0);
        } catch (const std::runtime_error&) {
            threw = true;
        }
        CHECK_TRUE(c, threw, "linear GEMM with a bias refuses to run without a reserved op workspace");
        mm.reserve_op_workspace(Device::HIP, 0, ws);
    }
    CHECK_TRUE(c, kernel::dispatch(&out, 0), "executor dispatches LINEAR");
    std::vector<uint16_t> want(size_t(M * cols));
    or_linear_bf16(want.data(), hx.data(), hw.data(), M, common, cols, with_bias ? hb.data() : nullptr);
    const auto got = to_host<uint16_t>(o.p, want.size());
    if (exact) {
        CHECK_TRUE(c, got == want, "linear bit-exact against the oracle");
    } else {
        // both sides are one bf16 rounding of an fp32 sum: |got - want| <= one
        // bf16 ulp of the larger plus twice the fp32 accumulation bound
        // common * 2^-24 * sum_k |x_k w_k|
        size_t far = 0;
        for (int64_t r = 0; r < M; ++r)
            for (int64_t c = 0; c < cols; ++c) {
                double mag = with_bias ? std::abs(double(or_bf16_to_f32(hb[c]))) : 0.0;
                for (int64_t k = 0; k < common; ++k)
                    mag += std::abs(double(or_bf16_to_f32(hx[r * common + k])) * or_bf16_to_f32(hw[c * common + k]));
                const double a = or_bf16_to_f32(got[r * cols + c]), b = or_bf16_to_f32(want[r * cols + c]);
                const double big = std::max(std::abs(a), std::abs(b));
                const double ulp = std::ldexp(1.0, std::ilogb(std::max(big, 1e-38)) - 7);
                if (std::abs(a - b) > ulp + 2.0 * double(common) * std::ldexp(1.0, -24) * mag) ++far;
            }
        CHECK_TRUE(c, far == 0, "linear GEMM within one bf16 rounding + fp32 accumulation error of the oracle");
    }
}

void test_linear_decode(check::Context& c) {
    run_linear(c, 1, 2560, 1024, false, 31, true);
    if (c.ok()) run_linear(c, 3, 1024, 300, true, 32, true);
}
void test_linear_prefill(check::Context& c) {
    run_linear(c, 64, 1024, 512, true, 33, false);
    if (c.ok()) run_linear(c, 64, 1024, 512, false, 34, false);
}

// Host cost of one PAGED_ATTN dispatch at config 3's shape (Qwen3-4B heads,
// 8192 cached tokens, one decode token): `calls` dispatches back to back
// through kernel::dispatch, timed on the host without synchronising while the
// GPU runs them (host bookkeeping, the split plan and two kernel launches).
// Prints one JSON line.
int host_cost(int calls) {
    const int32_t Hq = 32, Hkv = 8, D = 128, G = Hq / Hkv, cached = 8192;
    const int32_t max_seq = cached + calls + 64;
    MemoryManager mm;
    Tensor kproto = make_tensor(nullptr, {1, Hkv, 1, D});
    Tensor proto = make_tensor(nullptr, {1, Hq, 1, D});
    proto.op_type = OperationType::OP_TYPE_PAGED_ATTN;
    proto.src[1] = &kproto;
    proto.layer_id = 0;
    std::vector<Tensor*> graph{&proto};
    PagedAttentionManager& pam =
        mm.create_attention_manager(Device::HIP, 0, kv_cache_bytes(graph, Device::HIP, max_seq));
    initialize_kv_cache(pam, graph, max_seq);
    pam.append_kv_pages(0, cached);
    DevBuf q(size_t(Hq) * D * 2), k(size_t(Hkv) * D * 2), v(size_t(Hkv) * D * 2), o(size_t(Hq) * D * 2);
    fill_normal(q, 1);
    fill_normal(k, 2);
    fill_normal(v, 3);
    Tensor Q = make_tensor(q.p, {1, Hq, 1, D}), K = make_tensor(k.p, {1, Hkv, 1, D}), V = make_tensor(v.p, {1, Hkv, 1, D});
    Tensor out = make_tensor(o.p, {1, Hq, 1, D});
    out.op_type = OperationType::OP_TYPE_PAGED_ATTN;
    out.layer_id = 0;
    out.src = {&Q, &K, &V, nullptr, nullptr, nullptr};
    out.op_params = {float(D), 1.0f / std::sqrt(float(D)), 1.0f, float(G)};
    for (int i = 0; i < 16; ++i)
        if (!kernel::dispatch(&out, 0)) return 1;
    if (hipDeviceSynchronize() != hipSuccess) return 1;
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < calls; ++i)
        if (!kernel::dispatch(&out, 0)) return 1;
    const auto t1 = std::chrono::steady_clock::now();
    if (hipDeviceSynchronize() != hipSuccess) return 1;
    if (pam.get_layer(0).num_cached != cached + 16 + calls) {  // every call appended its token
        std::printf("host cost: the op did not run (num_cached %d)\n", pam.get_layer(0).num_cached);
        return 1;
    }
    const double us = std::chrono::duration<double, std::micro>(t1 - t0).count() / calls;
    std::printf("{\"host_us_per_call\": %.3f, \"calls\": %d, \"shape\": \"Hq %d, Hkv %d, D %d, %d+ cached\"}\n", us,
                calls, Hq, Hkv, D, cached);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
        std::printf("no HIP device\n");
        return 2;
    }
    if (argc == 3 && std::strcmp(argv[1], "--host-cost") == 0) return host_cost(std::max(1, std::atoi(argv[2])));
    return check::main({
        {"device enum", test_device_enum},
        {"block_pool alloc/free", test_block_pool_alloc_free},
        {"block_pool many allocs", test_block_pool_many_allocs},
        {"block_pool reset", test_block_pool_reset},
        {"page_table append_kv", test_page_table_append_kv},
        {"page_table multi layer", test_page_table_multi_layer},
        {"get_layer edit in place", test_get_layer_edit_in_place},
        {"kv_cache_per_layer switch + sizing", test_kv_cache_per_layer_switch},
        {"paged attention graph Qwen3-0.6B shape", test_paged_attention_qwen06b},
        {"paged attention graph Qwen3-4B shape", test_paged_attention_qwen4b},
        {"paged attention errors", test_paged_attention_errors},
        {"decode step graph (device position)", test_decode_step_graph},
        {"flash attention causal", test_flash_attention_causal},
        {"flash attention full", test_flash_attention_full},
        {"flash attention one token", test_flash_attention_one_token},
        {"rms_norm / rope_cache / apply_rope nodes", test_rms_norm_rope_nodes},
        {"linear node, decode rows (bit-exact)", test_linear_decode},
        {"linear node, prefill rows (GEMM)", test_linear_prefill},
    }, argc, argv);
}
