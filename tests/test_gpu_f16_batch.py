"""The op (genllm_paged_attention) on fp16 layers and with batch > 1, against
the oracle op on the same seeded inputs.

fp16: the reference reads K/V as Q's dtype and stores out through float16_t
(attention.cpp:186-200, dtype_traits.hpp:52-69, float16.hpp); the decode and
prefill kernels run the fp16 MFMAs.  Page tables and pools bit-exact, outputs
within max-abs <= 2^-8 max|ref| and rel-L2 <= 4e-3 (fp16 outputs).  Shapes:
Qwen3-0.6B (config 1: 1024 cached, 16 q / 8 kv heads), Qwen3-4B (config 3:
8192 cached, one appended token), Qwen3.5 (head_dim 256).

batch > 1: every batch entry attends the layer's one cache and only the first
entry's k/v rows are appended (attention.cpp:146, 156)."""
import numpy as np
import pytest
import torch

from genllm_amd import paged, synth
from helpers import assert_attn_close, assert_attn_close_f16, scale_for

pytestmark = pytest.mark.gpu


def make(orc, Hkv, D, pool, seed, dtype):
    perm_k, perm_v = synth.shuffled(seed, pool), synth.shuffled(seed + 1, pool)
    mgr = paged.PagedAttentionManager(2 * pool * 16 * Hkv * D * 2 + (1 << 20))
    mgr.init_layer(0, Hkv, D, dtype)
    mgr.reserve_layer(0, pool)
    mgr.fragment(0, perm_k, perm_v)
    ref = orc.Manager(with_pool=True)
    ref.init_layer(0, Hkv, D, dtype)
    ref.reserve_layer(0, pool)
    for which, perm in ((0, perm_k), (1, perm_v)):
        p = ref.pool(0, which)
        for _ in range(pool):
            p.alloc()
        for b in perm[::-1]:
            p.free(int(b))
    return mgr, ref


def step(orc, mgr, ref, Hq, Hkv, S, D, seed, label, f16=True, batch=1):
    G = Hq // Hkv
    gen = synth.normal_f16 if f16 else synth.normal_bf16
    dev = paged.to_device_f16 if f16 else paged.to_device_bf16
    q = gen(seed, (batch, Hq, S, D))
    k = gen(seed + 1, (batch, Hkv, S, D))
    v = gen(seed + 2, (batch, Hkv, S, D))
    out = torch.zeros((batch, Hq, S, D), dtype=torch.float16 if f16 else torch.bfloat16, device="cuda")
    print(f"op step {label}: batch={batch} S={S} {'fp16' if f16 else 'bf16'}", flush=True)
    paged.paged_attention(mgr, 0, dev(q), dev(k), dev(v), out, G, scale_for(D))
    torch.cuda.synchronize()
    want, rc = ref.paged_attention(0, q, k, v, G, scale_for(D), True, dtype=orc.F16 if f16 else orc.BF16)
    assert rc == 0
    got = paged.to_host_bits(out)
    (assert_attn_close_f16 if f16 else assert_attn_close)(got, want, label)
    kt, vt = mgr.page_table(0)
    rk, rv = ref.page_table(0)
    assert np.array_equal(kt, rk) and np.array_equal(vt, rv)
    assert mgr.get_layer(0).num_cached == ref.num_cached(0)
    return got


def check_pools(mgr, ref, label):
    assert np.array_equal(mgr.read_pool(0, 0), ref.pool_array(0, 0)), f"{label}: K pages"
    assert np.array_equal(mgr.read_pool(0, 1), ref.pool_array(0, 1)), f"{label}: V pages"


def test_f16_op_config1_shape(orc):
    """Qwen3-0.6B heads: a 1024-token prefill chunk through the op (append, then
    the fp16 prefill kernel), then decode steps (fused append + the fp16 split
    kernel) across a page boundary."""
    Hq, Hkv, D, pool = 16, 8, 128, 256
    mgr, ref = make(orc, Hkv, D, pool, synth.config_seed(1), orc.F16)
    step(orc, mgr, ref, Hq, Hkv, 1024, D, 100, "f16 prefill 1024")
    for i in range(17):
        step(orc, mgr, ref, Hq, Hkv, 1, D, 200 + 3 * i, f"f16 decode {1025 + i}")
    check_pools(mgr, ref, "f16 config1")
    mgr.close()


def test_f16_op_config3_shape(orc):
    """Qwen3-4B heads at 8K: 512 full pages of fp16 K/V in a shuffled 2048-page
    pool, then the op appends a token at 8192 (opening page 513) and attends
    over 8193 keys, twice."""
    Hq, Hkv, D, pool, N = 32, 8, 128, 2048, 8192
    seed = synth.config_seed(3) + 16
    mgr, ref = make(orc, Hkv, D, pool, seed, orc.F16)
    mgr.append_kv_pages(0, N)
    ref.append_kv_pages(0, N)
    kp = synth.normal_f16(seed + 2, (pool, 16, Hkv, D))
    vp = synth.normal_f16(seed + 3, (pool, 16, Hkv, D))
    ref.pool_array(0, 0)[:] = kp
    ref.pool_array(0, 1)[:] = vp
    mgr.write_pool(0, 0, kp)
    mgr.write_pool(0, 1, vp)
    step(orc, mgr, ref, Hq, Hkv, 1, D, seed + 4, "f16 config3 step 0")
    step(orc, mgr, ref, Hq, Hkv, 1, D, seed + 7, "f16 config3 step 1")
    assert mgr.get_layer(0).num_pages == 513
    check_pools(mgr, ref, "f16 config3")
    mgr.close()


def test_f16_op_head_dim_256(orc):
    """Qwen3.5 heads (8 q / 2 kv, head_dim 256): prefill chunk, then decode."""
    Hq, Hkv, D, pool = 8, 2, 256, 64
    mgr, ref = make(orc, Hkv, D, pool, 4321, orc.F16)
    step(orc, mgr, ref, Hq, Hkv, 300, D, 300, "f16 D256 prefill 300")
    for i in range(3):
        step(orc, mgr, ref, Hq, Hkv, 1, D, 400 + 3 * i, f"f16 D256 decode {301 + i}")
    check_pools(mgr, ref, "f16 D256")
    mgr.close()


def test_f16_special_values(orc):
    """Equal scores (q = 0), so the last query's output is the mean of V over
    its 20 keys, through float16_t: a NaN becomes an infinity (bit-equal to the
    oracle up to the sign, which NaN arithmetic does not fix), 65504 stays the
    largest finite value, a subnormal mean stays subnormal (gradual underflow,
    where bf16 would flush), a mean below half the smallest subnormal becomes
    zero -- bit-equal to the oracle op."""
    Hq, Hkv, D, pool = 2, 1, 128, 8
    mgr, ref = make(orc, Hkv, D, pool, 77, orc.F16)
    N = 20
    k = np.zeros((1, Hkv, N, D), dtype=np.uint16)
    v = np.zeros((1, Hkv, N, D), dtype=np.uint16)
    v[0, 0, :, 0] = np.float16(np.nan).view(np.uint16)
    v[0, 0, :, 1] = np.float16(65504.0).view(np.uint16)
    v[0, 0, :, 2] = np.uint16(0x0010)  # 16 x 2^-24: the mean is that subnormal
    v[0, 0, 0, 3] = np.uint16(0x0001)  # mean 2^-24 / 20 -> 0
    q = np.zeros((1, Hq, N, D), dtype=np.uint16)
    out = torch.zeros((1, Hq, N, D), dtype=torch.float16, device="cuda")
    paged.paged_attention(mgr, 0, paged.to_device_f16(q), paged.to_device_f16(k), paged.to_device_f16(v), out, 2,
                          scale_for(D))
    torch.cuda.synchronize()
    want, _ = ref.paged_attention(0, q, k, v, 2, scale_for(D), True, dtype=orc.F16)
    got = paged.to_host_bits(out)
    g, w = got[0, :, -1], want[0, :, -1]
    assert np.array_equal(g[:, 0] & 0x7FFF, w[:, 0] & 0x7FFF) and set((g[:, 0] & 0x7FFF).tolist()) == {0x7C00}
    assert np.array_equal(g[:, 1:4], w[:, 1:4]), (g[:, 1:4], w[:, 1:4])
    assert set(g[:, 1].tolist()) == {0x7BFF} and set(g[:, 2].tolist()) == {0x0010} and set(g[:, 3].tolist()) == {0}
    mgr.close()


def test_f16_decode_chunk_special_values(orc):
    """A 3-query decode chunk on fp16 layers whose own second key holds a NaN
    and a +inf in one V row (kv head 1): the chunk's first query does not see
    that key and stays finite, as in the reference; the two others get the
    reference's non-finite outputs (float16_t turns the NaN into an infinity;
    bit-equal up to the sign); every finite output is held to the fp16
    attention tolerance."""
    Hq, Hkv, D, pool, P, S = 4, 2, 128, 8, 30, 3
    G = Hq // Hkv
    mgr, ref = make(orc, Hkv, D, pool, 91, orc.F16)
    step(orc, mgr, ref, Hq, Hkv, P, D, 9100, "f16 prompt")
    q = synth.normal_f16(9200, (1, Hq, S, D))
    k = synth.normal_f16(9201, (1, Hkv, S, D))
    v = synth.normal_f16(9202, (1, Hkv, S, D)).copy()
    v[0, 1, 1, 5] = np.float16(np.nan).view(np.uint16)
    v[0, 1, 1, 7] = np.float16(np.inf).view(np.uint16)
    out = torch.zeros((1, Hq, S, D), dtype=torch.float16, device="cuda")
    paged.paged_attention(mgr, 0, paged.to_device_f16(q), paged.to_device_f16(k), paged.to_device_f16(v), out, G,
                          scale_for(D))
    torch.cuda.synchronize()
    want, rc = ref.paged_attention(0, q, k, v, G, scale_for(D), True, dtype=orc.F16)
    assert rc == 0
    got = paged.to_host_bits(out)
    w_nf = ~np.isfinite(want.view(np.float16))
    g_nf = ~np.isfinite(got.view(np.float16))
    assert np.array_equal(w_nf, g_nf), f"non-finite outputs at {np.argwhere(w_nf != g_nf)[:6]}"
    assert np.array_equal(got[w_nf] & 0x7FFF, want[w_nf] & 0x7FFF)
    heads = slice(G, 2 * G)  # the q heads of kv head 1
    assert not w_nf[0, heads, 0].any() and w_nf[0, heads, 1:][..., [5, 7]].all() and w_nf.sum() == 2 * 2 * 2
    assert_attn_close_f16(np.where(w_nf, 0, got).astype(np.uint16), np.where(w_nf, 0, want).astype(np.uint16),
                          "f16 decode chunk, finite outputs")
    mgr.close()


@pytest.mark.parametrize("f16", [False, True])
def test_batch2_entries_share_the_cache(orc, f16):
    """batch = 2 through the op: a 40-token prefill chunk, then decode steps;
    both entries attend the one cache, the first entry's k/v are appended."""
    Hq, Hkv, D, pool = 16, 8, 128, 24
    mgr, ref = make(orc, Hkv, D, pool, 99 + int(f16), orc.F16 if f16 else orc.BF16)
    step(orc, mgr, ref, Hq, Hkv, 40, D, 500, "batch2 prefill", f16=f16, batch=2)
    for i in range(3):
        step(orc, mgr, ref, Hq, Hkv, 1, D, 600 + 3 * i, f"batch2 decode {41 + i}", f16=f16, batch=2)
    check_pools(mgr, ref, "batch2")
    mgr.close()


def test_fill_normal_f16_matches_host_formula():
    """genllm_fill_normal_f16 (the benchmark's fp16 pools) against the host
    formula of genllm_amd/synth.py: the same samples within one fp16 rounding
    of each other (device and numpy libm differ by a few fp32 ulps)."""
    t = torch.empty(1 << 16, dtype=torch.float16, device="cuda")
    paged.fill_normal_f16(t, 1234, 77)
    torch.cuda.synchronize()
    got = paged.to_host_bits(t).view(np.float16).astype(np.float64)
    want = synth.normal_f16(1234, (1 << 16,), 77).view(np.float16).astype(np.float64)
    ulp = np.maximum(np.abs(want), 2.0 ** -14) * 2.0 ** -10
    assert np.all(np.abs(got - want) <= ulp), np.max(np.abs(got - want) / ulp)
    assert abs(want.mean()) < 0.02 and abs(want.std() - 1) < 0.02


@pytest.mark.parametrize("P,steps,merge", [(40, 12, "kernel"), (200, 6, "fused"), (40, 12, "heads4")])
def test_f16_device_position_step(orc, request, P, steps, merge):
    """fp16 layers through the device-position decode step: the step staged
    (genllm_kv_stage_decode), genllm_paged_attention_step captured once into a
    HIP graph and replayed token after token across a page boundary (and with
    the single-launch merge), each replay against the oracle's fp16 path at the
    host position, pools bit-exact; after genllm_kv_sync_decode the host page
    table and num_cached equal the oracle's."""
    if merge == "heads4":  # split workgroups reading 4 kv heads each
        paged.decode_tuning(0, "kernel", 4)
        request.addfinalizer(lambda: paged.decode_tuning(0, "kernel"))
    elif merge != "kernel":
        paged.decode_tuning(0, merge)
        request.addfinalizer(lambda: paged.decode_tuning(0, "kernel"))
    Hq, Hkv, D = 32, 8, 128
    G, pool = Hq // Hkv, (P + steps + 15) // 16 + 3
    mgr, ref = make(orc, Hkv, D, pool, 0x5EED0500 + P, orc.F16)
    step(orc, mgr, ref, Hq, Hkv, P, D, 12000 + P, f"f16 prompt {P}")
    dev = dict(dtype=torch.float16, device="cuda")
    q_in, out = torch.zeros((1, Hq, 1, D), **dev), torch.zeros((1, Hq, 1, D), **dev)
    k_in, v_in = torch.zeros((1, Hkv, 1, D), **dev), torch.zeros((1, Hkv, 1, D), **dev)
    mgr.stage_decode(0, steps)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        paged.paged_attention_step(mgr, 0, q_in, k_in, v_in, out, G, scale_for(D))
    for i in range(steps):
        print(f"f16 step replay {i}: position {P + i} ({merge} merge)", flush=True)
        q = synth.normal_f16(13000 + 10 * i, (1, Hq, 1, D))
        k = synth.normal_f16(13001 + 10 * i, (1, Hkv, 1, D))
        v = synth.normal_f16(13002 + 10 * i, (1, Hkv, 1, D))
        q_in.copy_(paged.to_device_f16(q))
        k_in.copy_(paged.to_device_f16(k))
        v_in.copy_(paged.to_device_f16(v))
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        want, rc = ref.paged_attention(0, q, k, v, G, scale_for(D), True, dtype=orc.F16)
        assert rc == 0
        assert_attn_close_f16(paged.to_host_bits(out), want, f"f16 step replay {i}")
        check_pools(mgr, ref, f"f16 step replay {i}")
    assert mgr.sync_decode(0) == P + steps
    kt, vt = mgr.page_table(0)
    rk, rv = ref.page_table(0)
    assert np.array_equal(kt, rk) and np.array_equal(vt, rv)
    assert mgr.get_layer(0).num_cached == ref.num_cached(0) == P + steps
    mgr.close()
