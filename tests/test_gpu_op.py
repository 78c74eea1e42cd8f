"""The op end to end: genllm_paged_attention (PagedAttentionImpl<HIP>::execute)
against the oracle's PagedAttentionImpl<CPU>::execute over a prefill /
decode / append_tokens sequence, with the reference's state semantics (LIFO
block pools, separate K/V ids, append-then-attend, reset), and its error paths."""
import numpy as np
import pytest
import torch

from genllm_amd import paged, synth
from genllm_amd._lib import ERR_INVALID, ERR_POOL_FULL, ERR_UNSUPPORTED, GenllmError
from helpers import assert_attn_close, oracle_fragmented, scale_for

pytestmark = pytest.mark.gpu


def make(orc, Hkv, D, pool, seed, layer=0):
    perm_k, perm_v = synth.shuffled(seed, pool), synth.shuffled(seed + 1, pool)
    mgr = paged.PagedAttentionManager(2 * pool * 16 * Hkv * D * 2 + (1 << 20))
    mgr.init_layer(layer, Hkv, D)
    mgr.reserve_layer(layer, pool)
    mgr.fragment(layer, perm_k, perm_v)
    ref = oracle_fragmented(orc, Hkv, D, pool, perm_k, perm_v, layer)
    return mgr, ref


def step(mgr, ref, layer, Hq, Hkv, S, D, seed, label):
    G = Hq // Hkv
    q = synth.normal_bf16(seed, (1, Hq, S, D))
    k = synth.normal_bf16(seed + 1, (1, Hkv, S, D))
    v = synth.normal_bf16(seed + 2, (1, Hkv, S, D))
    out = torch.zeros((1, Hq, S, D), dtype=torch.bfloat16, device="cuda")
    print(f"op step {label}: S={S}", flush=True)
    paged.paged_attention(mgr, layer, paged.to_device_bf16(q), paged.to_device_bf16(k), paged.to_device_bf16(v), out,
                          G, scale_for(D))
    torch.cuda.synchronize()
    want, rc = ref.paged_attention(layer, q, k, v, G, scale_for(D))
    assert rc == 0
    assert_attn_close(paged.to_host_bits(out), want, label)
    kt, vt = mgr.page_table(layer)
    rk, rv = ref.page_table(layer)
    assert np.array_equal(kt, rk) and np.array_equal(vt, rv)
    assert mgr.get_layer(layer).num_cached == ref.num_cached(layer)


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (16, 8)])
def test_op_prefill_decode_append_sequence(orc, Hq, Hkv):
    D, pool = 128, 24
    mgr, ref = make(orc, Hkv, D, pool, 11 + Hq)
    seed = 500
    step(mgr, ref, 0, Hq, Hkv, 40, D, seed, "prefill 40")              # MFMA prefill path
    for i in range(20):                                                # decode, crossing pages 3 and 4
        step(mgr, ref, 0, Hq, Hkv, 1, D, seed + 10 * (i + 1), f"decode {41 + i}")
    step(mgr, ref, 0, Hq, Hkv, 16 // (Hq // Hkv), D, seed + 999, "append_tokens")  # short chunk: decode kernel
    step(mgr, ref, 0, Hq, Hkv, 100, D, seed + 1999, "append 100")      # chunked prefill on a warm cache
    # the op appends K/V unmodified: both pools equal the oracle's bit for bit
    assert np.array_equal(mgr.read_pool(0, 0), ref.pool_array(0, 0))
    assert np.array_equal(mgr.read_pool(0, 1), ref.pool_array(0, 1))
    # reset: host state rewinds like the reference; the next step reuses pages LIFO
    mgr.reset()
    ref.reset()
    step(mgr, ref, 0, Hq, Hkv, 1, D, seed + 7, "after reset")
    mgr.close()


def test_op_config3_decode_with_append(orc):
    """Qwen3-4B decode at 8K context -- 512 full pages from a
    shuffled 2048-page pool, append one token at 8192 (opens page 513), attend
    over 8193 keys."""
    seed = synth.config_seed(3)
    Hq, Hkv, D, pool, N = 32, 8, 128, 2048, 8192
    mgr, ref = make(orc, Hkv, D, pool, seed)
    mgr.append_kv_pages(0, N)
    ref.append_kv_pages(0, N)
    kp = synth.normal_bf16(seed + 2, (pool, 16, Hkv, D))
    vp = synth.normal_bf16(seed + 3, (pool, 16, Hkv, D))
    ref.pool_array(0, 0)[:] = kp
    ref.pool_array(0, 1)[:] = vp
    mgr.write_pool(0, 0, kp)
    mgr.write_pool(0, 1, vp)
    step(mgr, ref, 0, Hq, Hkv, 1, D, seed + 4, "config3")
    assert mgr.get_layer(0).num_pages == 513
    # the same op with one split of all pages: each wave walks 129 pages, three
    # blocks of page ids, and the wave that reads the last page writes the
    # appended token through the ids it loaded that page with
    with paged.decode_tuned(600):
        for i in range(3):
            step(mgr, ref, 0, Hq, Hkv, 1, D, seed + 5 + i, f"config3, one split, step {i}")
    assert np.array_equal(mgr.read_pool(0, 0), ref.pool_array(0, 0)), "K pages"
    assert np.array_equal(mgr.read_pool(0, 1), ref.pool_array(0, 1)), "V pages"
    # split workgroups reading 4 kv heads each (the long-context plan, forced
    # here): the wave of each head that reads the last page writes that
    # head's appended token
    with paged.decode_tuned(0, "kernel", 4):
        for i in range(3):
            step(mgr, ref, 0, Hq, Hkv, 1, D, seed + 15 + i, f"config3, 4 kv heads per workgroup, step {i}")
        with paged.decode_tuned(7, "kernel", 4):
            step(mgr, ref, 0, Hq, Hkv, 1, D, seed + 19, "config3, 4 kv heads per workgroup, 7 pages per split")
    assert np.array_equal(mgr.read_pool(0, 0), ref.pool_array(0, 0)), "K pages (4 heads)"
    assert np.array_equal(mgr.read_pool(0, 1), ref.pool_array(0, 1)), "V pages (4 heads)"
    mgr.close()


def test_op_errors_and_noops(orc):
    D, Hkv = 128, 8
    mgr, ref = make(orc, Hkv, D, 2, 3)
    q = paged.to_device_bf16(synth.normal_bf16(1, (1, 16, 1, D)))
    kv = paged.to_device_bf16(synth.normal_bf16(2, (1, Hkv, 1, D)))
    out = torch.zeros((1, 16, 1, D), dtype=torch.bfloat16, device="cuda")
    # inactive layer: silent no-op, output untouched (attention.cpp:127)
    paged.paged_attention(mgr, 7, q, kv, kv, out, 2, 0.1)
    torch.cuda.synchronize()
    assert not out.float().abs().sum().item()
    # head_dim != 128 is unsupported (attention.cu:511)
    q64 = torch.zeros((1, 16, 1, 64), dtype=torch.bfloat16, device="cuda")
    kv64 = torch.zeros((1, Hkv, 1, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(GenllmError) as e:
        paged.paged_attention(mgr, 0, q64, kv64, kv64, q64.clone(), 2, 0.1)
    assert e.value.code == ERR_UNSUPPORTED
    # groups inconsistent with the head counts
    with pytest.raises(GenllmError) as e:
        paged.paged_attention(mgr, 0, q, kv, kv, out, 3, 0.1)
    assert e.value.code == ERR_INVALID
    # pool exhaustion: 2 pages hold 32 tokens; the 33rd is refused, state unchanged
    big_q = paged.to_device_bf16(synth.normal_bf16(3, (1, 16, 32, D)))
    big_kv = paged.to_device_bf16(synth.normal_bf16(4, (1, Hkv, 32, D)))
    big_out = torch.zeros_like(big_q)
    paged.paged_attention(mgr, 0, big_q, big_kv, big_kv, big_out, 2, 0.1)
    before = (mgr.get_layer(0).num_cached, mgr.page_table(0))
    with pytest.raises(GenllmError) as e:
        paged.paged_attention(mgr, 0, q, kv, kv, out, 2, 0.1)
    assert e.value.code == ERR_POOL_FULL
    after = (mgr.get_layer(0).num_cached, mgr.page_table(0))
    assert before[0] == after[0] == 32 and np.array_equal(before[1][0], after[1][0])
    # set_page_table refuses ids the pool never handed out
    with pytest.raises(GenllmError):
        mgr.set_page_table(0, [5], [0], 16)
    torch.cuda.synchronize()
    mgr.close()


def test_manager_state_machine_matches_oracle(orc):
    """Host state only (no kernels): the reference's unit-test sequences on the
    product's manager."""
    mgr = paged.PagedAttentionManager(1 << 20)
    mgr.init_layer(0, 8, 128)
    assert mgr.is_active(0) and not mgr.is_active(2)
    mgr.append_kv_pages(0, 1)   # no reserved pools: page logic only, like the pool-less fake
    assert mgr.get_layer(0).num_cached == 1
    mgr.append_kv_pages(0, 31)
    assert mgr.get_layer(0).num_cached == 32 and mgr.get_layer(0).num_pages == 2
    mgr.init_layer(1, 4, 64, 0)
    mgr.append_kv_pages(1, 20)
    mgr.reset()
    assert mgr.get_layer(0).num_cached == 0 and mgr.get_layer(1).num_pages == 0
    # block pools: ids 0,1, reuse of a freed id, LIFO after reset
    mgr.init_layer(3, 8, 128)
    mgr.reserve_layer(3, 10)
    assert [mgr.block_alloc(3, 0) for _ in range(3)] == [0, 1, 2]
    mgr.block_free(3, 0, 1)
    assert mgr.block_alloc(3, 0) == 1
    mgr.reset()
    assert mgr.block_alloc(3, 0) == 2
    for _ in range(9):
        mgr.block_alloc(3, 1)
    mgr.block_alloc(3, 1)
    assert mgr.block_alloc(3, 1) == -1
    mgr.close()


def test_op_qwen35_decode_with_append(orc):
    """The op at the Qwen3.5 attention shape (head_dim 256, 8 q / 2 kv heads):
    a warm cache of 150 tokens, then decode steps that append and attend
    (crossing a page boundary) and a short chunk."""
    Hq, Hkv, D, pool = 8, 2, 256, 30
    mgr, ref = make(orc, Hkv, D, pool, 77)
    mgr.append_kv_pages(0, 150)
    ref.append_kv_pages(0, 150)
    kp = synth.normal_bf16(78, (pool, 16, Hkv, D))
    vp = synth.normal_bf16(79, (pool, 16, Hkv, D))
    ref.pool_array(0, 0)[:] = kp
    ref.pool_array(0, 1)[:] = vp
    mgr.write_pool(0, 0, kp)
    mgr.write_pool(0, 1, vp)
    for i in range(12):
        step(mgr, ref, 0, Hq, Hkv, 1, D, 800 + 10 * i, f"qwen35 decode {151 + i}")
    step(mgr, ref, 0, Hq, Hkv, 4, D, 990, "qwen35 chunk of 4")
    assert np.array_equal(mgr.read_pool(0, 0), ref.pool_array(0, 0))
    assert np.array_equal(mgr.read_pool(0, 1), ref.pool_array(0, 1))
    mgr.close()


def test_op_qwen35_prefill_decode_sequence(orc):
    """The op at the Qwen3.5 shape through every kernel: a 70-token prefill (the
    D = 256 MFMA prefill), decode steps (split-K decode with the append fused)
    and a 40-token chunk on the warm cache."""
    Hq, Hkv, D, pool = 8, 2, 256, 16
    mgr, ref = make(orc, Hkv, D, pool, 91)
    step(mgr, ref, 0, Hq, Hkv, 70, D, 1200, "qwen35 prefill 70")
    for i in range(5):
        step(mgr, ref, 0, Hq, Hkv, 1, D, 1300 + 10 * i, f"qwen35 decode {71 + i}")
    step(mgr, ref, 0, Hq, Hkv, 40, D, 1400, "qwen35 chunk 40")
    assert np.array_equal(mgr.read_pool(0, 0), ref.pool_array(0, 0))
    assert np.array_equal(mgr.read_pool(0, 1), ref.pool_array(0, 1))
    mgr.close()


def layer_snapshot(mgr, layer):
    """Host state, device page table and pool counters of a layer."""
    i = mgr.get_layer(layer)
    kt, vt = mgr.page_table(layer)
    dk, dv = mgr.read_device_table(layer)
    return (i.num_cached, i.num_pages, i.k_num_blocks, i.k_num_free, i.v_num_blocks, i.v_num_free,
            kt.tolist(), vt.tolist(), dk.tolist(), dv.tolist())


@pytest.mark.parametrize("S", [1, 40])
def test_op_errors_leave_layer_unchanged(orc, S):
    """A call the op refuses (misaligned q, NaN scale, a head-count mismatch)
    changes nothing: num_cached, the host and device page tables and the block
    pools are as before, and the next valid call matches the oracle.  Decode
    (S = 1, the fused append) and prefill (S = 40, separate append kernel)."""
    D, Hkv, Hq = 128, 8, 32
    mgr, ref = make(orc, Hkv, D, 16, 77 + S)
    step(mgr, ref, 0, Hq, Hkv, 31, D, 900, "prefill 31")   # next token opens page 2
    before = layer_snapshot(mgr, 0)
    buf = torch.zeros(Hq * S * D + 8, dtype=torch.bfloat16, device="cuda")
    q_mis = buf[1:1 + Hq * S * D].view(1, Hq, S, D)          # 2-byte offset: not 16-byte aligned
    q = paged.to_device_bf16(synth.normal_bf16(5, (1, Hq, S, D)))
    kv = paged.to_device_bf16(synth.normal_bf16(6, (1, Hkv, S, D)))
    out = torch.zeros((1, Hq, S, D), dtype=torch.bfloat16, device="cuda")
    for label, args in (("misaligned q", (q_mis, kv, kv, out, Hq // Hkv, 0.1)),
                        ("NaN scale", (q, kv, kv, out, Hq // Hkv, float("nan"))),
                        ("infinite scale", (q, kv, kv, out, Hq // Hkv, float("inf")))):
        with pytest.raises(GenllmError) as e:
            paged.paged_attention(mgr, 0, *args)
        assert e.value.code == ERR_INVALID, label
        torch.cuda.synchronize()
        assert layer_snapshot(mgr, 0) == before, f"{label} changed the layer"
    step(mgr, ref, 0, Hq, Hkv, S, D, 901, "valid call after the errors")
    assert np.array_equal(mgr.read_pool(0, 0), ref.pool_array(0, 0))
    assert np.array_equal(mgr.read_pool(0, 1), ref.pool_array(0, 1))
    mgr.close()


def test_reserve_fits_exact_scheduler_sizing(orc):
    """The kv_cache pool sized exactly as the reference scheduler does
    (2 * max_blocks * block_bytes per layer, scheduler.cpp:62-79, 371) holds
    every layer's pools: the device page tables and the decode workspace live
    outside it.  One byte less and the last reserve_layer fails."""
    from genllm_amd._lib import ERR_NO_MEMORY
    Hq, Hkv, D, L, max_blocks = 32, 8, 128, 3, 40
    exact = L * 2 * max_blocks * 16 * Hkv * D * 2
    mgr = paged.PagedAttentionManager(exact)
    for l in range(L):
        mgr.init_layer(l, Hkv, D)
        mgr.reserve_layer(l, max_blocks)
    # the last layer's pools work: prefill chunks, then decode steps crossing a page
    ref = orc.Manager(with_pool=True)
    ref.init_layer(L - 1, Hkv, D)
    ref.reserve_layer(L - 1, max_blocks)
    for i, S in enumerate((17, 14, 1, 1)):
        step(mgr, ref, L - 1, Hq, Hkv, S, D, 40 + i, f"exact-size step {i} S={S}")
    mgr.close()
    short = paged.PagedAttentionManager(exact - 1)
    for l in range(L - 1):
        short.init_layer(l, Hkv, D)
        short.reserve_layer(l, max_blocks)
    short.init_layer(L - 1, Hkv, D)
    with pytest.raises(GenllmError) as e:
        short.reserve_layer(L - 1, max_blocks)
    assert e.value.code == ERR_NO_MEMORY
    short.close()


def test_reserve_refuses_workspace_growth_while_staged(orc):
    """A layer whose decode plans need a larger workspace is refused while
    another layer is staged for device-position steps (a captured step holds
    the workspace's address): GENLLM_ERR_INVALID, and nothing of the call is
    kept -- the pool cursor is where it was, so after sync the same reserve
    succeeds and the new layer's pools work."""
    Hq, Hkv, D = 32, 8, 128
    small, big = 8, 600
    mgr = paged.PagedAttentionManager(2 * (small + big) * 16 * Hkv * D * 2)
    mgr.init_layer(0, Hkv, D)
    mgr.reserve_layer(0, small)
    mgr.append_kv_pages(0, 20)
    mgr.stage_decode(0, 8)
    mgr.init_layer(1, Hkv, D)
    with pytest.raises(GenllmError) as e:
        mgr.reserve_layer(1, big)
    assert e.value.code == ERR_INVALID and "staged" in str(e.value)
    assert mgr.get_layer(1).max_blocks == 0
    assert mgr.sync_decode(0) == 20
    mgr.reserve_layer(1, big)  # fits: the refused call carved nothing
    assert mgr.get_layer(1).max_blocks == big
    ref = orc.Manager(with_pool=True)
    ref.init_layer(1, Hkv, D)
    ref.reserve_layer(1, big)
    for i, S in enumerate((40, 1)):
        step(mgr, ref, 1, Hq, Hkv, S, D, 60 + i, f"after the refused reserve, step {i}")
    mgr.close()


def test_append_kv_from_pos_matches_oracle(orc):
    """append_kv_from_pos (page_attention.cpp:164-203) through the product
    manager against the oracle: writing from position 0, rewriting positions
    inside the cache across a multiple of 16 (a block is still taken there),
    extending past the end (page opened at 48), an unaligned append that opens
    the page at 64; then the refusals -- a position whose page is neither in
    the table nor opened by the call, a pool without enough pages -- leave the
    layer as it was; finally a decode step attends over the rewritten cache."""
    Hq, Hkv, D, pool = 32, 8, 128, 8
    mgr, ref = make(orc, Hkv, D, pool, 7070)

    def put(g0, count, seed):
        K = synth.normal_bf16(seed, (Hkv, count, D))
        V = synth.normal_bf16(seed + 1, (Hkv, count, D))
        print(f"append_kv_from_pos({g0}, {count})", flush=True)
        mgr.append_kv_from_pos(0, paged.to_device_bf16(K), paged.to_device_bf16(V), g0)
        ref.append_kv_from_pos(0, K, V, g0)

    def same(label):
        torch.cuda.synchronize()
        info = mgr.get_layer(0)
        assert info.num_cached == ref.num_cached(0), label
        kt, vt = mgr.page_table(0)
        rk, rv = ref.page_table(0)
        assert np.array_equal(kt, rk) and np.array_equal(vt, rv), label
        assert (info.k_num_blocks, info.k_num_free) == (ref.pool(0, 0).num_blocks(), ref.pool(0, 0).num_free())
        assert (info.v_num_blocks, info.v_num_free) == (ref.pool(0, 1).num_blocks(), ref.pool(0, 1).num_free())
        assert np.array_equal(mgr.read_pool(0, 0), ref.pool_array(0, 0)), label
        assert np.array_equal(mgr.read_pool(0, 1), ref.pool_array(0, 1)), label
        dk, dv = mgr.read_device_table(0)
        assert np.array_equal(dk, rk) and np.array_equal(dv, rv), label

    put(0, 40, 10)
    same("write 0..39")
    put(10, 9, 20)
    same("rewrite 10..18")
    put(40, 13, 30)
    same("extend 40..52")
    put(53, 20, 40)
    same("append 53..72")

    before = (mgr.get_layer(0).num_cached, mgr.page_table(0), mgr.read_pool(0, 0))
    K = paged.to_device_bf16(synth.normal_bf16(50, (Hkv, 5, D)))
    with pytest.raises(GenllmError) as e:  # page 6 (position 100) is not in the 5-page table
        mgr.append_kv_from_pos(0, K, K, 100)
    assert e.value.code == ERR_INVALID
    K2 = paged.to_device_bf16(synth.normal_bf16(51, (Hkv, 60, D)))
    with pytest.raises(GenllmError) as e:  # 80..139 takes 4 blocks per pool; 2 are left (6 of 8 taken)
        mgr.append_kv_from_pos(0, K2, K2, 80)
    assert e.value.code == ERR_POOL_FULL
    torch.cuda.synchronize()
    after = (mgr.get_layer(0).num_cached, mgr.page_table(0), mgr.read_pool(0, 0))
    assert before[0] == after[0] and np.array_equal(before[1][0], after[1][0])
    assert np.array_equal(before[2], after[2])
    same("after the refusals")
    step(mgr, ref, 0, Hq, Hkv, 1, D, 60, "decode over the rewritten cache")
    mgr.close()
