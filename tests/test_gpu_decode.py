"""GPU parity of the split-K paged decode kernel (genllm_paged_decode) against
the oracle's PagedAttentionImpl<CPU> attention loop, on identical pools and
block tables.  Tolerance (bf16 output, fp32 accumulate): max-abs <= 2^-7 *
max|ref| and rel-L2 <= 1e-2 (helpers.assert_attn_close)."""

import numpy as np
import pytest
import torch

from genllm_amd import paged, synth
from helpers import assert_attn_close, oracle_fragmented, scale_for

pytestmark = pytest.mark.gpu


class Context:
    """A GPU manager and an oracle manager holding the same n_ctx cached tokens
    in identically fragmented pools (pool contents random everywhere, so
    unfilled slots of the last page hold junk the kernels must ignore)."""

    def __init__(self, orc, Hkv, D, pool, n_ctx, seed, nan_tail=False):
        self.Hkv, self.D, self.pool = Hkv, D, pool
        perm_k, perm_v = synth.shuffled(seed, pool), synth.shuffled(seed + 1, pool)
        self.mgr = paged.PagedAttentionManager(2 * pool * 16 * Hkv * D * 2 + (1 << 20))
        self.mgr.init_layer(0, Hkv, D)
        self.mgr.reserve_layer(0, pool)
        self.mgr.fragment(0, perm_k, perm_v)
        self.mgr.append_kv_pages(0, n_ctx)
        self.ref = oracle_fragmented(orc, Hkv, D, pool, perm_k, perm_v)
        self.ref.append_kv_pages(0, n_ctx)
        kp = synth.normal_bf16(seed + 2, (pool, 16, Hkv, D))
        vp = synth.normal_bf16(seed + 3, (pool, 16, Hkv, D))
        self.ref.pool_array(0, 0)[:] = kp
        self.ref.pool_array(0, 1)[:] = vp
        if nan_tail and n_ctx % 16:
            kt, vt = self.ref.page_table(0)
            kp = kp.copy()
            vp = vp.copy()
            kp[kt[-1], n_ctx % 16:] = 0x7FC0  # NaN in the unfilled slots (GPU copy only)
            vp[vt[-1], n_ctx % 16:] = 0xFF80  # -inf
        self.mgr.write_pool(0, 0, kp)
        self.mgr.write_pool(0, 1, vp)
        kt, vt = self.mgr.page_table(0)
        rk, rv = self.ref.page_table(0)
        assert np.array_equal(kt, rk) and np.array_equal(vt, rv)
        self.info = self.mgr.get_layer(0)
        self.n_ctx = n_ctx

    def decode(self, q_bits, causal=True, pps=None, merge=None, heads=0):
        Hq, S, D = q_bits.shape
        out = torch.zeros((Hq, S, D), dtype=torch.bfloat16, device="cuda")
        n_pages = (self.n_ctx + 15) // 16
        ws = torch.zeros(paged.decode_workspace_bytes(Hq, self.Hkv, S, D, n_pages), dtype=torch.uint8,
                         device="cuda")
        with paged.decode_tuned(pps or 0, merge or "kernel", heads):
            info = self.info
            paged.paged_decode(paged.to_device_bf16(q_bits), out, info.k_pool, info.v_pool, info.k_ids, info.v_ids,
                               n_pages, self.n_ctx, self.Hkv, scale_for(D), ws, causal=causal)
            torch.cuda.synchronize()
        return paged.to_host_bits(out), ws

    def oracle(self, q_bits, causal=True):
        Hq, S, D = q_bits.shape
        out, rc = self.ref.paged_attend(0, q_bits[None], self.Hkv, Hq // self.Hkv, scale_for(D), causal)
        assert rc == 0
        return out[0]

    def close(self):
        self.mgr.close()


def test_decode_config1(orc):
    """Qwen3-0.6B shape, 1024 cached tokens = 64 pages of a
    randomly permuted 256-page pool, GQA 2:1."""
    seed = synth.config_seed(1)
    ctx = Context(orc, 8, 128, 256, 1024, seed)
    q = synth.normal_bf16(seed, (16, 1, 128), offset=7 << 28)
    got, _ = ctx.decode(q)
    assert_attn_close(got, ctx.oracle(q), "config1")
    ctx.close()


@pytest.mark.parametrize("Hq,Hkv,N", [(32, 8, 1), (32, 8, 15), (32, 8, 16), (32, 8, 17), (16, 8, 100),
                                      (8, 8, 33), (64, 8, 47), (32, 4, 250), (32, 8, 2049)])
def test_decode_shapes(orc, Hq, Hkv, N):
    pool = max(8, (N + 15) // 16 + 3)
    ctx = Context(orc, Hkv, 128, pool, N, 1000 + N + Hq, nan_tail=True)
    q = synth.normal_bf16(2000 + N, (Hq, 1, 128))
    got, ws = ctx.decode(q)
    assert_attn_close(got, ctx.oracle(q), f"Hq{Hq} Hkv{Hkv} N{N}")
    ctx.close()


@pytest.mark.parametrize("N", [131073, 262145])
def test_decode_very_long_context(orc, N):
    """131,073 and 262,145 cached keys (8,193 and 16,385 pages of a shuffled
    pool, the last page holding one key).  The default plan reads 4 kv heads
    per split workgroup: 65 pages per split over 127 splits (33 pages per
    wave), then 129 pages per split over 128 splits (65 pages per wave, two
    blocks of page ids)."""
    pool = (N + 15) // 16 + 7
    ctx = Context(orc, 8, 128, pool, N, N - 73, nan_tail=True)
    q = synth.normal_bf16(N - 72, (32, 1, 128))
    got, _ = ctx.decode(q)
    assert_attn_close(got, ctx.oracle(q), f"N{N}")
    ctx.close()


@pytest.mark.parametrize("pps", [1, 2, 4, 8, 1000])
def test_decode_split_plans(orc, pps):
    ctx = Context(orc, 8, 128, 80, 1000, 77)
    q = synth.normal_bf16(78, (32, 1, 128))
    got, _ = ctx.decode(q, pps=pps)
    assert_attn_close(got, ctx.oracle(q), f"pps{pps}")
    ctx.close()


@pytest.mark.parametrize("pps", [17, 32, 64, 128, 129, 200])
def test_decode_wave_forms(orc, pps):
    """Head_dim 128 splits of at most 128 pages run 8-wave workgroups, longer
    ones 4 waves; both forms against the oracle over 4100 keys (257 pages,
    the last one partial), with a fresh and a stale workspace."""
    ctx = Context(orc, 8, 128, 300, 4100, 91 + pps, nan_tail=True)
    q = synth.normal_bf16(92 + pps, (32, 1, 128))
    ref = ctx.oracle(q)
    got, _ = ctx.decode(q, pps=pps)
    assert_attn_close(got, ref, f"pps{pps}")
    got2, _ = ctx.decode(q, pps=pps)
    assert np.array_equal(got, got2)
    ctx.close()


@pytest.mark.parametrize("pps", [None, 1, 2, 7, 16, 64, 129])
def test_decode_four_heads_per_workgroup(orc, pps):
    """Split workgroups that read 4 kv heads of their pages (the plan for long
    page ranges; forced here at every split size, 2 waves per head) against
    the oracle over 4100 keys with a NaN/-inf tail past the cache end, twice
    on one workspace (bit-identical)."""
    ctx = Context(orc, 8, 128, 300, 4100, 191 + (pps or 0), nan_tail=True)
    q = synth.normal_bf16(192 + (pps or 0), (32, 1, 128))
    ref = ctx.oracle(q)
    got, _ = ctx.decode(q, pps=pps, heads=4)
    assert_attn_close(got, ref, f"4 heads pps{pps}")
    got2, _ = ctx.decode(q, pps=pps, heads=4)
    assert np.array_equal(got, got2)
    one, _ = ctx.decode(q, pps=pps, heads=1)
    assert_attn_close(got, one, f"4 heads against 1, pps{pps}")
    ctx.close()


@pytest.mark.parametrize("S,Hq,Hkv,causal,N", [(2, 32, 8, True, 3000), (4, 32, 8, True, 1000), (8, 16, 8, True, 777),
                                               (2, 32, 8, False, 1000), (1, 16, 4, True, 2049), (16, 4, 4, True, 300)])
def test_decode_four_heads_rows(orc, S, Hq, Hkv, causal, N):
    """4 kv heads per split workgroup with several query rows per kv head (up
    to 16: 64 (head, row) pairs merged by the workgroup's 8 waves), causal and
    not, against the oracle."""
    ctx = Context(orc, Hkv, 128, (N + 15) // 16 + 3, N, 700 + S + N, nan_tail=True)
    q = synth.normal_bf16(701 + S, (Hq, S, 128))
    got, _ = ctx.decode(q, causal=causal, heads=4)
    assert_attn_close(got, ctx.oracle(q, causal), f"4 heads S{S} Hq{Hq} Hkv{Hkv} causal{causal}")
    ctx.close()


def test_decode_four_heads_fall_back(orc):
    """Shapes the 4-head form does not serve (2 kv heads; head_dim 256; the
    single-launch merge) run the 1-head form when 4 are asked for."""
    for Hkv, D, merge in ((2, 128, "kernel"), (8, 256, "kernel"), (8, 128, "fused")):
        ctx = Context(orc, Hkv, D, 80, 1200, 910 + Hkv + D, nan_tail=True)
        q = synth.normal_bf16(911 + D, (4 * Hkv, 1, D))
        got, _ = ctx.decode(q, merge=merge, heads=4)
        assert_attn_close(got, ctx.oracle(q), f"fall back Hkv{Hkv} D{D} {merge}")
        ctx.close()


@pytest.mark.parametrize("S,Hq,causal", [(2, 32, True), (4, 32, True), (3, 16, True), (8, 16, True),
                                         (2, 32, False)])
def test_decode_multi_query(orc, S, Hq, causal):
    """Short chunks (append_tokens with a few tokens): rows = (query, q head),
    query s at n_cached - S + s; causal masks keys after it."""
    N = 61
    ctx = Context(orc, 8, 128, 8, N, 300 + S, nan_tail=True)
    q = synth.normal_bf16(301 + S, (Hq, S, 128))
    got, _ = ctx.decode(q, causal=causal)
    assert_attn_close(got, ctx.oracle(q, causal), f"S{S} Hq{Hq} causal{causal}")
    ctx.close()


def test_decode_repeat_is_deterministic(orc):
    ctx = Context(orc, 8, 128, 64, 900, 5)
    q = synth.normal_bf16(6, (32, 1, 128))
    a, _ = ctx.decode(q)
    b, _ = ctx.decode(q)
    assert np.array_equal(a, b)
    ctx.close()


@pytest.mark.parametrize("N,pps", [(1024, 1), (1025, 1), (2049, 1), (2049, 2), (4097, 1)])
def test_decode_merge_workgroup_sizes(orc, N, pps):
    """Split counts on both sides of the merge's 4-wave / 8-wave switch (64
    splits): 64, 65, 129, 65 and 129 (257 pages exceed the 256-split cap, so
    the plan raises pps to 2)."""
    ctx = Context(orc, 8, 128, (N + 15) // 16 + 3, N, 500 + N, nan_tail=True)
    q = synth.normal_bf16(600 + N, (32, 1, 128))
    got, _ = ctx.decode(q, pps=pps)
    assert_attn_close(got, ctx.oracle(q), f"N{N} pps{pps}")
    ctx.close()


@pytest.mark.parametrize("N,pps", [(1, None), (17, None), (300, None), (4099, None), (1000, 3)])
def test_decode_qwen35_head_dim_256(orc, N, pps):
    """Qwen3.5 attention layer shape (Qwen35.hpp:14-16): 8 q heads, 2 kv heads,
    head_dim 256 (GQA 4:1)."""
    pool = max(8, (N + 15) // 16 + 3)
    ctx = Context(orc, 2, 256, pool, N, 3000 + N, nan_tail=True)
    q = synth.normal_bf16(3100 + N, (8, 1, 256))
    got, _ = ctx.decode(q, pps=pps)
    assert_attn_close(got, ctx.oracle(q), f"D256 N{N} pps{pps}")
    ctx.close()


@pytest.mark.parametrize("S,causal", [(2, True), (4, True), (3, False)])
def test_decode_multi_query_head_dim_256(orc, S, causal):
    N = 190
    ctx = Context(orc, 2, 256, 16, N, 3300 + S, nan_tail=True)
    q = synth.normal_bf16(3400 + S, (8, S, 256))
    got, _ = ctx.decode(q, causal=causal)
    assert_attn_close(got, ctx.oracle(q, causal), f"D256 S{S} causal{causal}")
    ctx.close()


@pytest.mark.parametrize("Hq,Hkv,D,N,S,pps", [(32, 8, 128, 8193, 1, None), (32, 8, 128, 4100, 1, 64),
                                            (16, 8, 128, 1000, 8, 3), (8, 2, 256, 4099, 1, None)])
def test_decode_single_launch_merge(orc, Hq, Hkv, D, N, S, pps):
    """GENLLM_DECODE_MERGE=fused: the last split workgroup of each kv head
    merges the head's splits in the same launch (arrival counters in the
    workspace).  Against the oracle, with the counters back at zero after the
    launch (what makes a workspace reusable), and the default two-kernel merge
    on the same inputs."""
    pool = (N + 15) // 16 + 3
    ctx = Context(orc, Hkv, D, pool, N, 7000 + N + S, nan_tail=True)
    q = synth.normal_bf16(7100 + N, (Hq, S, D))
    ref = ctx.oracle(q)
    got, ws = ctx.decode(q, pps=pps, merge="fused")
    assert_attn_close(got, ref, f"fused merge Hq{Hq} Hkv{Hkv} D{D} N{N} S{S}")
    assert not ws[:1024].any().item(), "arrival counters not back at zero"
    two, _ = ctx.decode(q, pps=pps)
    assert_attn_close(two, ref, "two-kernel merge")
    ctx.close()


@pytest.mark.parametrize("Hq,Hkv,D,N,S,pps", [(32, 8, 128, 8193, 1, None), (32, 8, 128, 32761, 1, None),
                                            (16, 8, 128, 1000, 8, 3), (8, 2, 256, 8193, 1, None),
                                            (32, 8, 128, 4100, 1, 64)])
def test_decode_merge_forms_agree(orc, Hq, Hkv, D, N, S, pps):
    """The merge kernel (default) and the single-launch merge give the same
    bits on the same inputs, match the oracle, and leave the arrival counters
    at zero -- also over several launches in a row on one workspace."""
    pool = (N + 15) // 16 + 3
    ctx = Context(orc, Hkv, D, pool, N, 7300 + N + S, nan_tail=True)
    q = synth.normal_bf16(7400 + N, (Hq, S, D))
    ref = ctx.oracle(q)
    outs = {}
    for merge in ("kernel", "fused", "kernel", "fused"):
        got, ws = ctx.decode(q, pps=pps, merge=merge)
        assert_attn_close(got, ref, f"{merge} merge Hq{Hq} Hkv{Hkv} D{D} N{N} S{S}")
        assert not ws[:1024].any().item(), f"{merge}: arrival counters not back at zero"
        if merge in outs:
            assert np.array_equal(outs[merge], got), f"{merge}: repeat differs"
        outs[merge] = got
    ctx.close()


@pytest.mark.parametrize("Hq,Hkv,D,N,pps", [(32, 8, 128, 8193, 513), (32, 8, 128, 8193, 300),
                                          (16, 8, 128, 20000, 1250), (8, 2, 256, 8193, 300)])
def test_decode_splits_spanning_several_id_blocks(orc, Hq, Hkv, D, N, pps):
    """Splits longer than 64 pages per wave: a wave moves through blocks of 64
    page ids (the next block requested as it enters the current one), so a
    split may span any number of pages -- one split of all 513 pages, two of
    300, one of 1250 (5 id blocks per wave) and the head_dim 256 form (two
    pages in flight), against the oracle."""
    pool = (N + 15) // 16 + 5
    ctx = Context(orc, Hkv, D, pool, N, 7600 + N + pps, nan_tail=True)
    q = synth.normal_bf16(7700 + N, (Hq, 1, D))
    got, _ = ctx.decode(q, pps=pps)
    assert_attn_close(got, ctx.oracle(q), f"{pps} pages per split, Hq{Hq} Hkv{Hkv} D{D} N{N}")
    ctx.close()
