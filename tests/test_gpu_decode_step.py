"""Device-position decode steps, captured once into a HIP graph and replayed
for successive tokens: the decode loop of src/core/executor.cpp:227-236 over
the layer forward (:94-174), with the position and the next pages on the
device.  Per layer and step: RoPE of q and k at the device position
(ApplyRopeImpl, rope.cpp:76-119), then append + attend
(PagedAttentionImpl::execute, attention.cpp:123-216).  After every replay the
outputs, the RoPE'd q, both pools and the device page table are checked against
the oracle run step by step with host positions; after genllm_kv_sync_decode
the host tables, num_cached and the block pools must equal the oracle's, so
that the device-driven steps are indistinguishable from per-step appends."""
import numpy as np
import pytest
import torch

from genllm_amd import paged, synth
from genllm_amd._lib import ERR_INVALID, ERR_POOL_FULL, GenllmError
from helpers import assert_attn_close, oracle_fragmented, scale_for

pytestmark = pytest.mark.gpu

THETA = 1.0e6


class Stack:
    """L layers of the product manager and the oracle, same fragmented pools,
    each filled with a P-token prompt through the host-position op."""

    def __init__(self, orc, L, Hq, Hkv, D, pool, P, seed, prompt=True):
        self.L, self.Hq, self.Hkv, self.D, self.G = L, Hq, Hkv, D, Hq // Hkv
        self.orc = orc
        self.mgr = paged.PagedAttentionManager(L * (2 * pool * 16 * Hkv * D * 2 + 4096) + (1 << 20))
        self.ref = orc.Manager(with_pool=True)
        for l in range(L):
            perm_k, perm_v = synth.shuffled(seed + 2 * l, pool), synth.shuffled(seed + 2 * l + 1, pool)
            self.mgr.init_layer(l, Hkv, D)
            self.mgr.reserve_layer(l, pool)
            self.mgr.fragment(l, perm_k, perm_v)
            oracle_fragmented(orc, Hkv, D, pool, perm_k, perm_v, layer=l, m=self.ref)
        print(f"prefill {L} layers x {P} tokens", flush=True)
        for l in range(L):
            if not prompt:  # long context: P cached tokens of random K/V, no prefill attention
                self.mgr.append_kv_pages(l, P)
                self.ref.append_kv_pages(l, P)
                for which in (0, 1):
                    data = synth.normal_bf16(seed + 400 + 2 * l + which, (pool, 16, Hkv, D))
                    self.ref.pool_array(l, which)[:] = data
                    self.mgr.write_pool(l, which, data)
                continue
            q = synth.normal_bf16(seed + 100 + l, (1, Hq, P, D))
            k = synth.normal_bf16(seed + 200 + l, (1, Hkv, P, D))
            v = synth.normal_bf16(seed + 300 + l, (1, Hkv, P, D))
            out = torch.empty((1, Hq, P, D), dtype=torch.bfloat16, device="cuda")
            paged.paged_attention(self.mgr, l, paged.to_device_bf16(q), paged.to_device_bf16(k),
                                  paged.to_device_bf16(v), out, self.G, scale_for(D))
            _, rc = self.ref.paged_attention(l, q, k, v, self.G, scale_for(D))
            assert rc == 0
        torch.cuda.synchronize()

    def check_pools(self, label):
        for l in range(self.L):
            for which in (0, 1):
                assert np.array_equal(self.mgr.read_pool(l, which), self.ref.pool_array(l, which)), \
                    f"{label}: layer {l} {'KV'[which]} pool differs from the oracle"

    def check_device_table_prefix(self, label):
        for l in range(self.L):
            rk, rv = self.ref.page_table(l)
            dk, dv = self.mgr.read_device_table(l)
            assert np.array_equal(dk[:rk.size], rk) and np.array_equal(dv[:rv.size], rv), \
                f"{label}: layer {l} device table differs from the oracle's pages"

    def check_host_state(self, label):
        for l in range(self.L):
            info = self.mgr.get_layer(l)
            assert info.num_cached == self.ref.num_cached(l), f"{label}: layer {l} num_cached"
            kt, vt = self.mgr.page_table(l)
            rk, rv = self.ref.page_table(l)
            assert np.array_equal(kt, rk) and np.array_equal(vt, rv), f"{label}: layer {l} page table"
            for which, (nb, nf) in ((0, (info.k_num_blocks, info.k_num_free)),
                                    (1, (info.v_num_blocks, info.v_num_free))):
                p = self.ref.pool(l, which)
                assert (nb, nf) == (p.num_blocks(), p.num_free()), f"{label}: layer {l} block pool {which}"

    def close(self):
        self.mgr.close()


class StepBuffers:
    """Fixed device buffers of one decode token per layer (a captured graph
    holds their addresses; each step writes new contents into them)."""

    def __init__(self, st, max_seq):
        L, Hq, Hkv, D = st.L, st.Hq, st.Hkv, st.D
        dev = dict(dtype=torch.bfloat16, device="cuda")
        self.q_raw = torch.zeros((L, Hq, 1, D), **dev)
        self.k_raw = torch.zeros((L, Hkv, 1, D), **dev)
        self.v = torch.zeros((L, 1, Hkv, 1, D), **dev)
        self.q_rot = torch.zeros((L, 1, Hq, 1, D), **dev)
        self.k_rot = torch.zeros((L, 1, Hkv, 1, D), **dev)
        self.out = torch.zeros((L, 1, Hq, 1, D), **dev)
        self.cos, self.sin = st.orc.rope_cache(THETA, D, max_seq)
        self.cos_t = torch.from_numpy(self.cos).cuda()
        self.sin_t = torch.from_numpy(self.sin).cuda()

    def layer_step(self, st, l, rope=True):
        if rope:
            paged.apply_rope_step(st.mgr, l, self.q_rot[l, 0], self.q_raw[l], self.cos_t, self.sin_t)
            paged.apply_rope_step(st.mgr, l, self.k_rot[l, 0], self.k_raw[l], self.cos_t, self.sin_t)
        q = self.q_rot[l] if rope else self.q_raw[l].unsqueeze(0)
        k = self.k_rot[l] if rope else self.k_raw[l].unsqueeze(0)
        paged.paged_attention_step(st.mgr, l, q, k, self.v[l], self.out[l], st.G, scale_for(st.D))

    def load(self, st, seed):
        """New token: host copies (bf16 bits) and their upload."""
        q = synth.normal_bf16(seed, (st.L, st.Hq, 1, st.D))
        k = synth.normal_bf16(seed + 1, (st.L, st.Hkv, 1, st.D))
        v = synth.normal_bf16(seed + 2, (st.L, 1, st.Hkv, 1, st.D))
        self.q_raw.copy_(paged.to_device_bf16(q))
        self.k_raw.copy_(paged.to_device_bf16(k))
        self.v.copy_(paged.to_device_bf16(v))
        return q, k, v


def bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def run_checked_replays(st, buf, g, n, pos0, seed, rope=True, layers=None):
    """n replays of graph g, each checked against the oracle at host position pos0 + i."""
    layers = range(st.L) if layers is None else layers
    for i in range(n):
        pos = pos0 + i
        print(f"replay {i}: position {pos}", flush=True)
        q, k, v = buf.load(st, seed + 10 * i)
        buf.out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        got = bits(buf.out)
        q_rot = bits(buf.q_rot)
        for l in layers:
            if rope:
                qr = st.orc.apply_rope(q[l], buf.cos, buf.sin, pos)
                kr = st.orc.apply_rope(k[l], buf.cos, buf.sin, pos)
                assert np.array_equal(q_rot[l, 0], qr), f"replay {i} layer {l}: RoPE'd q differs from the oracle"
            else:
                qr, kr = q[l], k[l]
            want, rc = st.ref.paged_attention(l, qr[None], kr[None], v[l], st.G, scale_for(st.D))
            assert rc == 0
            assert_attn_close(got[l], want, f"replay {i} layer {l} pos {pos}")
        st.check_pools(f"replay {i}")
        st.check_device_table_prefix(f"replay {i}")


def test_captured_36_layer_step_replays_20_tokens(orc):
    """Qwen3-4B shape (32 q / 8 kv heads, head_dim 128), 36 layers, a 100-token
    prompt; one step (RoPE q, RoPE k, append + attend per layer) captured once
    and replayed for positions 100..119, opening page 7 at position 112."""
    L, Hq, Hkv, D, P, steps = 36, 32, 8, 128, 100, 20
    st = Stack(orc, L, Hq, Hkv, D, pool=12, P=P, seed=0x5EED0100)
    buf = StepBuffers(st, max_seq=256)
    for l in range(L):
        st.mgr.stage_decode(l, steps)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for l in range(L):
            buf.layer_step(st, l)
    run_checked_replays(st, buf, g, steps, P, seed=7000)
    for l in range(L):
        assert st.mgr.sync_decode(l) == P + steps
    st.check_host_state("after sync")
    # the host-position op continues from the synced state like the reference
    q = synth.normal_bf16(91, (1, Hq, 1, D))
    k = synth.normal_bf16(92, (1, Hkv, 1, D))
    v = synth.normal_bf16(93, (1, Hkv, 1, D))
    out = torch.empty((1, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    paged.paged_attention(st.mgr, 0, paged.to_device_bf16(q), paged.to_device_bf16(k), paged.to_device_bf16(v),
                          out, Hq // Hkv, scale_for(D))
    torch.cuda.synchronize()
    want, rc = st.ref.paged_attention(0, q, k, v, Hq // Hkv, scale_for(D))
    assert rc == 0
    assert_attn_close(paged.to_host_bits(out), want, "host step after sync")
    st.check_host_state("host step after sync")
    st.close()


def test_partial_window_sync_and_exhaustion(orc):
    """A window staged for 40 tokens of which 5 run: sync gives the 3 unused
    pages back so that later host appends hand out the reference's ids; a
    window of 3 replayed 4 times: the 4th step does nothing and sync reports
    it; host-driven calls are refused while staged."""
    L, Hq, Hkv, D, P = 2, 16, 8, 128, 30
    st = Stack(orc, L, Hq, Hkv, D, pool=10, P=P, seed=0x5EED0200)
    buf = StepBuffers(st, max_seq=128)
    for l in range(L):
        st.mgr.stage_decode(l, 40)  # opens pages 2, 3, 4 (positions 32, 48, 64)
    assert st.mgr.get_layer(0).num_pages == 5
    with pytest.raises(GenllmError) as e:  # host-driven op on a staged layer
        paged.paged_attention(st.mgr, 0, buf.q_raw[0].unsqueeze(0), buf.k_raw[0].unsqueeze(0), buf.v[0],
                              buf.out[0], Hq // Hkv, scale_for(D))
    assert e.value.code == ERR_INVALID
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for l in range(L):
            buf.layer_step(st, l, rope=False)
    run_checked_replays(st, buf, g, 5, P, seed=8000, rope=False)
    for l in range(L):
        assert st.mgr.sync_decode(l) == P + 5
    st.check_host_state("window of 40, 5 used")
    # host appends after the sync allocate what the reference allocates
    for l in range(L):
        st.mgr.append_kv_pages(l, 20)
        st.ref.append_kv_pages(l, 20)
    st.check_host_state("host appends after sync")

    pos = P + 25
    for l in range(L):
        st.mgr.stage_decode(l, 3)
    run_checked_replays(st, buf, g, 3, pos, seed=9000, rope=False)
    # the 4th step passes the window: nothing is written, the position stays
    buf.out.fill_(1.0)
    buf.load(st, 9999)
    g.replay()
    torch.cuda.synchronize()
    assert torch.all(buf.out == 1.0).item(), "a refused step wrote its output"
    st.check_pools("refused step")
    for l in range(L):
        with pytest.raises(GenllmError) as e:
            st.mgr.sync_decode(l)
        assert e.value.code == ERR_POOL_FULL
        assert st.mgr.get_layer(l).num_cached == pos + 3
    st.check_host_state("after the refused step")
    st.close()


def test_step_head_dim_256_across_8192(orc):
    """Qwen3.5 shape (8 q / 2 kv heads, head_dim 256): the split-K plan at 8K
    keys with the device position, replayed across the page boundary at 8192."""
    L, Hq, Hkv, D, P = 1, 8, 2, 256, 8185
    st = Stack(orc, L, Hq, Hkv, D, pool=520, P=P, seed=0x5EED0300, prompt=False)
    buf = StepBuffers(st, max_seq=8256)
    st.mgr.stage_decode(0, 16)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        buf.layer_step(st, 0)
    run_checked_replays(st, buf, g, 12, P, seed=9500)
    assert st.mgr.sync_decode(0) == P + 12
    st.check_host_state("after sync")
    st.close()


@pytest.mark.parametrize("Hq,Hkv,D,S,P,rope_dim,merge", [
    (16, 8, 128, 2, 40, 128, None),     # two tokens per step (append_tokens), pages opened at 48 and 64
    (32, 8, 128, 1, 5, 128, None),      # one split: the last split workgroup advances the position
    (32, 8, 128, 1, 200, 128, "fused"),  # single-launch merge: no merge kernel either
    (8, 2, 256, 1, 90, 64, None),       # Qwen3.5: RoPE on the first 64 of 256 dims
    (16, 8, 128, 2, 40, 128, "heads4"),  # split workgroups reading 4 kv heads each, steps crossing pages
])
def test_step_variants(orc, request, Hq, Hkv, D, S, P, rope_dim, merge):
    """Device-position steps beyond the single-token default plan: the query
    chunk, the split plan, the merge form and the rotary width change, and
    every replay still matches the oracle run with host positions (RoPE'd q
    bit-exact, attention within tolerance, pools bit-exact)."""
    if merge == "heads4":
        paged.decode_tuning(0, "kernel", 4)
        request.addfinalizer(lambda: paged.decode_tuning(0, "kernel"))
    elif merge:
        paged.decode_tuning(0, merge)
        request.addfinalizer(lambda: paged.decode_tuning(0, "kernel"))
    G, L, steps, max_seq = Hq // Hkv, 2, 8, 512
    pool = (P + S * steps + 15) // 16 + 2
    st = Stack(orc, L, Hq, Hkv, D, pool=pool, P=P, seed=0x5EED0400 + S + D + P)
    dev = dict(dtype=torch.bfloat16, device="cuda")
    q_raw = torch.zeros((L, Hq, S, D), **dev)
    k_raw = torch.zeros((L, Hkv, S, D), **dev)
    v_in = torch.zeros((L, 1, Hkv, S, D), **dev)
    q_rot = torch.zeros((L, 1, Hq, S, D), **dev)
    k_rot = torch.zeros((L, 1, Hkv, S, D), **dev)
    out = torch.zeros((L, 1, Hq, S, D), **dev)
    cos, sin = orc.rope_cache(THETA, rope_dim, max_seq)
    cos_t, sin_t = torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda()
    rope = orc.apply_rope if rope_dim == D else orc.apply_rope_partial
    for l in range(L):
        st.mgr.stage_decode(l, S * steps)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for l in range(L):
            paged.apply_rope_step(st.mgr, l, q_rot[l, 0], q_raw[l], cos_t, sin_t)
            paged.apply_rope_step(st.mgr, l, k_rot[l, 0], k_raw[l], cos_t, sin_t)
            paged.paged_attention_step(st.mgr, l, q_rot[l], k_rot[l], v_in[l], out[l], G, scale_for(D))
    for i in range(steps):
        pos = P + S * i
        print(f"replay {i}: positions {pos}..{pos + S - 1}", flush=True)
        q = synth.normal_bf16(11000 + 10 * i, (L, Hq, S, D))
        k = synth.normal_bf16(11001 + 10 * i, (L, Hkv, S, D))
        v = synth.normal_bf16(11002 + 10 * i, (L, 1, Hkv, S, D))
        q_raw.copy_(paged.to_device_bf16(q))
        k_raw.copy_(paged.to_device_bf16(k))
        v_in.copy_(paged.to_device_bf16(v))
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        got, got_q = bits(out), bits(q_rot)
        for l in range(L):
            qr, kr = rope(q[l], cos, sin, pos), rope(k[l], cos, sin, pos)
            assert np.array_equal(got_q[l, 0], qr), f"replay {i} layer {l}: RoPE'd q"
            want, rc = st.ref.paged_attention(l, qr[None], kr[None], v[l], G, scale_for(D))
            assert rc == 0
            assert_attn_close(got[l], want, f"replay {i} layer {l} positions {pos}..")
        st.check_pools(f"replay {i}")
    for l in range(L):
        assert st.mgr.sync_decode(l) == P + S * steps
    st.check_host_state("after sync")
    st.close()
