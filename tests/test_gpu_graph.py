"""HIP-graph capture of a 36-layer decode-attention sequence (the shape of
Qwen3-4B, 32 q heads, 8 kv heads, head_dim 128, one query
per layer over a fixed cached context), the executor pattern of
src/core/executor.cpp:94-174 without its per-op synchronisation.

A decode launch is a plan computed on the host plus two kernel launches with
arguments only (no allocation, no memset, no copy), so the captured graph must
reproduce the eager results bit for bit on every replay -- with eager work on
the same stream between replays, and after the pools' contents change (the
graph holds pointers, not data)."""
import numpy as np
import pytest
import torch

from genllm_amd import paged, synth
from genllm_amd._lib import call

pytestmark = pytest.mark.gpu

Hq, Hkv, D, L = 32, 8, 128, 36
SCALE = 1.0 / np.sqrt(D)


class Layers:
    def __init__(self, n_cached, pool, seed):
        self.N, self.pool = n_cached, pool
        self.mgr = paged.PagedAttentionManager(L * (2 * pool * 16 * Hkv * D * 2 + 8 * pool + 8192) + (1 << 20))
        for l in range(L):
            self.mgr.init_layer(l, Hkv, D)
            self.mgr.reserve_layer(l, pool)
            self.mgr.fragment(l, synth.shuffled(seed + 2 * l, pool), synth.shuffled(seed + 2 * l + 1, pool))
            self.mgr.append_kv_pages(l, n_cached)
        self.infos = [self.mgr.get_layer(l) for l in range(L)]
        self.fill(seed)
        self.q = torch.empty((L, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
        paged.fill_normal_bf16(self.q, seed + 7)
        self.ws = torch.zeros(paged.decode_workspace_bytes(Hq, Hkv, 1, D, pool), dtype=torch.uint8, device="cuda")

    def fill(self, seed):
        for l, inf in enumerate(self.infos):
            n = self.pool * 16 * Hkv * D
            call("genllm_fill_normal_bf16", inf.k_pool, n, seed + 100 + l, 0, None)
            call("genllm_fill_normal_bf16", inf.v_pool, n, seed + 200 + l, 0, None)

    def decode_all(self, out):
        n_pages = (self.N + 15) // 16
        for l, inf in enumerate(self.infos):
            paged.paged_decode(self.q[l], out[l], inf.k_pool, inf.v_pool, inf.k_ids, inf.v_ids, n_pages, self.N,
                               Hkv, SCALE, self.ws)

    def close(self):
        self.mgr.close()


def bits(t):
    return t.view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("n_cached", [1000, 4099])
def test_graph_replays_match_eager(n_cached):
    pool = (n_cached + 15) // 16 + 3
    ly = Layers(n_cached, pool, 9100 + n_cached)
    eager = torch.empty((L, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    ly.decode_all(eager)  # also the warm-up before capture
    torch.cuda.synchronize()
    want = bits(eager)

    out = torch.zeros_like(eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ly.decode_all(out)
    other = torch.empty_like(eager)
    for rep in range(3):
        out.fill_(0)
        ly.decode_all(other)  # eager work on the stream between replays
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), want), f"replay {rep} differs from the eager run"
        assert np.array_equal(bits(other), want)

    # new pool contents: the replay reads them (pointers were captured, not data)
    ly.fill(7777)
    ly.decode_all(eager)
    torch.cuda.synchronize()
    want2 = bits(eager)
    assert not np.array_equal(want2, want)
    for rep in range(2):
        out.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), want2), f"replay {rep} after the pool change differs"
    ly.close()
