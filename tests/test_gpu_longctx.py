"""BASELINE config 5 at its full size: Qwen3-4B-shape long-context decode across
all 36 layers back to back (32 q heads, 8 kv heads, head_dim 128; per layer
32,761 cached keys = 2047 full pages + 9 tokens, 2048 pages drawn from a
seeded shuffle of a per-layer 4096-page pool; bf16 K/V ~ N(0,1), ~4.8 GB of
KV in total).  This is the attention loop of PagedAttentionImpl<CPU>
(src/backend/cpu/attention.cpp:148-215) as the executor's decode step drives
it layer after layer (src/core/executor.cpp:94-174, 227-236).

Checks, on exactly the workload bench.py times:
  * every layer against an fp32 torch reference on the GPU (page gather by the
    block table, softmax(q K^T * scale) V in fp32);
  * layers 0 and 35, all 32 heads, against the oracle restatement on the host;
  * the 36-layer sequence captured into one HIP graph and replayed twice, with
    eager work between the replays: every replay equals the eager run bit for
    bit.
Tolerance (bf16 output, fp32 accumulate): max-abs <= 2^-7 max|ref| and rel-L2
<= 1e-2 (helpers.assert_attn_close)."""
import numpy as np
import pytest
import torch

from genllm_amd import paged, synth
from genllm_amd._lib import call
from helpers import assert_attn_close, oracle_fragmented

pytestmark = pytest.mark.gpu

Hq, Hkv, D, L = 32, 8, 128, 36
N, POOL = 32761, 4096
G = Hq // Hkv
SCALE = 1.0 / np.sqrt(D)


def fp32_reference(pool_k, pool_v, k_ids, v_ids, q):
    """softmax(q K^T * scale) V in fp32 over the first N tokens of the pages
    k_ids / v_ids (torch on the GPU).  q [Hq][D] bf16 -> out [Hq][D] fp32."""
    n_pages = (N + 15) // 16
    kk = pool_k.index_select(0, k_ids[:n_pages].long()).reshape(n_pages * 16, Hkv, D)[:N].float()
    vv = pool_v.index_select(0, v_ids[:n_pages].long()).reshape(n_pages * 16, Hkv, D)[:N].float()
    out = torch.empty((Hq, D), dtype=torch.float32, device="cuda")
    qf = q.float()
    for h in range(Hkv):
        kh = kk[:, h, :].contiguous()                     # [N][D]
        vh = vv[:, h, :].contiguous()
        s = torch.matmul(qf[h * G:(h + 1) * G], kh.t().contiguous()) * SCALE  # [G][N]
        p = torch.softmax(s, dim=-1)
        out[h * G:(h + 1) * G] = torch.matmul(p, vh)
    return out


def test_longctx_config5_full_size(orc):
    seed = synth.config_seed(5)
    print(f"config5: {L} layers x {N} keys, pool {POOL} pages per layer, seed {seed:#x}", flush=True)
    mgr = paged.PagedAttentionManager(L * 2 * POOL * 16 * Hkv * D * 2)
    perms = []
    for l in range(L):
        perm_k, perm_v = synth.shuffled(seed + 2 * l, POOL), synth.shuffled(seed + 2 * l + 1, POOL)
        perms.append((perm_k, perm_v))
        mgr.init_layer(l, Hkv, D)
        mgr.reserve_layer(l, POOL)
        mgr.fragment(l, perm_k, perm_v)
        mgr.append_kv_pages(l, N)
        inf = mgr.get_layer(l)
        call("genllm_fill_normal_bf16", inf.k_pool, POOL * 16 * Hkv * D, seed + 100 + l, 0, None)
        call("genllm_fill_normal_bf16", inf.v_pool, POOL * 16 * Hkv * D, seed + 200 + l, 0, None)
    infos = [mgr.get_layer(l) for l in range(L)]
    assert all(i.num_pages == 2048 and i.num_cached == N for i in infos)
    q = torch.empty((L, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    paged.fill_normal_bf16(q, seed)
    ws = torch.zeros(paged.decode_workspace_bytes(Hq, Hkv, 1, D, POOL), dtype=torch.uint8, device="cuda")
    n_pages = (N + 15) // 16

    def all_layers(out):
        for l in range(L):
            inf = infos[l]
            paged.paged_decode(q[l], out[l], inf.k_pool, inf.v_pool, inf.k_ids, inf.v_ids, n_pages, N, Hkv,
                               SCALE, ws)

    eager = torch.zeros((L, Hq, 1, D), dtype=torch.bfloat16, device="cuda")
    all_layers(eager)
    torch.cuda.synchronize()
    print("config5: eager run done", flush=True)

    # every layer against the fp32 reference on the GPU
    for l in range(L):
        kt = mgr.device_table(l, 0)
        vt = mgr.device_table(l, 1)
        ref = fp32_reference(mgr.pool(l, 0), mgr.pool(l, 1), kt, vt, q[l, :, 0, :])
        assert_attn_close(paged.to_host_bits(eager[l, :, 0, :]), paged.to_host_bits(ref.to(torch.bfloat16)),
                          f"config5 layer {l} vs fp32 torch")

    # layers 0 and 35, every head, against the oracle on identical pools and tables
    for l in (0, L - 1):
        perm_k, perm_v = perms[l]
        ref = oracle_fragmented(orc, Hkv, D, POOL, perm_k, perm_v)
        ref.append_kv_pages(0, N)
        rk, rv = ref.page_table(0)
        kt, vt = mgr.page_table(l)
        assert np.array_equal(kt, rk) and np.array_equal(vt, rv)
        dk, dv = mgr.read_device_table(l)
        assert np.array_equal(dk, rk) and np.array_equal(dv, rv)
        ref.pool_array(0, 0)[:] = mgr.read_pool(l, 0)
        ref.pool_array(0, 1)[:] = mgr.read_pool(l, 1)
        qb = paged.to_host_bits(q[l])                      # [Hq][1][D]
        want, rc = ref.paged_attend(0, qb[None], Hkv, G, SCALE, True)
        assert rc == 0
        assert_attn_close(paged.to_host_bits(eager[l]), want[0], f"config5 layer {l} vs oracle")

    # the 36-layer sequence as one HIP graph: replays equal the eager run bit for bit
    want_bits = eager.view(torch.int16).cpu().numpy()
    out = torch.zeros_like(eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        all_layers(out)
    other = torch.zeros_like(eager)
    for rep in range(2):
        out.fill_(0)
        all_layers(other)  # eager work on the same stream between replays
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.view(torch.int16).cpu().numpy(), want_bits), f"graph replay {rep} differs"
        assert np.array_equal(other.view(torch.int16).cpu().numpy(), want_bits)
    del g
    mgr.close()
