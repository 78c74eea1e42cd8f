"""GPU parity of the causal paged prefill kernel (genllm_paged_prefill, bf16
MFMA) against the oracle at sizes it finishes in seconds, and at BASELINE
config 4's full size against a float32 torch reference of the same attention
(K/V gathered through the block table) plus the oracle on a subset of heads.
Tolerance as for decode: max-abs <= 2^-7 max|ref|, rel-L2 <= 1e-2."""
import numpy as np
import pytest
import torch

from genllm_amd import paged, synth
from helpers import assert_attn_close, scale_for
from test_gpu_decode import Context

pytestmark = pytest.mark.gpu


def run_prefill(ctx, q_bits, causal=True, q_layout="head"):
    info = ctx.info
    if q_layout == "head":
        Hq, S, D = q_bits.shape
        out = torch.zeros((Hq, S, D), dtype=torch.bfloat16, device="cuda")
    else:
        S, Hq, D = q_bits.shape
        out = torch.zeros((S, Hq, D), dtype=torch.bfloat16, device="cuda")
    n_pages = (ctx.n_ctx + 15) // 16
    paged.paged_prefill(paged.to_device_bf16(q_bits), out, info.k_pool, info.v_pool, info.k_ids, info.v_ids, n_pages,
                        ctx.n_ctx, ctx.Hkv, scale_for(D), causal=causal, q_layout=q_layout)
    torch.cuda.synchronize()
    return paged.to_host_bits(out)


@pytest.mark.parametrize("Hq,Hkv,S,N,causal", [
    (16, 8, 64, 64, True),
    (16, 8, 128, 128, True),
    (16, 8, 300, 300, True),      # ragged query tile and page
    (32, 8, 200, 333, True),      # chunked prefill: 133 tokens already cached
    (8, 8, 129, 129, True),
    (4, 2, 257, 257, False),
])
def test_prefill_vs_oracle(orc, Hq, Hkv, S, N, causal):
    pool = (N + 15) // 16 + 5
    ctx = Context(orc, Hkv, 128, pool, N, 4000 + S + N, nan_tail=True)
    q = synth.normal_bf16(4100 + S, (Hq, S, 128))
    got = run_prefill(ctx, q, causal)
    assert_attn_close(got, ctx.oracle(q, causal), f"prefill Hq{Hq} Hkv{Hkv} S{S} N{N} causal{causal}")
    ctx.close()


@pytest.mark.parametrize("Hq,Hkv,D,S,N,causal", [
    (8, 4, 128, 128, 5000, True),    # 79 key tiles: the page ids are reloaded past tile 64
    (4, 2, 128, 70, 4500, False),
    (8, 2, 256, 64, 4200, True),     # the D = 256 kernel over 132 key tiles
])
def test_prefill_long_context_vs_oracle(orc, Hq, Hkv, D, S, N, causal):
    """A chunk of S queries after N - S cached tokens, past the first block of
    page ids the kernel fetches at once."""
    pool = (N + 15) // 16 + 7
    ctx = Context(orc, Hkv, D, pool, N, 6000 + S + N + D, nan_tail=True)
    q = synth.normal_bf16(6100 + S + D, (Hq, S, D))
    got = run_prefill(ctx, q, causal)
    assert_attn_close(got, ctx.oracle(q, causal), f"long prefill Hq{Hq} D{D} S{S} N{N} causal{causal}")
    ctx.close()


def torch_reference(ctx, q_bits, heads, causal=True):
    """float32 attention on the GPU for the given q heads; K/V gathered from
    the pools through the page table."""
    Hq, S, D = q_bits.shape
    G = Hq // ctx.Hkv
    N = ctx.n_ctx
    kt, vt = ctx.mgr.page_table(0)
    kp = torch.from_numpy(ctx.mgr.read_pool(0, 0).view(np.int16)).view(torch.bfloat16).cuda()
    vp = torch.from_numpy(ctx.mgr.read_pool(0, 1).view(np.int16)).view(torch.bfloat16).cuda()
    K = kp[torch.from_numpy(kt).long().cuda()].reshape(-1, ctx.Hkv, D)[:N].float()  # [N][Hkv][D]
    V = vp[torch.from_numpy(vt).long().cuda()].reshape(-1, ctx.Hkv, D)[:N].float()
    q = paged.to_device_bf16(q_bits).float()
    qpos = torch.arange(N - S, N, device="cuda")[:, None]
    kpos = torch.arange(N, device="cuda")[None, :]
    out = {}
    for h in heads:
        sc = (q[h] @ K[:, h // G, :].T.contiguous()) * scale_for(D)
        if causal:
            sc = sc.masked_fill(kpos > qpos, float("-inf"))
        p = torch.softmax(sc, dim=-1)
        out[h] = (p @ V[:, h // G, :].contiguous()).cpu().numpy()
    return out


def test_prefill_config4(orc):
    """Qwen3-1.7B causal paged prefill, 2048-token prompt,
    Q [2048,16,128] token-major, K/V in 128 pages of a random table."""
    seed = synth.config_seed(4)
    Hq, Hkv, S, D = 16, 8, 2048, 128
    ctx = Context(orc, Hkv, D, 128, S, seed)
    q = synth.normal_bf16(seed, (S, Hq, D), offset=9 << 28)
    got = run_prefill(ctx, q, True, q_layout="token")  # [S][Hq][D]
    q_head = np.ascontiguousarray(q.transpose(1, 0, 2))
    ref = torch_reference(ctx, q_head, range(Hq))
    got_h = np.ascontiguousarray(got.transpose(1, 0, 2))
    want = np.stack([ref[h] for h in range(Hq)])
    want_bits = synth.f32_to_bf16_bits(want.astype(np.float32))
    assert_attn_close(got_h, want_bits, "config4 vs torch fp32")
    # the oracle on q heads 0 and 1 (they share kv head 0: kv_h = h / groups)
    G = Hq // Hkv
    o, rc = ctx.ref.paged_attend(0, np.ascontiguousarray(q_head[:G])[None], Hkv, G, scale_for(D), True)
    assert rc == 0
    assert_attn_close(got_h[:G], o[0], "config4 heads 0-1 vs oracle")
    ctx.close()


@pytest.mark.parametrize("S,N,causal", [
    (64, 64, True),
    (300, 300, True),     # ragged query tile and page
    (200, 333, True),     # chunked prefill: 133 tokens already cached
    (129, 129, False),
    (17, 40, True),
])
def test_prefill_head_dim_256_vs_oracle(orc, S, N, causal):
    """Qwen3.5 attention layer (Qwen35.cpp:191-226): head_dim 256, 8 q heads
    over 2 kv heads, the D = 256 prefill kernel."""
    Hq, Hkv, D = 8, 2, 256
    pool = (N + 15) // 16 + 5
    ctx = Context(orc, Hkv, D, pool, N, 5000 + S + N, nan_tail=True)
    q = synth.normal_bf16(5100 + S, (Hq, S, D))
    got = run_prefill(ctx, q, causal)
    assert_attn_close(got, ctx.oracle(q, causal), f"prefill D256 S{S} N{N} causal{causal}")
    ctx.close()


def test_prefill_head_dim_256_long_vs_torch(orc):
    """2048-token Qwen3.5-shape causal prefill against float32 torch (all heads)."""
    Hq, Hkv, S, D = 8, 2, 2048, 256
    ctx = Context(orc, Hkv, D, 128, S, 5500)
    q = synth.normal_bf16(5501, (Hq, S, D))
    got = run_prefill(ctx, q, True)
    ref = torch_reference(ctx, q, range(Hq))
    want = synth.f32_to_bf16_bits(np.stack([ref[h] for h in range(Hq)]).astype(np.float32))
    assert_attn_close(got, want, "prefill D256 2048 vs torch fp32")
    ctx.close()
