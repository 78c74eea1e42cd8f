"""Non-paged attention (FlashAttentionImpl, src/backend/cpu/attention.cpp:39-121;
the op type of kv_cache_per_layer = 0) on the GPU, through
genllm_flash_attention, against the CPU oracle (small shapes) and a float32
torch reference (prefill size).  Tolerance: max-abs <= 2^-7 * max|ref|,
relative L2 <= 1e-2."""
from __future__ import annotations

import numpy as np
import pytest

from helpers import assert_attn_close

pytestmark = pytest.mark.gpu


def _inputs(synth, seed, B, Hq, Hkv, S, D=128):
    q = synth.normal_bf16(seed, (B, Hq, S, D))
    k = synth.normal_bf16(seed, (B, Hkv, S, D), offset=1 << 26)
    v = synth.normal_bf16(seed, (B, Hkv, S, D), offset=2 << 26)
    return q, k, v


@pytest.mark.parametrize("B,Hq,Hkv,S,causal", [
    (2, 8, 2, 77, True),     # GQA 4:1, ragged last page, two batch entries
    (1, 16, 8, 130, False),  # no mask: every query sees all 130 keys
    (1, 4, 4, 1, True),      # one token: out = v
    (1, 16, 8, 16, True),    # exactly one page
])
def test_flash_vs_oracle(orc, B, Hq, Hkv, S, causal):
    import torch

    from genllm_amd import paged, synth

    print(f"flash B{B} Hq{Hq} Hkv{Hkv} S{S} causal={causal}", flush=True)
    scale = 1.0 / np.sqrt(128)
    q, k, v = _inputs(synth, 900 + S, B, Hq, Hkv, S)
    out = torch.empty((B, Hq, S, 128), dtype=torch.bfloat16, device="cuda")
    paged.flash_attention(paged.to_device_bf16(q), paged.to_device_bf16(k), paged.to_device_bf16(v), out,
                          Hq // Hkv, scale, causal)
    torch.cuda.synchronize()
    want = orc.flash_attention(q, k, v, Hq // Hkv, scale, causal)
    got = paged.to_host_bits(out)
    assert_attn_close(got, want, f"flash S{S}")
    if S == 1:
        # a single key: softmax weight 1, the output is that key's V row, exactly
        assert np.array_equal(got[0, :, 0, :], v[0, np.arange(Hq) // (Hq // Hkv), 0, :])


def test_flash_prefill_size_vs_torch():
    """Qwen3-1.7B prefill shape (config 4 without paging): 2048 tokens, 16 q
    heads over 8 kv heads, causal; heads 0, 1 and 15 against float32 torch."""
    import torch

    from genllm_amd import paged, synth

    B, Hq, Hkv, S, D = 1, 16, 8, 2048, 128
    print("flash prefill 2048", flush=True)
    scale = 1.0 / np.sqrt(D)
    q = torch.empty((B, Hq, S, D), dtype=torch.bfloat16, device="cuda")
    k = torch.empty((B, Hkv, S, D), dtype=torch.bfloat16, device="cuda")
    v = torch.empty_like(k)
    for i, t in enumerate((q, k, v)):
        paged.fill_normal_bf16(t, synth.config_seed(4) + 70 + i)
    out = torch.empty_like(q)
    paged.flash_attention(q, k, v, out, Hq // Hkv, scale, True)
    torch.cuda.synchronize()
    qf, kf, vf = (t.float().cpu() for t in (q, k, v))
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool), 1)
    for h in (0, 1, 15):
        s = (qf[0, h] @ kf[0, h // 2].T) * scale
        s.masked_fill_(mask, float("-inf"))
        ref = torch.softmax(s, dim=-1) @ vf[0, h // 2]
        want = ref.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        assert_attn_close(paged.to_host_bits(out[0, h]), want, f"flash 2048 head {h}")


@pytest.mark.parametrize("Hq,Hkv,S,D", [(32, 8, 8192, 128), (8, 2, 8192, 256)])
def test_flash_long_vs_torch(Hq, Hkv, S, D):
    """The prefill kernel at 8192 tokens (the bench's prefill_scale shapes),
    causal: the first and last q heads against a float32 torch reference
    computed on the GPU (float32 products: no bf16 batched matmul)."""
    import torch

    from genllm_amd import paged

    print(f"flash long Hq{Hq} Hkv{Hkv} S{S} D{D}", flush=True)
    scale = 1.0 / np.sqrt(D)
    q = torch.empty((1, Hq, S, D), dtype=torch.bfloat16, device="cuda")
    k = torch.empty((1, Hkv, S, D), dtype=torch.bfloat16, device="cuda")
    v = torch.empty_like(k)
    for i, t in enumerate((q, k, v)):
        paged.fill_normal_bf16(t, 8800 + 10 * D + i)
    out = torch.empty_like(q)
    paged.flash_attention(q, k, v, out, Hq // Hkv, scale, True)
    torch.cuda.synchronize()
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool, device="cuda"), 1)
    G = Hq // Hkv
    for h in (0, Hq - 1):
        qf = q[0, h].float()
        kf = k[0, h // G].float()
        vf = v[0, h // G].float()
        s = (qf @ kf.T.contiguous()) * scale
        s.masked_fill_(mask, float("-inf"))
        ref = torch.softmax(s, dim=-1) @ vf
        want = ref.to(torch.bfloat16).cpu().view(torch.int16).numpy().view(np.uint16)
        assert_attn_close(paged.to_host_bits(out[0, h]), want, f"flash {S} D{D} head {h}")
        del s, ref


@pytest.mark.parametrize("S,causal", [(77, True), (200, False), (1, True)])
def test_flash_head_dim_256_vs_oracle(orc, S, causal):
    """Qwen3.5 attention shape (head_dim 256, 8 q / 2 kv heads) without paging."""
    import torch

    from genllm_amd import paged, synth

    B, Hq, Hkv, D = 1, 8, 2, 256
    scale = 1.0 / np.sqrt(D)
    q, k, v = _inputs(synth, 950 + S, B, Hq, Hkv, S, D)
    out = torch.empty((B, Hq, S, D), dtype=torch.bfloat16, device="cuda")
    paged.flash_attention(paged.to_device_bf16(q), paged.to_device_bf16(k), paged.to_device_bf16(v), out,
                          Hq // Hkv, scale, causal)
    torch.cuda.synchronize()
    assert_attn_close(paged.to_host_bits(out), orc.flash_attention(q, k, v, Hq // Hkv, scale, causal),
                      f"flash D256 S{S}")


def test_flash_rejects_bad_shapes():
    import torch

    from genllm_amd import paged
    from genllm_amd._lib import GenllmError

    q = torch.zeros((1, 4, 8, 64), dtype=torch.bfloat16, device="cuda")
    k = torch.zeros((1, 2, 8, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(GenllmError):  # head_dim 64: unsupported, as the CUDA op throws
        paged.flash_attention(q, k, k, torch.empty_like(q), 2, 0.125)
    q = torch.zeros((1, 6, 8, 128), dtype=torch.bfloat16, device="cuda")
    k = torch.zeros((1, 4, 8, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(GenllmError):  # 6 q heads cannot map onto 4 kv heads with groups 2
        paged.flash_attention(q, k, k, torch.empty_like(q), 2, 0.125)


@pytest.mark.parametrize("D", [128, 256])
def test_flash_special_values_vs_oracle(orc, D):
    """Non-paged causal attention with a NaN and a +inf in V rows and a NaN in
    a K row, each past some queries' causal limit.  The reference's two
    backends differ here: its CUDA kernel skips masked keys
    (src/backend/cuda/attention.cu:278-279), so such a V row reaches only the
    queries that see it, while its CPU loop (attention.cpp:39-121) gives
    masked keys a zero weight and 0 x NaN, 0 x inf are NaN for every earlier
    query.  The GPU op follows the CUDA kernel, exactly: outputs of queries
    that see a planted row are the oracle's, those of queries that do not are
    the oracle's with the planted V values zeroed (a masked key adds
    nothing); NaN and infinite outputs in the same places (values up to the
    sign of a NaN), finite outputs within the tolerance.  The CPU loop's
    non-finite set contains the GPU's."""
    import torch

    from genllm_amd import paged, synth
    from helpers import f32

    B, Hq, Hkv, S = 2, 8, 2, 150
    scale = 1.0 / np.sqrt(D)
    q, k, v = _inputs(synth, 1700 + D, B, Hq, Hkv, S, D)
    k, v = k.copy(), v.copy()
    v0 = v.copy()
    v[0, 1, 60, 7] = 0x7FC0   # NaN: batch 0, kv head 1 (q heads 4-7), key 60
    v[1, 0, 100, 3] = 0x7F80  # +inf: batch 1, kv head 0 (q heads 0-3), key 100
    k[1, 1, 120, 9] = 0xFFC0  # NaN score for key 120 of kv head 1 (q heads 4-7)
    out = torch.empty((B, Hq, S, D), dtype=torch.bfloat16, device="cuda")
    paged.flash_attention(paged.to_device_bf16(q), paged.to_device_bf16(k), paged.to_device_bf16(v), out,
                          Hq // Hkv, scale, True)
    torch.cuda.synchronize()
    cpu = orc.flash_attention(q, k, v, Hq // Hkv, scale, True)
    zeroed = orc.flash_attention(q, k, v0, Hq // Hkv, scale, True)
    sees = np.zeros(cpu.shape, dtype=bool)
    sees[0, 4:8, 60:] = True
    sees[1, 0:4, 100:] = True
    want = np.where(sees, cpu, zeroed).astype(np.uint16)
    got = paged.to_host_bits(out)
    gf, wf = f32(got), f32(want)
    assert np.array_equal(np.isnan(gf), np.isnan(wf)), "NaN outputs differ"
    assert np.array_equal(np.isinf(gf), np.isinf(wf)), "infinite outputs differ"
    nf = ~np.isfinite(wf)
    assert nf[0, 4:8, 60:, 7].all() and not nf[0, 4:8, :60].any(), "the NaN V row reaches queries 60.. only"
    assert np.isposinf(wf[1, 0:4, 100:, 3]).all() and not nf[1, 0:4, :100].any(), "+inf reaches queries 100.."
    assert np.isnan(wf[1, 4:8, 120:]).all() and not nf[1, 4:8, :120].any(), "the NaN score: queries 120.."
    assert np.array_equal(got[nf] & 0x7FFF, want[nf] & 0x7FFF)
    assert (~np.isfinite(f32(cpu)))[nf].all(), "the CPU loop's non-finite set contains the GPU's"
    assert_attn_close(np.where(nf, 0, got).astype(np.uint16), np.where(nf, 0, want).astype(np.uint16),
                      f"flash D{D} special values, finite outputs")
