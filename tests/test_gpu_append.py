"""GPU parity: MFMA operand layout, stand-alone RMSNorm / RoPE, page scatter and
the fused q/k-norm -> RoPE -> scatter append, all through libgenllm_hip.so,
against the CPU oracle on the same seeded inputs.

Bars: page placement, block-table gathers and V pages bit-exact; RMSNorm and
RoPE bit-exact (the kernels reproduce the reference's summation order, its
truncating store and GCC's contraction of the rotation); RoPE'd K within one
bf16 ulp (fractions reported).
"""
import numpy as np
import pytest
import torch

from genllm_amd import paged, synth
from helpers import f32, oracle_fragmented, ulp_diff

pytestmark = pytest.mark.gpu


def dev(bits):
    return paged.to_device_bf16(bits)


@pytest.mark.parametrize("k", [32, 16])
def test_mfma_operand_layout(k):
    a = synth.normal_bf16(1, (16, k))
    b = synth.normal_bf16(2, (k, 16))
    c = torch.zeros((16, 16), dtype=torch.float32, device="cuda")
    paged.selftest_mfma(dev(a), dev(b), c)
    torch.cuda.synchronize()
    want = f32(a).astype(np.float64) @ f32(b).astype(np.float64)
    got = c.cpu().numpy().astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want)) + 1e-5


@pytest.mark.parametrize("hidden,rows", [(128, 4096), (4, 2), (12, 33), (64, 100), (256, 50), (2560, 7)])
def test_rms_norm_bit_exact(orc, hidden, rows):
    x = synth.normal_bf16(10 + hidden, (rows, hidden))
    w = synth.uniform_f32(11, (hidden,), 0.5, 1.5)
    out = torch.empty((rows, hidden), dtype=torch.bfloat16, device="cuda")
    paged.rms_norm(out, dev(x), torch.from_numpy(w).cuda(), 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(paged.to_host_bits(out), orc.rms_norm(x, w, 1e-6))


def test_rms_norm_reference_case(orc):
    x = synth.f32_to_bf16_bits(np.array([[1, 2, 3, 4], [2, 4, 6, 8]], dtype=np.float32))
    w = np.ones(4, dtype=np.float32)
    out = torch.empty((2, 4), dtype=torch.bfloat16, device="cuda")
    paged.rms_norm(out, dev(x), torch.from_numpy(w).cuda(), 1e-5)
    torch.cuda.synchronize()
    assert np.array_equal(paged.to_host_bits(out), orc.rms_norm(x, w, 1e-5))


@pytest.mark.parametrize("H,S,start", [(8, 4096, 0), (32, 1, 8192), (3, 17, 5)])
def test_apply_rope_bit_exact(orc, H, S, start):
    D = 128
    cos, sin = paged.rope_cache(1e6, D, start + S)
    x = synth.normal_bf16(20 + H, (H, S, D))
    out = torch.empty((H, S, D), dtype=torch.bfloat16, device="cuda")
    paged.apply_rope(out, dev(x), torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(), start)
    torch.cuda.synchronize()
    assert np.array_equal(paged.to_host_bits(out), orc.apply_rope(x, cos, sin, start))


def test_kv_scatter_bit_exact():
    """Plain scatter: every row lands at pool[id[g/16]][g%16][h] (closed form)."""
    S, Hkv, D, blocks = 77, 8, 128, 40
    pos0 = 13
    k = synth.normal_bf16(30, (S, Hkv, D))
    v = synth.normal_bf16(31, (S, Hkv, D))
    n_pages = (pos0 + S + 15) // 16
    ids_k = synth.shuffled(32, blocks)[:n_pages].astype(np.int32)
    ids_v = synth.shuffled(33, blocks)[:n_pages].astype(np.int32)
    kp = torch.zeros((blocks, 16, Hkv, D), dtype=torch.bfloat16, device="cuda")
    vp = torch.zeros_like(kp)
    paged.kv_scatter(dev(k), dev(v), kp, vp, torch.from_numpy(ids_k).cuda(), torch.from_numpy(ids_v).cuda(), pos0)
    torch.cuda.synchronize()
    kh, vh = paged.to_host_bits(kp), paged.to_host_bits(vp)
    want_k = np.zeros_like(kh)
    want_v = np.zeros_like(vh)
    for t in range(S):
        g = pos0 + t
        want_k[ids_k[g // 16], g % 16] = k[t]
        want_v[ids_v[g // 16], g % 16] = v[t]
    assert np.array_equal(kh, want_k) and np.array_equal(vh, want_v)


def _append_case(orc, S, Hkv, D, pool, start_tokens, seed, with_q=False, Hq=32, head_major=False, rope_dim=None,
                 theta=1e6):
    cos, sin = paged.rope_cache(theta, rope_dim or D, start_tokens + S + 1)
    k = synth.normal_bf16(seed, (S, Hkv, D))
    v = synth.normal_bf16(seed, (S, Hkv, D), offset=1 << 26)
    gk = synth.uniform_f32(seed + 1, (D,), 0.5, 1.5)
    gq = synth.uniform_f32(seed + 2, (D,), 0.5, 1.5)
    q = synth.normal_bf16(seed, (S, Hq, D), offset=2 << 26) if with_q else None
    perm_k, perm_v = synth.shuffled(seed, pool), synth.shuffled(seed + 3, pool)

    mgr = paged.PagedAttentionManager(2 * pool * 16 * Hkv * D * 2 + (1 << 20))
    mgr.init_layer(0, Hkv, D)
    mgr.reserve_layer(0, pool)
    mgr.fragment(0, perm_k, perm_v)
    ref = oracle_fragmented(orc, Hkv, D, pool, perm_k, perm_v)
    if start_tokens:
        mgr.append_kv_pages(0, start_tokens)
        ref.append_kv_pages(0, start_tokens)
    if head_major:
        kd = dev(np.ascontiguousarray(k.transpose(1, 0, 2))).permute(1, 0, 2)
        vd = dev(np.ascontiguousarray(v.transpose(1, 0, 2))).permute(1, 0, 2)
    else:
        kd, vd = dev(k), dev(v)
    q_out = torch.empty((Hq, S, D), dtype=torch.bfloat16, device="cuda") if with_q else None
    print(f"append S={S} Hkv={Hkv} D={D} pool={pool} start={start_tokens} q={with_q} head_major={head_major}",
          flush=True)
    paged.qk_norm_rope_append(mgr, 0, kd, vd, torch.from_numpy(gk).cuda(), 1e-6, torch.from_numpy(cos).cuda(),
                              torch.from_numpy(sin).cuda(), start_tokens,
                              q=dev(q) if with_q else None, gamma_q=torch.from_numpy(gq).cuda() if with_q else None,
                              q_out=q_out)
    torch.cuda.synchronize()
    want_q = ref.qk_norm_rope_append(0, k, v, gk, 1e-6, cos, sin, start_tokens, q_tok=q, gamma_q=gq)
    # page tables: host, device and oracle agree bit for bit
    kt, vt = mgr.page_table(0)
    rk, rv = ref.page_table(0)
    assert np.array_equal(kt, rk) and np.array_equal(vt, rv)
    dk, dv = mgr.read_device_table(0)
    assert np.array_equal(dk, kt) and np.array_equal(dv, vt)
    # V pages bit-exact, K within one bf16 ulp
    assert np.array_equal(mgr.read_pool(0, 1), ref.pool_array(0, 1))
    gk_pool, rk_pool = mgr.read_pool(0, 0), ref.pool_array(0, 0)
    d = ulp_diff(gk_pool, rk_pool)
    n = d.size
    print(f"  K exact {np.mean(d == 0):.6f}, 1-ulp {np.mean(d == 1):.2e}, >1-ulp {np.sum(d > 1)} of {n}", flush=True)
    assert np.all(d <= 1)
    if with_q:
        dq = ulp_diff(paged.to_host_bits(q_out), want_q)
        print(f"  q exact {np.mean(dq == 0):.6f}, >1-ulp {np.sum(dq > 1)}", flush=True)
        assert np.all(dq <= 1)
    mgr.close()
    return d


def test_fused_append_config2(orc):
    """Qwen3-4B K/V append of one 4096-token chunk into 256
    pages of a shuffled 1024-page pool."""
    _append_case(orc, 4096, 8, 128, 1024, 0, synth.config_seed(2))


def test_fused_append_decode_step_with_q(orc):
    """Config 3's append: one token at position 8192 opens page 513; q fused."""
    _append_case(orc, 1, 8, 128, 2048, 8192, synth.config_seed(3), with_q=True, Hq=32)


@pytest.mark.parametrize("S,start", [(37, 5), (16, 16), (3, 14)])
def test_fused_append_ragged_and_head_major(orc, S, start):
    _append_case(orc, S, 8, 128, 16, start, 90 + S, head_major=True)


@pytest.mark.parametrize("D,Hkv", [(64, 4), (256, 2), (128, 3)])
def test_fused_append_other_shapes(orc, D, Hkv):
    _append_case(orc, 45, Hkv, D, 8, 7, 123 + D, with_q=True, Hq=2 * Hkv)


@pytest.mark.parametrize("S,start", [(45, 7), (1, 300)])
def test_fused_append_qwen35_partial_rotary(orc, S, start):
    """Qwen3.5 attention layer (Qwen35.cpp:191-226): head_dim 256, 8 q / 2 kv
    heads, RoPE on the first 64 dims (rope_dimension_count, Qwen35.hpp:14-16,
    theta 1e7), the other 192 passed through after the norm."""
    _append_case(orc, S, 2, 256, 40, start, 350 + S, with_q=True, Hq=8, rope_dim=64, theta=1e7)


def test_fused_append_partial_rotary_d128(orc):
    _append_case(orc, 33, 8, 128, 8, 3, 360, with_q=True, Hq=16, rope_dim=64)


@pytest.mark.parametrize("D,rope_dim", [(256, 64), (256, 128), (128, 64), (256, 256)])
def test_apply_rope_partial_bit_exact(orc, D, rope_dim):
    H, S, start = 5, 19, 11
    cos, sin = paged.rope_cache(1e7, rope_dim, start + S)
    x = synth.normal_bf16(40 + D + rope_dim, (H, S, D))
    out = torch.empty((H, S, D), dtype=torch.bfloat16, device="cuda")
    paged.apply_rope(out, dev(x), torch.from_numpy(cos).cuda(), torch.from_numpy(sin).cuda(), start)
    torch.cuda.synchronize()
    assert np.array_equal(paged.to_host_bits(out), orc.apply_rope_partial(x, cos, sin, start))
