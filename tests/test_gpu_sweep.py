"""Seeded random shapes through the decode and prefill kernels, against the
oracle's PagedAttentionImpl<CPU> loop (attention.cpp:148-215): kv heads, GQA
groups, head_dim, chunk length, cached tokens, causal or not and the pool's
fragmentation drawn from one generator per case, so that combinations the
named tests do not list (odd page counts, chunks that straddle pages, groups
of 1) are covered.  Tolerance as everywhere: max-abs <= 2^-7 max|ref|, rel-L2
<= 1e-2.  Sizes stay where the oracle takes well under a second."""
import numpy as np
import pytest

from genllm_amd import synth
from helpers import assert_attn_close, f32
from test_gpu_decode import Context
from test_gpu_prefill import run_prefill

pytestmark = pytest.mark.gpu


def decode_case(i):
    r = np.random.default_rng(0xDEC0 + i)
    D = int(r.choice([128, 256]))
    Hkv = int(r.choice([1, 2, 4, 8]))
    S = int(r.choice([1, 1, 1, 2, 3, 4]))
    G = int(r.choice([g for g in (1, 2, 4, 8, 16) if g * S <= 16]))
    N = int(r.integers(S, 3000))
    causal = bool(r.random() < 0.8)
    return D, Hkv, G, S, N, causal


def prefill_case(i):
    r = np.random.default_rng(0x9EF0 + i)
    D = int(r.choice([128, 256]))
    Hkv = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 4]))
    S = int(r.integers(17, 260))           # above the decode kernel's rows
    N = S + int(r.integers(0, 500))        # chunked: N - S tokens already cached
    causal = bool(r.random() < 0.8)
    return D, Hkv, G, S, N, causal


@pytest.mark.parametrize("i", range(24))
def test_decode_random_shapes(orc, i):
    D, Hkv, G, S, N, causal = decode_case(i)
    pool = (N + 15) // 16 + 1 + i % 7
    ctx = Context(orc, Hkv, D, pool, N, 9000 + i, nan_tail=True)
    q = synth.normal_bf16(9100 + i, (Hkv * G, S, D))
    got, _ = ctx.decode(q, causal=causal)
    assert_attn_close(got, ctx.oracle(q, causal), f"decode case {i}: D{D} Hkv{Hkv} G{G} S{S} N{N} causal{causal}")
    ctx.close()


@pytest.mark.parametrize("i", range(16))
def test_prefill_random_shapes(orc, i):
    D, Hkv, G, S, N, causal = prefill_case(i)
    pool = (N + 15) // 16 + 1 + i % 5
    ctx = Context(orc, Hkv, D, pool, N, 9500 + i, nan_tail=True)
    q = synth.normal_bf16(9600 + i, (Hkv * G, S, D))
    got = run_prefill(ctx, q, causal)
    assert_attn_close(got, ctx.oracle(q, causal), f"prefill case {i}: D{D} Hkv{Hkv} G{G} S{S} N{N} causal{causal}")
    ctx.close()


@pytest.mark.parametrize("i", range(8))
def test_decode_random_special_values(orc, i):
    """Seeded multi-query decode chunks with a NaN and a +inf planted in V rows
    and a NaN in a K row of the chunk's own keys (random kv head, dims and
    positions): the set of NaN and infinite outputs equals the oracle's (the
    values up to the sign of a NaN), and every finite output is held to the
    attention tolerance."""
    r = np.random.default_rng(0x5EC0 + i)
    D = int(r.choice([128, 256]))
    Hkv = int(r.choice([1, 2, 4, 8]))
    S = int(r.choice([2, 3, 4, 8]))
    G = int(r.choice([g for g in (1, 2, 4, 8) if g * S <= 16]))
    N = int(r.integers(S + 20, 2000))
    pool = (N + 15) // 16 + 2
    ctx = Context(orc, Hkv, D, pool, N, 9700 + i, nan_tail=True)
    kt, vt = ctx.ref.page_table(0)
    kp, vp = ctx.ref.pool_array(0, 0), ctx.ref.pool_array(0, 1)
    chunk = np.arange(N - S, N)
    h = int(r.integers(Hkv))
    t_nan, t_inf, t_k = (int(x) for x in r.choice(chunk, 3))
    d_nan, d_inf, d_k = (int(x) for x in r.integers(D, size=3))
    vp[vt[t_nan // 16], t_nan % 16, h, d_nan] = 0x7FC0
    vp[vt[t_inf // 16], t_inf % 16, h, d_inf] = 0x7F80
    kp[kt[t_k // 16], t_k % 16, h, d_k] = 0xFFC0
    ctx.mgr.write_pool(0, 0, np.ascontiguousarray(kp))
    ctx.mgr.write_pool(0, 1, np.ascontiguousarray(vp))
    q = synth.normal_bf16(9800 + i, (Hkv * G, S, D))
    got, _ = ctx.decode(q)
    want = ctx.oracle(q)
    label = f"special case {i}: D{D} Hkv{Hkv} G{G} S{S} N{N} v-nan {t_nan} v-inf {t_inf} k-nan {t_k}"
    gf, wf = f32(got), f32(want)
    assert np.array_equal(np.isnan(gf), np.isnan(wf)), label + ": NaN outputs differ"
    assert np.array_equal(np.isinf(gf), np.isinf(wf)), label + ": infinite outputs differ"
    nf = ~np.isfinite(wf)
    assert np.array_equal(got[nf] & 0x7FFF, want[nf] & 0x7FFF), label + ": non-finite bits"
    assert nf.any(), label + ": nothing planted reached an output"
    assert_attn_close(np.where(nf, 0, got).astype(np.uint16), np.where(nf, 0, want).astype(np.uint16), label)
    ctx.close()


@pytest.mark.parametrize("i", range(8))
def test_prefill_random_special_values(orc, i):
    """Seeded prefill chunks with a NaN and a +inf planted in V rows and a NaN
    in a K row of the chunk's own keys (random kv head, dims and positions,
    so that each row is past some queries' causal limit): the set of NaN and
    infinite outputs equals the oracle's (the values up to the sign of a NaN),
    and every finite output is held to the attention tolerance."""
    r = np.random.default_rng(0x5ED0 + i)
    D = int(r.choice([128, 256]))
    Hkv = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 4]))
    S = int(r.integers(40, 300))
    N = S + int(r.integers(0, 300))
    pool = (N + 15) // 16 + 2
    ctx = Context(orc, Hkv, D, pool, N, 9900 + i, nan_tail=True)
    kt, vt = ctx.ref.page_table(0)
    kp, vp = ctx.ref.pool_array(0, 0), ctx.ref.pool_array(0, 1)
    chunk = np.arange(N - S, N)
    h = int(r.integers(Hkv))
    t_nan, t_inf, t_k = (int(x) for x in r.choice(chunk, 3))
    d_nan, d_inf, d_k = (int(x) for x in r.integers(D, size=3))
    vp[vt[t_nan // 16], t_nan % 16, h, d_nan] = 0x7FC0
    vp[vt[t_inf // 16], t_inf % 16, h, d_inf] = 0x7F80
    kp[kt[t_k // 16], t_k % 16, h, d_k] = 0xFFC0
    ctx.mgr.write_pool(0, 0, np.ascontiguousarray(kp))
    ctx.mgr.write_pool(0, 1, np.ascontiguousarray(vp))
    q = synth.normal_bf16(9950 + i, (Hkv * G, S, D))
    got = run_prefill(ctx, q, True)
    want = ctx.oracle(q, True)
    label = f"prefill special case {i}: D{D} Hkv{Hkv} G{G} S{S} N{N} v-nan {t_nan} v-inf {t_inf} k-nan {t_k}"
    gf, wf = f32(got), f32(want)
    assert np.array_equal(np.isnan(gf), np.isnan(wf)), label + ": NaN outputs differ"
    assert np.array_equal(np.isinf(gf), np.isinf(wf)), label + ": infinite outputs differ"
    nf = ~np.isfinite(wf)
    assert np.array_equal(got[nf] & 0x7FFF, want[nf] & 0x7FFF), label + ": non-finite bits"
    assert nf.any(), label + ": nothing planted reached an output"
    assert_attn_close(np.where(nf, 0, got).astype(np.uint16), np.where(nf, 0, want).astype(np.uint16), label)
    ctx.close()


@pytest.mark.parametrize("i", range(12))
def test_decode_random_tuned(orc, i):
    """Seeded decode shapes under a random decode tuning (genllm_decode_tuning):
    the merge in a kernel or in the last split workgroup, 1 or 4 kv heads per
    split workgroup, and forced split sizes from one page up."""
    r = np.random.default_rng(0x7E40 + i)
    D = int(r.choice([128, 256]))
    Hkv = int(r.choice([2, 4, 8]))
    S = int(r.choice([1, 1, 2, 4]))
    G = int(r.choice([g for g in (1, 2, 4, 8) if g * S <= 16]))
    N = int(r.integers(S, 5000))
    merge = str(r.choice(["kernel", "fused"]))
    heads = int(r.choice([0, 1, 4])) if Hkv % 4 == 0 else int(r.choice([0, 1]))
    pps = int(r.choice([0, 1, 3, 17, 64]))
    pool = (N + 15) // 16 + 1 + i % 3
    ctx = Context(orc, Hkv, D, pool, N, 9200 + i, nan_tail=True)
    q = synth.normal_bf16(9300 + i, (Hkv * G, S, D))
    got, _ = ctx.decode(q, pps=pps or None, merge=merge, heads=heads)
    assert_attn_close(got, ctx.oracle(q), f"tuned case {i}: D{D} Hkv{Hkv} G{G} S{S} N{N} {merge} heads{heads} pps{pps}")
    ctx.close()


@pytest.mark.parametrize("i", range(6))
def test_prefill_random_token_layout(orc, i):
    """Seeded prefill chunks with q and out token-major ([S][Hq][D], the
    layout a fused projection writes), against the head-major oracle."""
    D, Hkv, G, S, N, causal = prefill_case(100 + i)
    pool = (N + 15) // 16 + 1 + i % 4
    ctx = Context(orc, Hkv, D, pool, N, 9400 + i, nan_tail=True)
    q = synth.normal_bf16(9450 + i, (Hkv * G, S, D))
    got = run_prefill(ctx, np.ascontiguousarray(q.transpose(1, 0, 2)), causal, q_layout="token")
    assert_attn_close(np.ascontiguousarray(got.transpose(1, 0, 2)), ctx.oracle(q, causal),
                      f"token-layout prefill {i}: D{D} Hkv{Hkv} G{G} S{S} N{N} causal{causal}")
    ctx.close()


@pytest.mark.parametrize("i", range(10))
def test_op_random_sequences(orc, i):
    """Seeded sequences of op steps (genllm_paged_attention: append, then
    attend) on one layer: prefill chunks and decode steps of random length,
    batch 2 for short steps, fp16 or bf16 layers; every step's output, page
    tables and cached count against the oracle op's."""
    from test_gpu_f16_batch import make, step

    r = np.random.default_rng(0x0B5E80 + i)
    D = int(r.choice([128, 256]))
    Hkv = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 4]))
    f16 = bool(r.random() < 0.5)
    pool = int(r.integers(40, 120))
    mgr, ref = make(orc, Hkv, D, pool, 51000 + 11 * i, orc.F16 if f16 else orc.BF16)
    n = 0
    for j in range(int(r.integers(2, 6))):
        S = int(r.choice([1, 1, 2, 3, int(r.integers(4, 200))]))
        batch = int(r.choice([1, 1, 2])) if S <= 4 else 1
        if n + S > pool * 16 - 16:
            break
        step(orc, mgr, ref, Hkv * G, Hkv, S, D, 61000 + 97 * i + j,
             f"sequence {i} step {j}: D{D} Hkv{Hkv} G{G} {'fp16' if f16 else 'bf16'} n{n} S{S} batch{batch}",
             f16=f16, batch=batch)
        n += S
