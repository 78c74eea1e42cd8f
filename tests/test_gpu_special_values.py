"""Special values through the attention kernels, against the oracle's
PagedAttentionImpl<CPU> loop (attention.cpp:160-214): a NaN in one cached K
row, a NaN in two dims of one cached V row, and a kv head whose V rows are
all bf16 subnormals.

Every output goes through bfloat16_t's constructor (bfloat16.hpp:18-41): a
NaN becomes sign | 0x7F81 and an fp32 subnormal becomes a signed zero.  The
NaN's sign is whatever the arithmetic that produced it left (IEEE 754 does
not fix it), so NaN outputs are compared as (bits & 0x7FFF) == 0x7F81; the
subnormal head's outputs are compared bit for bit; every finite output is
held to the attention tolerance (max-abs <= 2^-7 max|ref|, rel-L2 <= 1e-2).

A NaN score (NaN in K) poisons exactly the queries whose window holds the
key in both: the reference's std::fmax keeps m and exp(NaN - m) feeds l and
o, the kernels' masked scores are -inf before the exponent.  A NaN in V
reaches exactly the queries that see its row in both as well: the kernels'
matrix products would also meet it with the zero probabilities of queries
that do not see it (0 x NaN is NaN), so a decode page holding the query
chunk's own keys with such a row leaves them out of the product and adds
them per row, and a prefill wave whose state comes out non-finite forms its
key half again per query over the keys each query sees.  No output may
differ from the reference's."""
import numpy as np
import pytest

from genllm_amd import synth
from helpers import assert_attn_close, f32
from test_gpu_decode import Context
from test_gpu_prefill import run_prefill

pytestmark = pytest.mark.gpu

D = 128
HKV = 8
HQ = 16
K_NAN_HEAD, K_NAN_DIM = 5, 9
V_NAN_HEAD, V_NAN_DIMS = 3, (5, 77)
SUB_HEAD = 1


def plant(ctx, k_pos, v_pos):
    """NaN into K[k_pos] (kv head K_NAN_HEAD, one dim) and V[v_pos] (kv head
    V_NAN_HEAD, two dims); V of kv head SUB_HEAD becomes positive subnormals
    in even dims and negative ones in odd dims.  Same bits in the oracle's
    pools and the GPU's."""
    kt, vt = ctx.ref.page_table(0)
    kp, vp = ctx.ref.pool_array(0, 0), ctx.ref.pool_array(0, 1)
    kp[kt[k_pos // 16], k_pos % 16, K_NAN_HEAD, K_NAN_DIM] = 0x7FC0
    for d in V_NAN_DIMS:
        vp[vt[v_pos // 16], v_pos % 16, V_NAN_HEAD, d] = 0xFFC1
    rng = np.random.default_rng(77)
    mant = rng.integers(1, 0x80, size=vp[:, :, SUB_HEAD, :].shape, dtype=np.uint16)
    sign = np.where(np.arange(D) % 2 == 1, 0x8000, 0).astype(np.uint16)
    vp[:, :, SUB_HEAD, :] = mant | sign
    ctx.mgr.write_pool(0, 0, np.ascontiguousarray(kp))
    ctx.mgr.write_pool(0, 1, np.ascontiguousarray(vp))


def check(got, want, exposed, label):
    """got/want [Hq][S][D] bf16 bits.  exposed: bool [Hq][S][D], where got may be
    NaN although want is finite (none of the tests below allows any)."""
    g_nan, w_nan = np.isnan(f32(got)), np.isnan(f32(want))
    assert np.all((want[w_nan] & 0x7FFF) == 0x7F81), f"{label}: oracle NaN pattern"
    assert np.all((got[w_nan] & 0x7FFF) == 0x7F81), f"{label}: NaN outputs not sign | 0x7F81"
    extra = g_nan & ~w_nan
    assert not np.any(extra & ~exposed), f"{label}: NaN where the reference is finite at {np.argwhere(extra & ~exposed)[:4]}"
    sub = slice(SUB_HEAD * (HQ // HKV), (SUB_HEAD + 1) * (HQ // HKV))
    even = want[sub][..., 0::2]
    odd = want[sub][..., 1::2]
    assert np.all(even == 0x0000) and np.all(odd == 0x8000), f"{label}: oracle subnormal outputs"
    assert np.array_equal(got[sub], want[sub]), f"{label}: subnormal outputs not the signed zeros of the reference"
    keep = ~(w_nan | extra)
    assert_attn_close(np.where(keep, got, 0).astype(np.uint16), np.where(keep, want, 0).astype(np.uint16), label)
    return int(extra.sum())


def expected_nan_rows(q_abs, k_pos, v_pos):
    """[Hq][S][D] mask of the reference's NaN outputs for absolute query positions q_abs."""
    m = np.zeros((HQ, len(q_abs), D), dtype=bool)
    G = HQ // HKV
    sees_k = np.asarray(q_abs) >= k_pos
    sees_v = np.asarray(q_abs) >= v_pos
    m[K_NAN_HEAD * G:(K_NAN_HEAD + 1) * G, sees_k, :] = True
    for d in V_NAN_DIMS:
        m[V_NAN_HEAD * G:(V_NAN_HEAD + 1) * G, sees_v, d] = True
    return m


@pytest.mark.parametrize("S,pps,k_pos,v_pos", [(1, None, 600, 517), (1, 4, 600, 517), (3, None, 600, 517),
                                               (3, None, 999, 998), (8, 3, 996, 994)])
def test_decode_special_values(orc, S, pps, k_pos, v_pos):
    """The planted rows either precede the whole query chunk, so every query
    sees them, or sit inside it.  A NaN K row inside the chunk stays exact (its
    score is masked to -inf before the exponent); so does a NaN V row inside
    it (the page leaves the chunk's keys out of the P.V MFMA and adds them per
    row, over the rows that see them): no output may differ from the
    reference's."""
    N = 1000
    ctx = Context(orc, HKV, D, (N + 15) // 16 + 4, N, 8100 + S + v_pos)
    plant(ctx, k_pos, v_pos)
    q = synth.normal_bf16(8200 + S, (HQ, S, D))
    got, _ = ctx.decode(q, pps=pps)
    want = ctx.oracle(q)
    q_abs = np.arange(N - S, N)
    assert np.array_equal(np.isnan(f32(want)), expected_nan_rows(q_abs, k_pos, v_pos))
    check(got, want, np.zeros_like(want, dtype=bool), f"decode S{S} pps{pps} k{k_pos} v{v_pos}")
    ctx.close()


@pytest.mark.parametrize("S,N", [(300, 300), (200, 333)])
def test_prefill_special_values(orc, S, N):
    ctx = Context(orc, HKV, D, (N + 15) // 16 + 5, N, 8300 + S + N)
    k_pos, v_pos = N - S + 120, N - S + 150
    plant(ctx, k_pos, v_pos)
    q = synth.normal_bf16(8400 + S, (HQ, S, D))
    got = run_prefill(ctx, q)
    want = ctx.oracle(q)
    q_abs = np.arange(N - S, N)
    assert np.array_equal(np.isnan(f32(want)), expected_nan_rows(q_abs, k_pos, v_pos))
    check(got, want, np.zeros_like(want, dtype=bool), f"prefill S{S} N{N}")
    ctx.close()
