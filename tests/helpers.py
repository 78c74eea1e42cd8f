"""Shared helpers for the GPU parity tests (error metrics, oracle set-up)."""
import math

import numpy as np

from genllm_amd import synth


def f32(bits):
    return synth.bf16_bits_to_f32(bits)


def attn_errors(got_bits, want_bits):
    """max-abs and relative-L2 error of bf16 attention outputs."""
    g = f32(got_bits).astype(np.float64)
    w = f32(want_bits).astype(np.float64)
    max_abs = float(np.max(np.abs(g - w)))
    rel_l2 = float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30))
    return max_abs, rel_l2, float(np.max(np.abs(w)))


# Attention tolerance (bf16 output, fp32 accumulate): max-abs <= 2^-7 max|ref|, rel-L2 <= 1e-2.
ATTN_MAX_ABS_FRAC = 2.0 ** -7
ATTN_REL_L2 = 1e-2


def assert_attn_close(got_bits, want_bits, label=""):
    max_abs, rel_l2, ref_max = attn_errors(got_bits, want_bits)
    print(f"[{label}] max_abs={max_abs:.3e} (bound {ATTN_MAX_ABS_FRAC * ref_max:.3e}) rel_l2={rel_l2:.3e}",
          flush=True)
    assert np.all(np.isfinite(f32(got_bits))), f"{label}: non-finite output"
    assert max_abs <= ATTN_MAX_ABS_FRAC * ref_max, f"{label}: max_abs {max_abs} > {ATTN_MAX_ABS_FRAC * ref_max}"
    assert rel_l2 <= ATTN_REL_L2, f"{label}: rel_l2 {rel_l2}"


def ulp_diff(a_bits, b_bits):
    """Distance in bf16 units in the last place (same-sign monotone mapping)."""
    def key(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(key(a_bits) - key(b_bits))


def oracle_fragmented(orc, Hkv, D, pool, perm_k, perm_v, layer=0, m=None):
    """Oracle manager (a new one, or layer `layer` added to `m`) whose block
    pools hand out perm_k / perm_v first, as PagedAttentionManager.fragment."""
    m = m if m is not None else orc.Manager(with_pool=True)
    m.init_layer(layer, Hkv, D)
    m.reserve_layer(layer, pool)
    for which, perm in ((0, perm_k), (1, perm_v)):
        p = m.pool(layer, which)
        for _ in range(pool):
            p.alloc()
        for b in np.asarray(perm)[::-1]:
            p.free(int(b))
    return m


def scale_for(D):
    return 1.0 / math.sqrt(D)


def f16(bits):
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# fp16 outputs (10-bit mantissa; probabilities rounded to fp16 in the MFMAs)
ATTN_F16_MAX_ABS_FRAC = 2.0 ** -8
ATTN_F16_REL_L2 = 4e-3


def assert_attn_close_f16(got_bits, want_bits, label=""):
    g = f16(got_bits).astype(np.float64)
    w = f16(want_bits).astype(np.float64)
    max_abs = float(np.max(np.abs(g - w)))
    rel_l2 = float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30))
    ref_max = float(np.max(np.abs(w)))
    print(f"[{label}] fp16 max_abs={max_abs:.3e} (bound {ATTN_F16_MAX_ABS_FRAC * ref_max:.3e}) rel_l2={rel_l2:.3e}",
          flush=True)
    assert np.all(np.isfinite(g)), f"{label}: non-finite output"
    assert max_abs <= ATTN_F16_MAX_ABS_FRAC * ref_max, f"{label}: max_abs {max_abs}"
    assert rel_l2 <= ATTN_F16_REL_L2, f"{label}: rel_l2 {rel_l2}"
