"""ctypes view of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by the ``cpu_baseline`` leg of ``bench.py`` -- always as the checker or the
timed CPU baseline, never as part of the product path.  The product
(``genllm_amd``) never imports this package.

Each wrapped function restates a reference function; the C sources cite the
reference file:line (see oracle.h).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")

BF16 = 30
F16 = 1
PAGE = 16


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_SO):
        subprocess.run(["make", "-s", "-C", _HERE, "-j4"], check=True)
    return _SO


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        build()
        _lib = C.CDLL(_SO)
        _declare(_lib)
    return _lib


_P = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_f = C.c_float
_sz = C.c_size_t


def _declare(L):
    sig = {
        "or_f32_to_f16": (C.c_uint16, [_f]),
        "or_f16_to_f32": (_f, [C.c_uint16]),
        "or_paged_attention_dt": (C.c_int, [_P, _i32, _P, _P, _P, _P, _i32, _i32, _i32, _i32, _i32, _i32, _f,
                                            C.c_int, _i32]),
        "or_paged_attend_dt": (C.c_int, [_P, _i32, _P, _P, _i32, _i32, _i32, _i32, _i32, _i32, _f, C.c_int, _i32]),
        "or_f32_to_bf16": (C.c_uint16, [_f]),
        "or_bf16_to_f32": (_f, [C.c_uint16]),
        "or_f32_to_bf16_array": (None, [_P, _P, _sz]),
        "or_bf16_to_f32_array": (None, [_P, _P, _sz]),
        "or_pool_create": (_P, [_P, _sz, _i32, _i32, _i32, _sz]),
        "or_pool_destroy": (None, [_P]),
        "or_pool_alloc": (_i32, [_P]),
        "or_pool_free": (None, [_P, _i32]),
        "or_pool_reset": (None, [_P]),
        "or_pool_block_data": (_P, [_P, _i32]),
        "or_pool_num_blocks": (_i32, [_P]),
        "or_pool_num_free": (_i32, [_P]),
        "or_mgr_create": (_P, [C.c_int]),
        "or_mgr_destroy": (None, [_P]),
        "or_mgr_init_layer": (None, [_P, _i32, _i32, _i32, _i32]),
        "or_mgr_reserve_layer": (None, [_P, _i32, _i32]),
        "or_mgr_append_kv_pages": (None, [_P, _i32, _i32]),
        "or_mgr_append_kv_from_tensor": (None, [_P, _i32, _P, _P, _i32, _i32, _i32, _i32]),
        "or_mgr_append_kv_from_pos": (None, [_P, _i32, _P, _P, _i32, _i32, _i32, _i32, _i32]),
        "or_mgr_reset": (None, [_P]),
        "or_mgr_is_active": (C.c_int, [_P, _i32]),
        "or_mgr_num_cached": (_i32, [_P, _i32]),
        "or_mgr_num_pages": (_i32, [_P, _i32]),
        "or_mgr_get_page_table": (_i32, [_P, _i32, _P, _P, _i32]),
        "or_mgr_set_page_table": (None, [_P, _i32, _P, _P, _i32, _i32]),
        "or_mgr_k_pool": (_P, [_P, _i32]),
        "or_mgr_v_pool": (_P, [_P, _i32]),
        "or_mgr_pool": (_P, [_P, _i32, C.c_int]),
        "or_rms_norm": (None, [_P, _P, _P, _sz, _sz, _f]),
        "or_rope_cache": (None, [_P, _f, C.c_int, C.c_int, C.c_int]),
        "or_apply_rope": (None, [_P, _P, _P, _P, _i64, _i64, _i64, _i64]),
        "or_permute_tok_to_head": (None, [_P, _P, _i64, _i64, _i64]),
        "or_permute_head_to_tok": (None, [_P, _P, _i64, _i64, _i64]),
        "or_paged_attention": (C.c_int, [_P, _i32, _P, _P, _P, _P, _i32, _i32, _i32, _i32, _i32, _i32, _f, C.c_int]),
        "or_paged_attend": (C.c_int, [_P, _i32, _P, _P, _i32, _i32, _i32, _i32, _i32, _i32, _f, C.c_int]),
        "or_flash_attention": (None, [_P, _P, _P, _P, _i32, _i32, _i32, _i32, _i32, _i32, _f, C.c_int]),
        "or_qk_norm_rope_append": (None, [_P, _i32, _P, _i32, _P, _P, _P, _P, _i32, _i32, _i32, _P, _f, _P, _P, _i32,
                                          _i64]),
        "or_apply_rope_partial": (None, [_P, _P, _P, _P, _i64, _i64, _i64, _i64, _i64]),
        "or_linear_bf16": (None, [_P, _P, _P, _i64, _i64, _i64, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return a.ctypes.data


# ---------------------------------------------------------------- helpers

def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_bf16_array(ptr(x), ptr(out), x.size)
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    """float16_t(float) bit patterns (or_f32_to_f16, one call per element)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = lib().or_f32_to_f16
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.uint16).reshape(x.shape)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    """float(float16_t) (or_f16_to_f32, one call per element)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    f = lib().or_f16_to_f32
    return np.array([f(int(v)) for v in h.ravel()], dtype=np.float32).reshape(h.shape)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.float32)
    hidden = w.size
    out = np.empty_like(x)
    lib().or_rms_norm(ptr(out), ptr(x), ptr(w), x.size // hidden, hidden, eps)
    return out


def rope_cache(theta: float, head_dim: int, max_seq: int):
    cos = np.empty((max_seq, head_dim), dtype=np.float32)
    sin = np.empty((max_seq, head_dim), dtype=np.float32)
    lib().or_rope_cache(ptr(cos), theta, head_dim, max_seq, 1)
    lib().or_rope_cache(ptr(sin), theta, head_dim, max_seq, 0)
    return cos, sin


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, start_pos: int) -> np.ndarray:
    """x head-major [H][S][D] bf16 bits."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    H, S, D = x.shape
    out = np.empty_like(x)
    lib().or_apply_rope(ptr(out), ptr(x), ptr(cos), ptr(sin), H, S, D, start_pos)
    return out


def linear(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """x [rows][common], w [cols][common], bias [cols] (bf16 bits) -> out [rows][cols]."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    rows, common = x.shape
    cols = w.shape[0]
    assert w.shape[1] == common
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.uint16)
        assert bias.shape == (cols,)
    out = np.empty((rows, cols), dtype=np.uint16)
    lib().or_linear_bf16(ptr(out), ptr(x), ptr(w), rows, common, cols, ptr(bias))
    return out


def apply_rope_partial(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, start_pos: int) -> np.ndarray:
    """x head-major [H][S][D] bf16 bits; tables [max_seq][rope_dim]."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    H, S, D = x.shape
    out = np.empty_like(x)
    lib().or_apply_rope_partial(ptr(out), ptr(x), ptr(cos), ptr(sin), H, S, D, cos.shape[1], start_pos)
    return out


def flash_attention(q, k, v, groups, scale, causal):
    """q [B,Hq,S,D], k/v [B,Hkv,S,D] bf16 bits."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    B, Hq, S, D = q.shape
    out = np.empty_like(q)
    lib().or_flash_attention(ptr(q), ptr(k), ptr(v), ptr(out), B, Hq, S, k.shape[1], D, groups, scale,
                             int(causal))
    return out


class BlockPool:
    """BlockPool (page_attention.h:11-45) over no real buffer (like the fakes of
    test_page_attention.cpp, whose block data is never touched)."""

    def __init__(self, capacity: int, n_kv_heads: int = 8, head_dim: int = 128, elem_size: int = 2):
        self._h = lib().or_pool_create(None, 0, capacity, n_kv_heads, head_dim, elem_size)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_pool_destroy(self._h)
            self._h = None

    def alloc(self) -> int:
        return lib().or_pool_alloc(self._h)

    def free(self, i: int):
        lib().or_pool_free(self._h, i)

    def reset(self):
        lib().or_pool_reset(self._h)

    def num_blocks(self) -> int:
        return lib().or_pool_num_blocks(self._h)

    def num_free(self) -> int:
        return lib().or_pool_num_free(self._h)


class _PoolView:
    def __init__(self, h):
        self._h = h

    def alloc(self):
        return lib().or_pool_alloc(self._h)

    def free(self, i):
        lib().or_pool_free(self._h, i)

    def num_blocks(self):
        return lib().or_pool_num_blocks(self._h)

    def num_free(self):
        return lib().or_pool_num_free(self._h)


class Manager:
    """PagedAttentionManager restated (page_attention.cpp:66-216)."""

    def __init__(self, with_pool: bool = True):
        # the destructor is held by the instance: at interpreter exit the
        # module's globals (lib) may already be gone when __del__ runs
        self._destroy = lib().or_mgr_destroy
        self._h = lib().or_mgr_create(int(with_pool))
        self._shapes = {}

    def close(self):
        h, self._h = getattr(self, "_h", None), None
        destroy = getattr(self, "_destroy", None)
        if h and destroy is not None:
            destroy(h)

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: nothing left to release
            pass

    def init_layer(self, layer, n_kv_heads, head_dim, dtype=BF16):
        self._shapes[layer] = (n_kv_heads, head_dim)
        lib().or_mgr_init_layer(self._h, layer, n_kv_heads, head_dim, dtype)

    def reserve_layer(self, layer, max_blocks):
        self._shapes.setdefault(layer, (0, 0))
        self._shapes[layer] = self._shapes[layer] + (max_blocks,)
        lib().or_mgr_reserve_layer(self._h, layer, max_blocks)

    def append_kv_pages(self, layer, count):
        lib().or_mgr_append_kv_pages(self._h, layer, count)

    def append_kv_from_tensor(self, layer, K, V):
        K = np.ascontiguousarray(K, dtype=np.uint16)
        V = np.ascontiguousarray(V, dtype=np.uint16)
        Hkv, S, D = K.shape
        lib().or_mgr_append_kv_from_tensor(self._h, layer, ptr(K), ptr(V), Hkv, S, D, BF16)

    def append_kv_from_pos(self, layer, K, V, global_pos):
        """K/V head-major [Hkv][count][D]."""
        K = np.ascontiguousarray(K, dtype=np.uint16)
        V = np.ascontiguousarray(V, dtype=np.uint16)
        Hkv, count, D = K.shape
        lib().or_mgr_append_kv_from_pos(self._h, layer, ptr(K), ptr(V), Hkv, D, BF16, global_pos, count)

    def reset(self):
        lib().or_mgr_reset(self._h)

    def is_active(self, layer) -> bool:
        return bool(lib().or_mgr_is_active(self._h, layer))

    def num_cached(self, layer) -> int:
        return lib().or_mgr_num_cached(self._h, layer)

    def num_pages(self, layer) -> int:
        return lib().or_mgr_num_pages(self._h, layer)

    def page_table(self, layer):
        n = lib().or_mgr_get_page_table(self._h, layer, None, None, 0)
        k = np.empty(n, dtype=np.int32)
        v = np.empty(n, dtype=np.int32)
        lib().or_mgr_get_page_table(self._h, layer, ptr(k), ptr(v), n)
        return k, v

    def set_page_table(self, layer, k_ids, v_ids, num_cached):
        k = np.ascontiguousarray(k_ids, dtype=np.int32)
        v = np.ascontiguousarray(v_ids, dtype=np.int32)
        lib().or_mgr_set_page_table(self._h, layer, ptr(k), ptr(v), k.size, num_cached)

    def pool(self, layer, which: int) -> _PoolView:
        return _PoolView(lib().or_mgr_pool(self._h, layer, which))

    def pool_array(self, layer, which: int) -> np.ndarray:
        """Writable numpy view [max_blocks][16][Hkv][D] of the layer's K (0) or V (1) pool."""
        Hkv, D, mb = self._shapes[layer]
        base = lib().or_mgr_v_pool(self._h, layer) if which else lib().or_mgr_k_pool(self._h, layer)
        n = mb * PAGE * Hkv * D
        buf = (C.c_uint16 * n).from_address(base)
        return np.ctypeslib.as_array(buf).reshape(mb, PAGE, Hkv, D)

    def paged_attention(self, layer, Q, K, V, groups, scale, causal=True, dtype=BF16):
        """PagedAttentionImpl<CPU>::execute; Q [B,Hq,S,D], K/V [B,Hkv,S,D] bit patterns of
        `dtype` (BF16 or F16)."""
        Q = np.ascontiguousarray(Q, dtype=np.uint16)
        K = np.ascontiguousarray(K, dtype=np.uint16)
        V = np.ascontiguousarray(V, dtype=np.uint16)
        B, Hq, S, D = Q.shape
        out = np.zeros_like(Q)
        rc = lib().or_paged_attention_dt(self._h, layer, ptr(Q), ptr(K), ptr(V), ptr(out), B, Hq, S, D,
                                         K.shape[1], groups, scale, int(causal), dtype)
        return out, rc

    def paged_attend(self, layer, Q, n_kv_heads, groups, scale, causal=True, dtype=BF16):
        Q = np.ascontiguousarray(Q, dtype=np.uint16)
        B, Hq, S, D = Q.shape
        out = np.zeros_like(Q)
        rc = lib().or_paged_attend_dt(self._h, layer, ptr(Q), ptr(out), B, Hq, S, D, n_kv_heads, groups, scale,
                                      int(causal), dtype)
        return out, rc

    def qk_norm_rope_append(self, layer, k_tok, v_tok, gamma_k, eps, cos, sin, start_pos,
                            q_tok=None, gamma_q=None):
        k_tok = np.ascontiguousarray(k_tok, dtype=np.uint16)
        v_tok = np.ascontiguousarray(v_tok, dtype=np.uint16)
        S, Hkv, D = k_tok.shape
        q_out = None
        Hq = 0
        if q_tok is not None:
            q_tok = np.ascontiguousarray(q_tok, dtype=np.uint16)
            Hq = q_tok.shape[1]
            q_out = np.empty((Hq, S, D), dtype=np.uint16)
            gamma_q = np.ascontiguousarray(gamma_q, dtype=np.float32)
        gamma_k = np.ascontiguousarray(gamma_k, dtype=np.float32)
        rope_dim = cos.shape[1] if cos is not None else D
        lib().or_qk_norm_rope_append(self._h, layer, ptr(q_tok), Hq, ptr(gamma_q), ptr(q_out), ptr(k_tok),
                                     ptr(v_tok), Hkv, S, D, ptr(gamma_k), eps, ptr(cos), ptr(sin), rope_dim,
                                     start_pos)
        return q_out
