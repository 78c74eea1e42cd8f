"""ctypes binding of include/genllm_paged.h (genllm_amd/libgenllm_hip.so).

torch is imported before the library is opened: torch ships its own HIP
runtime under the same soname (libamdhip64.so.7), and loading it first makes the
dynamic linker bind this library to that one runtime instead of a second copy.

There is no fallback: if the library is missing the import of any product entry
point raises, naming the build step.
"""
from __future__ import annotations

import ctypes as C
import os

try:  # the single HIP runtime of the process comes with torch
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - torch is part of the image
    torch = None

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgenllm_hip.so")

OK = 0
ERR_INVALID = 1
ERR_UNSUPPORTED = 2
ERR_NO_MEMORY = 3
ERR_POOL_FULL = 4
ERR_HIP = 5
_NAMES = {1: "INVALID", 2: "UNSUPPORTED", 3: "NO_MEMORY", 4: "POOL_FULL", 5: "HIP"}

PAGE = 16
DTYPE_BF16 = 30
DTYPE_F16 = 1


class GenllmError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"genllm error {code} ({_NAMES.get(code, '?')}): {msg}")
        self.code = code


class LayerInfo(C.Structure):
    _fields_ = [
        ("active", C.c_int32),
        ("num_cached", C.c_int32),
        ("num_pages", C.c_int32),
        ("n_kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("dtype", C.c_int32),
        ("max_blocks", C.c_int32),
        ("k_num_blocks", C.c_int32),
        ("k_num_free", C.c_int32),
        ("v_num_blocks", C.c_int32),
        ("v_num_free", C.c_int32),
        ("k_pool", C.c_void_p),
        ("v_pool", C.c_void_p),
        ("k_ids", C.c_void_p),
        ("v_ids", C.c_void_p),
        ("block_bytes", C.c_size_t),
    ]


_P = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_u64 = C.c_uint64
_f = C.c_float
_sz = C.c_size_t
_int = C.c_int

# name -> (restype, argtypes); every symbol of include/genllm_paged.h
SIGNATURES = {
    "genllm_last_error": (C.c_char_p, []),
    "genllm_kv_create": (_int, [_i32, _sz, C.POINTER(_P)]),
    "genllm_kv_destroy": (_int, [_P]),
    "genllm_kv_init_layer": (_int, [_P, _i32, _i32, _i32, _i32]),
    "genllm_kv_reserve_layer": (_int, [_P, _i32, _i32]),
    "genllm_kv_is_active": (_int, [_P, _i32, C.POINTER(_i32)]),
    "genllm_kv_append_pages": (_int, [_P, _i32, _i32, _P]),
    "genllm_kv_reset": (_int, [_P]),
    "genllm_kv_layer_info": (_int, [_P, _i32, C.POINTER(LayerInfo)]),
    "genllm_kv_page_table": (_int, [_P, _i32, _P, _P, _i32, C.POINTER(_i32)]),
    "genllm_kv_set_page_table": (_int, [_P, _i32, _P, _P, _i32, _i32, _P]),
    "genllm_kv_block_alloc": (_int, [_P, _i32, _i32, C.POINTER(_i32)]),
    "genllm_kv_block_free": (_int, [_P, _i32, _i32, _i32]),
    "genllm_paged_attention": (_int, [_P, _i32, _P, _P, _P, _P, _i32, _i32, _i32, _i32, _i32, _i32, _f, _i32, _P]),
    "genllm_kv_append_from_pos": (_int, [_P, _i32, _P, _P, _i32, _i32, _i32, _i32, _i32, _P]),
    "genllm_kv_stage_decode": (_int, [_P, _i32, _i32, _P]),
    "genllm_kv_sync_decode": (_int, [_P, _i32, _P, _P]),
    "genllm_paged_attention_step": (_int, [_P, _i32, _P, _P, _P, _P, _i32, _i32, _i32, _i32, _i32, _i32, _f, _i32,
                                           _P]),
    "genllm_apply_rope_step": (_int, [_P, _i32, _P, _P, _P, _P, _i32, _i32, _i32, _i32, _i32, _P]),
    "genllm_qk_norm_rope_append": (_int, [_P, _i32, _i32, _P, _i64, _i64, _P, _i64, _i64, _P, _P, _i64, _i64,
                                          _i32, _P, _P, _i64, _i64, _f, _P, _P, _i32, _i64, _P]),
    "genllm_rms_norm": (_int, [_P, _P, _P, _i64, _i32, _f, _P]),
    "genllm_apply_rope": (_int, [_P, _P, _P, _P, _i32, _i32, _i32, _i32, _i64, _P]),
    "genllm_rope_cache": (_int, [_P, _f, _i32, _i32, _i32]),
    "genllm_kv_scatter": (_int, [_P, _i64, _i64, _P, _i64, _i64, _P, _P, _P, _P, _i32, _i32, _i32, _i32, _P]),
    "genllm_paged_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "genllm_decode_tuning": (_int, [_i32, _i32, _i32]),
    "genllm_paged_decode": (_int, [_P, _i64, _i64, _P, _i64, _i64, _P, _P, _P, _P, _i32, _i32, _i32, _i32, _i32,
                                   _i32, _f, _i32, _P, _sz, _P]),
    "genllm_paged_decode_noalloc": (_int, [_P, _i64, _i64, _P, _i64, _i64, _P, _P, _P, _P, _i32, _i32, _i32, _i32,
                                           _i32, _i32, _f, _i32, _P]),
    "genllm_paged_prefill": (_int, [_P, _i64, _i64, _P, _i64, _i64, _P, _P, _P, _P, _i32, _i32, _i32, _i32, _i32,
                                    _i32, _f, _i32, _P]),
    "genllm_flash_attention": (_int, [_P, _P, _P, _P, _i32, _i32, _i32, _i32, _i32, _i32, _f, _i32, _P]),
    "genllm_linear_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "genllm_linear": (_int, [_P, _P, _P, _P, _i64, _i64, _i64, _P, _sz, _P]),
    "genllm_fill_normal_bf16": (_int, [_P, _sz, _u64, _u64, _P]),
    "genllm_fill_normal_f16": (_int, [_P, _sz, _u64, _u64, _P]),
    "genllm_selftest_mfma": (_int, [_i32, _P, _P, _P, _P]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (make -C genllm_amd/csrc)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int):
    if rc != OK:
        raise GenllmError(rc, lib().genllm_last_error().decode())
    return rc


def call(name: str, *args):
    return check(getattr(lib(), name)(*args))
