"""CPU-side checks of the C ABI: libgenllm_hip.so loads without a GPU, exports
every function include/genllm_paged.h declares, and its host-only entry points
(RoPE table, workspace sizing, error reporting) behave."""
import ctypes as C
import os
import re
import subprocess

import numpy as np

from genllm_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "genllm_paged.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(genllm_[a-z0-9_]+)\s*\(", text)))


def test_header_functions_all_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 20
    L = _lib.lib()
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.SIGNATURES), set(names) ^ set(_lib.SIGNATURES)
    dyn = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (genllm_\w+)", dyn))
    assert set(names) <= exported


def test_rope_cache_matches_oracle(orc):
    for D, S, theta in [(128, 4100, 1e6), (64, 300, 1e4)]:
        cos = np.empty((S, D), np.float32)
        sin = np.empty((S, D), np.float32)
        _lib.call("genllm_rope_cache", cos.ctypes.data, theta, D, S, 1)
        _lib.call("genllm_rope_cache", sin.ctypes.data, theta, D, S, 0)
        oc, os_ = orc.rope_cache(theta, D, S)
        assert np.array_equal(cos, oc) and np.array_equal(sin, os_)


def test_errors_are_reported():
    L = _lib.lib()
    rc = L.genllm_rope_cache(None, 1e6, 128, 4, 1)
    assert rc == _lib.ERR_INVALID
    assert b"rope_cache" in L.genllm_last_error()
    try:
        _lib.call("genllm_rope_cache", None, 1e6, 128, 4, 1)
    except _lib.GenllmError as e:
        assert e.code == _lib.ERR_INVALID
    else:
        raise AssertionError("no error raised")


def test_decode_workspace_closed_form():
    L = _lib.lib()
    # 1 KiB of per-kv-head arrival counters, then partials: Hkv x splits x rows
    # (= groups * seq_len) x (D+2) fp32, splits <= min(pages, 256)
    for Hq, Hkv, S, D, pages in [(32, 8, 1, 128, 513), (16, 8, 1, 128, 64), (32, 8, 3, 128, 10)]:
        rows = Hq // Hkv * S
        want = 1024 + Hkv * min(pages, 256) * rows * (D + 2) * 4
        assert L.genllm_paged_decode_workspace_bytes(Hq, Hkv, S, D, pages) == want
    assert L.genllm_paged_decode_workspace_bytes(0, 8, 1, 128, 4) == 0


def test_attention_argument_checks():
    """The stateless attention entry points (genllm_paged_decode, _noalloc,
    _prefill) reject bad arguments with their error code and message before
    any device work: the addresses below are aligned placeholders that no
    check lets through to a launch."""
    L = _lib.lib()
    base = dict(q=0x10000, qh=128, qt=32 * 128, out=0x20000, oh=128, ot=32 * 128, kp=0x30000, vp=0x40000,
                kid=0x50000, vid=0x60000, n_pages=513, n_cached=8193, S=1, Hq=32, Hkv=8, D=128, scale=0.088)

    def args(**kw):
        a = dict(base, **kw)
        return [a["q"], a["qh"], a["qt"], a["out"], a["oh"], a["ot"], a["kp"], a["vp"], a["kid"], a["vid"],
                a["n_pages"], a["n_cached"], a["S"], a["Hq"], a["Hkv"], a["D"], a["scale"], 1]

    cases = [
        (dict(q=None), _lib.ERR_INVALID, b"null pointer"),
        (dict(vid=None), _lib.ERR_INVALID, b"null pointer"),
        (dict(D=96), _lib.ERR_UNSUPPORTED, b"head_dim 128 or 256"),
        (dict(Hq=12), _lib.ERR_INVALID, b"multiple of n_kv_heads"),
        (dict(Hkv=0), _lib.ERR_INVALID, b"multiple of n_kv_heads"),
        (dict(S=0), _lib.ERR_INVALID, b"seq_len <= n_cached"),
        (dict(S=9000), _lib.ERR_INVALID, b"seq_len <= n_cached"),
        (dict(n_pages=10), _lib.ERR_INVALID, b"16 * n_pages"),
        (dict(scale=-1.0), _lib.ERR_INVALID, b"scale must be finite"),
        (dict(scale=float("inf")), _lib.ERR_INVALID, b"scale must be finite"),
        (dict(scale=float("nan")), _lib.ERR_INVALID, b"scale must be finite"),
        (dict(q=0x10008), _lib.ERR_INVALID, b"16-byte aligned"),
        (dict(kp=0x30004), _lib.ERR_INVALID, b"16-byte aligned"),
        (dict(qh=132), _lib.ERR_INVALID, b"16-byte aligned"),
    ]
    for kw, code, msg in cases:
        a = args(**kw)
        for name, extra in (("genllm_paged_decode", [None, 0, None]), ("genllm_paged_decode_noalloc", [None]),
                            ("genllm_paged_prefill", [None])):
            rc = getattr(L, name)(*a, *extra)
            assert rc == code, (name, kw, rc)
            assert msg in L.genllm_last_error(), (name, kw, L.genllm_last_error())
    # more than 16 rows per kv head: the decode forms refuse (prefill takes them)
    a = args(S=5, Hkv=8)  # 4 q heads per kv head x 5 queries = 20 rows
    assert L.genllm_paged_decode(*a, None, 0, None) == _lib.ERR_INVALID
    assert b"<= 16" in L.genllm_last_error()
    assert L.genllm_paged_decode_noalloc(*a, None) == _lib.ERR_INVALID
    assert b"<= 16" in L.genllm_last_error()
