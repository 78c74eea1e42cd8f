"""Python face of the MI355X paged-attention path (over include/genllm_paged.h).

Names and argument meaning follow the reference's operator interface:
``PagedAttentionManager`` (include/core/page_attention.h:52-90) with
``init_layer / reserve_layer / append_kv_pages / reset / is_active / get_layer``,
and the op ``paged_attention`` = ``PagedAttentionImpl<D>::execute``
(src/backend/cpu/attention.cpp:123-216): append this step's K/V, then attend.
Tensors are torch tensors on the GPU (bf16 for activations, fp32 for gammas and
RoPE tables); torch is only the allocator and the stream source here -- every
computation runs in libgenllm_hip.so.
"""
from __future__ import annotations

import contextlib
import ctypes as C

import numpy as np
import torch

from . import _lib
from ._lib import DTYPE_BF16, DTYPE_F16, PAGE, GenllmError, LayerInfo, call, lib


def _stream(stream) -> int | None:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _ptr(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, torch.Tensor):
        if not t.is_cuda:
            raise ValueError("expected a GPU tensor")
        return t.data_ptr()
    return int(t)


class _DeviceArray:
    """Exposes raw device memory to torch through __cuda_array_interface__."""

    def __init__(self, ptr: int, shape, typestr: str):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr, "data": (ptr, False),
                                         "version": 3, "strides": None}


def device_view(ptr: int, shape, dtype=torch.bfloat16) -> torch.Tensor:
    """A torch tensor aliasing library-owned device memory (no copy)."""
    typestr = {torch.bfloat16: "<i2", torch.int32: "<i4", torch.float32: "<f4"}[dtype]
    t = torch.as_tensor(_DeviceArray(ptr, shape, typestr), device="cuda")
    return t.view(torch.bfloat16) if dtype == torch.bfloat16 else t


_hip_rt = None


def _hip():
    """The process's HIP runtime (the one torch loaded), for plain copies."""
    global _hip_rt
    if _hip_rt is None:
        _hip_rt = C.CDLL("libamdhip64.so.7")
        _hip_rt.hipMemcpy.restype = C.c_int
        _hip_rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    return _hip_rt


def copy_to_host(ptr: int, out: np.ndarray) -> np.ndarray:
    """Blocking device -> host copy of out.nbytes bytes at ptr."""
    torch.cuda.synchronize()
    rc = _hip().hipMemcpy(out.ctypes.data, ptr, out.nbytes, 2)
    if rc != 0:
        raise GenllmError(_lib.ERR_HIP, f"hipMemcpy D2H failed ({rc})")
    return out


def copy_to_device(ptr: int, src) -> None:
    """Blocking copy into device memory at ptr from a host array or a GPU tensor."""
    torch.cuda.synchronize()
    if isinstance(src, torch.Tensor):
        rc = _hip().hipMemcpy(ptr, src.data_ptr(), src.numel() * src.element_size(), 3)
    else:
        src = np.ascontiguousarray(src)
        rc = _hip().hipMemcpy(ptr, src.ctypes.data, src.nbytes, 1)
    if rc != 0:
        raise GenllmError(_lib.ERR_HIP, f"hipMemcpy to device failed ({rc})")


class PagedAttentionManager:
    """One device's kv_cache MemoryPool (kv_pool_bytes of HBM) and the paged
    attention state living in it."""

    def __init__(self, kv_pool_bytes: int, device: int = 0):
        h = C.c_void_p()
        call("genllm_kv_create", device, kv_pool_bytes, C.byref(h))
        self._h = h
        self.device = device

    def close(self):
        if getattr(self, "_h", None):
            lib().genllm_kv_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    # -- page_attention.cpp:72-216
    def init_layer(self, layer: int, n_kv_heads: int, head_dim: int, dtype: int = DTYPE_BF16):
        call("genllm_kv_init_layer", self._h, layer, n_kv_heads, head_dim, dtype)

    def reserve_layer(self, layer: int, max_blocks: int):
        call("genllm_kv_reserve_layer", self._h, layer, max_blocks)

    def is_active(self, layer: int) -> bool:
        a = C.c_int32()
        call("genllm_kv_is_active", self._h, layer, C.byref(a))
        return bool(a.value)

    def append_kv_pages(self, layer: int, count: int, stream=None):
        call("genllm_kv_append_pages", self._h, layer, count, _stream(stream))

    def append_kv_from_pos(self, layer: int, k, v, global_pos: int, stream=None):
        """append_kv_from_pos: k, v device head-major [Hkv][count][D], bf16 or
        fp16 as the layer's pools (the library refuses another type)."""
        Hkv, count, D = k.shape
        for t in (k, v):
            assert t.dtype in (torch.bfloat16, torch.float16) and t.dtype == k.dtype and t.is_contiguous()
        dtype = DTYPE_F16 if k.dtype == torch.float16 else DTYPE_BF16
        call("genllm_kv_append_from_pos", self._h, layer, _ptr(k), _ptr(v), Hkv, D, dtype, global_pos, count,
             _stream(stream))

    def reset(self):
        call("genllm_kv_reset", self._h)

    def get_layer(self, layer: int) -> LayerInfo:
        info = LayerInfo()
        call("genllm_kv_layer_info", self._h, layer, C.byref(info))
        return info

    def page_table(self, layer: int):
        n = C.c_int32()
        call("genllm_kv_page_table", self._h, layer, None, None, 0, C.byref(n))
        k = np.empty(n.value, dtype=np.int32)
        v = np.empty(n.value, dtype=np.int32)
        call("genllm_kv_page_table", self._h, layer, k.ctypes.data, v.ctypes.data, n.value, C.byref(n))
        return k, v

    def set_page_table(self, layer: int, k_ids, v_ids, num_cached: int, stream=None):
        k = np.ascontiguousarray(k_ids, dtype=np.int32)
        v = np.ascontiguousarray(v_ids, dtype=np.int32)
        call("genllm_kv_set_page_table", self._h, layer, k.ctypes.data, v.ctypes.data, k.size, num_cached,
             _stream(stream))

    def block_alloc(self, layer: int, which: int) -> int:
        i = C.c_int32()
        call("genllm_kv_block_alloc", self._h, layer, which, C.byref(i))
        return i.value

    def block_free(self, layer: int, which: int, block_id: int):
        call("genllm_kv_block_free", self._h, layer, which, block_id)

    def fragment(self, layer: int, perm_k, perm_v):
        """Hand out every block, then free them so that the next allocations
        return perm[0], perm[1], ... (the free list is LIFO, page_attention.cpp:37-51)."""
        info = self.get_layer(layer)
        for which in (0, 1):
            for _ in range(info.max_blocks):
                self.block_alloc(layer, which)
        for which, perm in ((0, perm_k), (1, perm_v)):
            for b in np.asarray(perm)[::-1]:
                self.block_free(layer, which, int(b))

    def pool(self, layer: int, which: int) -> torch.Tensor:
        """[max_blocks][16][Hkv][D] bf16 view of the K (0) or V (1) pool."""
        i = self.get_layer(layer)
        ptr = i.v_pool if which else i.k_pool
        return device_view(ptr, (i.max_blocks, PAGE, i.n_kv_heads, i.head_dim))

    def device_table(self, layer: int, which: int) -> torch.Tensor:
        i = self.get_layer(layer)
        ptr = i.v_ids if which else i.k_ids
        return device_view(ptr, (i.max_blocks,), torch.int32)

    def read_pool(self, layer: int, which: int) -> np.ndarray:
        """Host copy [max_blocks][16][Hkv][D] (bf16 bits) of the K (0) or V (1) pool."""
        i = self.get_layer(layer)
        out = np.empty((i.max_blocks, PAGE, i.n_kv_heads, i.head_dim), dtype=np.uint16)
        return copy_to_host(i.v_pool if which else i.k_pool, out)

    def write_pool(self, layer: int, which: int, src) -> None:
        """Overwrite the whole K (0) or V (1) pool (host bf16 bits or a GPU tensor)."""
        i = self.get_layer(layer)
        n = i.max_blocks * PAGE * i.n_kv_heads * i.head_dim * 2
        size = src.numel() * src.element_size() if isinstance(src, torch.Tensor) else np.asarray(src).nbytes
        if size != n:
            raise ValueError(f"pool is {n} bytes, source {size}")
        copy_to_device(i.v_pool if which else i.k_pool, src)

    # -- device-position decode (graph-capturable steps)
    def stage_decode(self, layer: int, n_tokens: int, stream=None):
        """Open the pages of the next n_tokens positions (as per-step appends
        would) and hand the layer's position to the device."""
        call("genllm_kv_stage_decode", self._h, layer, n_tokens, _stream(stream))

    def sync_decode(self, layer: int, stream=None) -> int:
        """Read the device position back (waits for `stream`); returns num_cached."""
        n = C.c_int32()
        call("genllm_kv_sync_decode", self._h, layer, _stream(stream), C.byref(n))
        return n.value

    def read_device_table(self, layer: int):
        i = self.get_layer(layer)
        k = copy_to_host(i.k_ids, np.empty(i.num_pages, dtype=np.int32))
        v = copy_to_host(i.v_ids, np.empty(i.num_pages, dtype=np.int32))
        return k, v


# ------------------------------------------------------------------ the op
def paged_attention(mgr: PagedAttentionManager, layer: int, q, k, v, out, n_kv_groups: int, scale: float,
                    causal: bool = True, stream=None):
    """PagedAttentionImpl<HIP>::execute: q/out [B,Hq,S,D], k/v [B,Hkv,S,D] head-major, of the
    layer's element type (bf16 or float16); every batch entry attends the one cache and the
    first entry's k/v rows are appended, as in the reference."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    for t in (q, k, v, out):
        assert t.dtype in (torch.bfloat16, torch.float16) and t.dtype == q.dtype and t.is_contiguous()
    call("genllm_paged_attention", mgr.handle, layer, _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, Hq, S, D, Hkv,
         n_kv_groups, float(scale), int(causal), _stream(stream))


def paged_attention_step(mgr: PagedAttentionManager, layer: int, q, k, v, out, n_kv_groups: int, scale: float,
                         causal: bool = True, stream=None):
    """The op at the layer's device position (a staged layer; capturable)."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    for t in (q, k, v, out):
        assert t.dtype in (torch.bfloat16, torch.float16) and t.dtype == q.dtype and t.is_contiguous()
    call("genllm_paged_attention_step", mgr.handle, layer, _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, Hq, S, D, Hkv,
         n_kv_groups, float(scale), int(causal), _stream(stream))


def apply_rope_step(mgr: PagedAttentionManager, layer: int, out, x, cos, sin, stream=None):
    """apply_rope with start_pos = the staged layer's device position (capturable)."""
    H, S, D = x.shape
    call("genllm_apply_rope_step", mgr.handle, layer, _ptr(out), _ptr(x), _ptr(cos), _ptr(sin), H, S, D,
         int(cos.shape[-1]), int(cos.shape[0]), _stream(stream))


def qk_norm_rope_append(mgr: PagedAttentionManager, layer: int, k, v, gamma_k, eps: float, cos, sin,
                        rope_pos0: int, q=None, gamma_q=None, q_out=None, stream=None):
    """Fused per-head RMSNorm -> RoPE -> page scatter.  k, v: token-major
    [S][Hkv][D]; q (optional) token-major [S][Hq][D]; q_out head-major [Hq][S][D].
    cos/sin [max_seq][rope_dim]: the first rope_dim dims rotate (all of them
    when rope_dim == D)."""
    S, Hkv, D = k.shape
    rope_dim = cos.shape[-1] if cos is not None else D
    Hq = q.shape[1] if q is not None else 0
    qs = (q.stride(0), q.stride(1)) if q is not None else (0, 0)
    qos = (q_out.stride(1), q_out.stride(0)) if q_out is not None else (0, 0)
    call("genllm_qk_norm_rope_append", mgr.handle, layer, S, _ptr(k), k.stride(0), k.stride(1), _ptr(v),
         v.stride(0), v.stride(1), _ptr(gamma_k), _ptr(q), qs[0], qs[1], Hq, _ptr(gamma_q), _ptr(q_out), qos[0],
         qos[1], float(eps), _ptr(cos), _ptr(sin), int(rope_dim), int(rope_pos0), _stream(stream))


# ------------------------------------------------------- stateless kernels
def rms_norm(out, x, w, eps: float, stream=None):
    hidden = w.numel()
    call("genllm_rms_norm", _ptr(out), _ptr(x), _ptr(w), x.numel() // hidden, hidden, float(eps), _stream(stream))


def apply_rope(out, x, cos, sin, start_pos: int, stream=None):
    """x head-major [H][S][D]; cos/sin [max_seq][rope_dim] (rope_dim <= D
    leading dims rotate)."""
    H, S, D = x.shape
    call("genllm_apply_rope", _ptr(out), _ptr(x), _ptr(cos), _ptr(sin), H, S, D, int(cos.shape[-1]),
         int(start_pos), _stream(stream))


def rope_cache(theta: float, head_dim: int, max_seq: int):
    """RopeCacheImpl: host fp32 tables [max_seq][head_dim] (cos, sin)."""
    cos = np.empty((max_seq, head_dim), dtype=np.float32)
    sin = np.empty((max_seq, head_dim), dtype=np.float32)
    call("genllm_rope_cache", cos.ctypes.data, float(theta), head_dim, max_seq, 1)
    call("genllm_rope_cache", sin.ctypes.data, float(theta), head_dim, max_seq, 0)
    return cos, sin


def kv_scatter(k, v, k_pool, v_pool, k_ids, v_ids, pos0: int, stream=None):
    """k, v token-major [S][Hkv][D]; pools [blocks][16][Hkv][D]."""
    S, Hkv, D = k.shape
    call("genllm_kv_scatter", _ptr(k), k.stride(0), k.stride(1), _ptr(v), v.stride(0), v.stride(1), _ptr(k_pool),
         _ptr(v_pool), _ptr(k_ids), _ptr(v_ids), pos0, S, Hkv, D, _stream(stream))


def decode_workspace_bytes(n_q_heads: int, n_kv_heads: int, seq_len: int, head_dim: int, max_pages: int) -> int:
    return lib().genllm_paged_decode_workspace_bytes(n_q_heads, n_kv_heads, seq_len, head_dim, max_pages)


def _attn_args(q, out, q_layout):
    # q/out given head-major [Hq][S][D] ("head") or token-major [S][Hq][D] ("token")
    if q_layout == "head":
        Hq, S, D = q.shape
        return Hq, S, D, (q.stride(0), q.stride(1)), (out.stride(0), out.stride(1))
    S, Hq, D = q.shape
    return Hq, S, D, (q.stride(1), q.stride(0)), (out.stride(1), out.stride(0))


def paged_decode(q, out, k_pool, v_pool, k_ids, v_ids, n_pages: int, n_cached: int, n_kv_heads: int,
                 scale: float, workspace=None, causal: bool = True, q_layout: str = "head", stream=None):
    """genllm_paged_decode.  workspace: a device buffer of at least
    decode_workspace_bytes(...) bytes, zero-filled before its first use (its
    arrival counters must start at zero; every launch leaves them at zero);
    None allocates a zero-filled one for this call."""
    Hq, S, D, qs, os_ = _attn_args(q, out, q_layout)
    if workspace is None:
        workspace = torch.zeros(decode_workspace_bytes(Hq, n_kv_heads, S, D, n_pages), dtype=torch.uint8,
                                device=q.device)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    call("genllm_paged_decode", _ptr(q), qs[0], qs[1], _ptr(out), os_[0], os_[1], _ptr(k_pool), _ptr(v_pool),
         _ptr(k_ids), _ptr(v_ids), n_pages, n_cached, S, Hq, n_kv_heads, D, float(scale), int(causal),
         _ptr(workspace), ws_bytes, _stream(stream))


DECODE_MERGE = {"kernel": 0, "fused": 1}


def decode_tuning(pages_per_split: int = 0, merge: str = "kernel", heads: int = 0):
    """genllm_decode_tuning: process-wide decode split size (0 = automatic),
    merge form ("kernel" or "fused") and kv heads per split workgroup (0 =
    automatic, 1 or 4) for later decode calls."""
    call("genllm_decode_tuning", int(pages_per_split), DECODE_MERGE[merge], int(heads))


@contextlib.contextmanager
def decode_tuned(pages_per_split: int = 0, merge: str = "kernel", heads: int = 0):
    """decode_tuning for the duration of a with-block, then the defaults."""
    decode_tuning(pages_per_split, merge, heads)
    try:
        yield
    finally:
        decode_tuning(0, "kernel", 0)


def paged_decode_noalloc(q, out, k_pool, v_pool, k_ids, v_ids, n_pages: int, n_cached: int, n_kv_heads: int,
                         scale: float, causal: bool = True, q_layout: str = "head", stream=None):
    """paged_decode without a workspace: the library's static per-GPU scratch
    holds the split partials (genllm_paged_decode_noalloc)."""
    Hq, S, D, qs, os_ = _attn_args(q, out, q_layout)
    call("genllm_paged_decode_noalloc", _ptr(q), qs[0], qs[1], _ptr(out), os_[0], os_[1], _ptr(k_pool), _ptr(v_pool),
         _ptr(k_ids), _ptr(v_ids), n_pages, n_cached, S, Hq, n_kv_heads, D, float(scale), int(causal),
         _stream(stream))


def paged_prefill(q, out, k_pool, v_pool, k_ids, v_ids, n_pages: int, n_cached: int, n_kv_heads: int,
                  scale: float, causal: bool = True, q_layout: str = "head", stream=None):
    Hq, S, D, qs, os_ = _attn_args(q, out, q_layout)
    call("genllm_paged_prefill", _ptr(q), qs[0], qs[1], _ptr(out), os_[0], os_[1], _ptr(k_pool), _ptr(v_pool),
         _ptr(k_ids), _ptr(v_ids), n_pages, n_cached, S, Hq, n_kv_heads, D, float(scale), int(causal),
         _stream(stream))


def flash_attention(q, k, v, out, n_kv_groups: int, scale: float, causal: bool = True, stream=None):
    """FlashAttentionImpl (attention.cpp:39-121) on contiguous bf16 tensors:
    q, out [B, Hq, S, D]; k, v [B, Hkv, S, D]; no KV cache involved."""
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    for t, shape in ((q, (B, Hq, S, D)), (out, (B, Hq, S, D)), (k, (B, Hkv, S, D)), (v, (B, Hkv, S, D))):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or tuple(t.shape) != shape:
            raise ValueError(f"flash_attention: expected contiguous bf16 {shape}, got {tuple(t.shape)} {t.dtype}")
    call("genllm_flash_attention", _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, Hq, S, Hkv, D, n_kv_groups,
         float(scale), int(causal), _stream(stream))


def linear_workspace_bytes(rows: int, common: int, cols: int) -> int:
    return lib().genllm_linear_workspace_bytes(rows, common, cols)


def linear(x, w, out, bias=None, workspace=None, stream=None):
    """LinearImpl (linear.cpp:46-122, linear.cu:72-126) on contiguous bf16
    tensors: x [rows, common], w [cols, common], bias [cols] or None,
    out [rows, cols]; workspace: a device buffer of at least
    linear_workspace_bytes(rows, common, cols) bytes when that is non-zero."""
    rows, common = x.shape
    cols = w.shape[0]
    for t, shape in ((x, (rows, common)), (w, (cols, common)), (out, (rows, cols))):
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or tuple(t.shape) != shape:
            raise ValueError(f"linear: expected contiguous bf16 {shape}, got {tuple(t.shape)} {t.dtype}")
    if bias is not None and (bias.dtype != torch.bfloat16 or tuple(bias.shape) != (cols,)):
        raise ValueError("linear: bias must be bf16 [cols]")
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    call("genllm_linear", _ptr(x), _ptr(w), _ptr(bias), _ptr(out), rows, common, cols, _ptr(workspace), ws_bytes,
         _stream(stream))


def fill_normal_bf16(t: torch.Tensor, seed: int, offset: int = 0, stream=None):
    call("genllm_fill_normal_bf16", _ptr(t), t.numel(), seed, offset, _stream(stream))


def fill_normal_f16(t: torch.Tensor, seed: int, offset: int = 0, stream=None):
    call("genllm_fill_normal_f16", _ptr(t), t.numel(), seed, offset, _stream(stream))


def selftest_mfma(a, b, c, stream=None):
    """a [16][k], b [k][16] bf16 (k = 32 or 16) -> c [16][16] fp32 via one MFMA."""
    call("genllm_selftest_mfma", a.shape[1], _ptr(a), _ptr(b), _ptr(c), _stream(stream))


# ------------------------------------------------------------- conversions
def to_device_bf16(bits: np.ndarray) -> torch.Tensor:
    """bf16 bit patterns (uint16 numpy) -> GPU bf16 tensor."""
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16).cuda()


def to_device_f16(bits: np.ndarray) -> torch.Tensor:
    """fp16 bit patterns (uint16 numpy) -> GPU float16 tensor."""
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.float16).cuda()


def to_host_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


__all__ = [
    "PagedAttentionManager", "paged_attention", "qk_norm_rope_append", "rms_norm", "apply_rope", "rope_cache",
    "kv_scatter", "paged_decode", "paged_decode_noalloc", "paged_prefill", "flash_attention", "decode_workspace_bytes", "fill_normal_bf16",
    "fill_normal_f16",
    "selftest_mfma", "device_view", "to_device_bf16", "to_device_f16", "to_host_bits", "GenllmError", "PAGE",
    "DTYPE_BF16", "DTYPE_F16",
]
