"""Seeded synthetic inputs (host side).

Counter-based: value i of stream `seed` is a function of (seed, i) only, so any
slice can be regenerated.  Normal samples: h = mix64(seed + i * golden), two
24-bit uniforms u1 in (0,1], u2 in [0,1), z = sqrt(-2 ln u1) cos(2 pi u2) in
fp32, rounded to bf16 with round-to-nearest-even (the bfloat16_t rounding of
include/utils/bfloat16.hpp:18-41).  genllm_fill_normal_bf16 evaluates the same
formula on the GPU (the two may differ in the last fp32 bit before rounding;
tests always hand both sides the same buffer).

Block tables: Fisher-Yates shuffle of [0, pool) driven by the same hash.
Config seeds are 0x5EED0000 + config number.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def config_seed(n: int) -> int:
    return 0x5EED0000 + n


def _mix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        x = (x ^ (x >> np.uint64(30))) * M1
        x = (x ^ (x >> np.uint64(27))) * M2
        return x ^ (x >> np.uint64(31))


def _hash(seed: int, n: int, offset: int = 0) -> np.ndarray:
    i = np.arange(offset, offset + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(np.uint64(seed) + i * GOLDEN)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """RNE to bf16 bit patterns with the bfloat16_t special cases (subnormal ->
    signed zero, NaN -> 0x7F81|sign)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    e = u & np.uint32(0x7F800000)
    with np.errstate(over="ignore"):
        rne = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    sign = (u >> np.uint32(16)) & np.uint32(0x8000)
    special = sign | np.uint32(0x7F80) | ((u & np.uint32(0x7FFFFF)) != 0).astype(np.uint32)
    out = np.where(e == np.uint32(0x7F800000), special, np.where(e == 0, sign, rne))
    return out.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_f32(seed: int, n: int, offset: int = 0) -> np.ndarray:
    h = _hash(seed, n, offset)
    u1 = ((h >> np.uint64(40)) + np.uint64(1)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    u2 = ((h >> np.uint64(16)) & np.uint64(0xFFFFFF)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    r = np.sqrt(np.float32(-2.0) * np.log(u1))
    return (r * np.cos(np.float32(6.2831853071795864) * u2)).astype(np.float32)


def normal_bf16(seed: int, shape, offset: int = 0) -> np.ndarray:
    n = int(np.prod(shape))
    return f32_to_bf16_bits(normal_f32(seed, n, offset)).reshape(shape)


def normal_f16(seed: int, shape, offset: int = 0) -> np.ndarray:
    """Bit patterns of N(0,1) samples rounded to nearest-even fp16 (inputs of
    the fp16 KV-pool tests)."""
    n = int(np.prod(shape))
    return normal_f32(seed, n, offset).astype(np.float16).view(np.uint16).reshape(shape)


def uniform_f32(seed: int, shape, lo: float, hi: float, offset: int = 0) -> np.ndarray:
    n = int(np.prod(shape))
    h = _hash(seed, n, offset)
    u = (h >> np.uint64(40)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    return (np.float32(lo) + u * np.float32(hi - lo)).astype(np.float32).reshape(shape)


def shuffled(seed: int, n: int) -> np.ndarray:
    """Fisher-Yates permutation of [0, n)."""
    perm = np.arange(n, dtype=np.int32)
    h = _hash(seed ^ 0xB10C, n)
    for i in range(n - 1, 0, -1):
        j = int(h[i] % np.uint64(i + 1))
        perm[i], perm[j] = perm[j], perm[i]
    return perm
