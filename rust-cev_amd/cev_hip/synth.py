"""Seeded synthetic inputs: a counter-based splitmix64 stream per tensor,
uniform doubles from its top 53 bits, normals by Box-Muller, then f32 (and
round-to-nearest-even bf16 for bf16 configs).

`normal(seed, stream, n)` depends only on (seed, stream, index), so a slice
of a tensor can be regenerated without the rest.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _key(seed: int, stream: int) -> np.uint64:
    with np.errstate(over="ignore"):
        k = _mix(np.array([np.uint64(seed) + _GOLDEN], np.uint64))[0]
        k = _mix(np.array([k ^ np.uint64(stream & 0xFFFFFFFFFFFFFFFF)], np.uint64))[0]
    return k


def _u64(key: np.uint64, idx: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return _mix(key + (idx.astype(np.uint64) + np.uint64(1)) * _GOLDEN)


def uniform(seed: int, stream: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    """n doubles in [lo, hi)."""
    key = _key(seed, stream)
    out = np.empty(n, np.float64)
    for s in range(0, n, _CHUNK):
        idx = np.arange(s, min(n, s + _CHUNK), dtype=np.uint64)
        out[s:s + idx.size] = (_u64(key, idx) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return lo + (hi - lo) * out


def normal(seed: int, stream: int, n: int) -> np.ndarray:
    """n standard normals (f64) by Box-Muller on consecutive uniform pairs:
    element 2j is r cos(a) and element 2j+1 is r sin(a) of pair j."""
    key = _key(seed, stream)
    out = np.empty(n, np.float64)
    for s in range(0, n, _CHUNK):  # _CHUNK is even, so every chunk starts on a pair
        e = min(n, s + _CHUNK)
        u = (_u64(key, np.arange(s, e + (e - s) % 2, dtype=np.uint64)) >> np.uint64(11)).astype(np.float64)
        u *= 1.0 / 9007199254740992.0
        r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
        ang = 2.0 * np.pi * u[1::2]
        both = np.empty(u.size, np.float64)
        both[0::2] = r * np.cos(ang)
        both[1::2] = r * np.sin(ang)
        out[s:e] = both[:e - s]
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    """f32 array holding the round-to-nearest-even bf16 value of each element."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    # no wrap-around for non-NaN values: |bits| <= 0x7F800000 before the sign
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    r = np.where(nan, (u | np.uint32(0x00400000)) & np.uint32(0xFFFF0000), r)
    return r.view(np.float32).reshape(x.shape)


def tensor(seed: int, stream: int, shape, bf16: bool, scale: float = 1.0, offset: float = 0.0) -> np.ndarray:
    """offset + scale * N(0,1) of `shape` as f32 (bf16-exact when bf16)."""
    n = int(np.prod(shape)) if len(shape) else 1
    x = (offset + scale * normal(seed, stream, n)).astype(np.float32).reshape(shape)
    return round_bf16(x) if bf16 else x
