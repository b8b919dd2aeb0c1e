"""Seeded synthetic inputs: SplitMix64 -> uniform -> Box-Muller normal.

Counter-based, so any element can be regenerated independently: output i of seed s is
mix(s + (i + 1) * 0x9E3779B97F4A7C15) with SplitMix64's finaliser (Steele, Lea, Flood 2014).
Normals pair consecutive uniforms (u1, u2): r = sqrt(-2 ln u1), z0 = r cos(2 pi u2),
z1 = r sin(2 pi u2). Computed in float64, returned as float32.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n consecutive SplitMix64 outputs of `seed`, starting at output index `offset`."""
    idx = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform01(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Uniform float64 in the open interval (0, 1) from the top 53 bits."""
    bits = splitmix64(seed, n, offset) >> np.uint64(11)
    return (bits.astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(seed: int, shape, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """float32 array of N(mean, std^2) values of the given shape."""
    n = int(np.prod(shape)) if np.ndim(shape) else int(shape)
    pairs = (n + 1) // 2
    out = np.empty(pairs * 2, dtype=np.float64)
    chunk = 1 << 22
    for p0 in range(0, pairs, chunk):
        p1 = min(pairs, p0 + chunk)
        u = uniform01(seed, 2 * (p1 - p0), offset=2 * p0)
        u1, u2 = u[0::2], u[1::2]
        r = np.sqrt(-2.0 * np.log(u1))
        out[2 * p0:2 * p1:2] = r * np.cos(2.0 * np.pi * u2)
        out[2 * p0 + 1:2 * p1:2] = r * np.sin(2.0 * np.pi * u2)
    vals = out[:n] * std + mean
    return vals.astype(np.float32).reshape(shape)


def normal_at(seed: int, index, std: float = 1.0) -> np.ndarray:
    """float32 values of normal(seed, ...) at the given flat element indices (any shape), without
    generating the rest: element i is the cos (i even) or sin (i odd) half of pair i // 2."""
    idx = np.asarray(index, dtype=np.int64)
    pair = idx // 2
    u1 = _uniform_at(seed, 2 * pair)
    u2 = _uniform_at(seed, 2 * pair + 1)
    r = np.sqrt(-2.0 * np.log(u1))
    ang = 2.0 * np.pi * u2
    z = np.where(idx % 2 == 0, r * np.cos(ang), r * np.sin(ang))
    return (z * std + 0.0).astype(np.float32)


def _uniform_at(seed: int, i) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + (np.asarray(i, dtype=np.uint64) + np.uint64(1)) * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal_tensor(seed: int, shape, std: float = 1.0, precision=None, ctx=None):
    """Device tensor holding normal(seed, shape, std) (BF16: rounded to nearest even), generated on
    the GPU by it_fill_normal -- the same stream as `normal`, for sizes the host makes slowly."""
    from ctypes import c_void_p

    from .errors import check
    from .tensor import Precision, Tensor

    prec = Precision.FP32 if precision is None else Precision(precision)
    t = Tensor.empty(list(shape), prec, ctx)
    if t.numel():
        check(t.ctx.lib.it_fill_normal(t.ctx.handle, int(prec), seed & 0xFFFFFFFFFFFFFFFF, 0, t.numel(),
                                       float(std), c_void_p(t.ptr)), "fill_normal")
    return t


def tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    """n token ids uniform over [0, vocab) (uint32), by multiply-shift of the 64-bit outputs."""
    bits = splitmix64(seed, n) >> np.uint64(32)
    return ((bits * np.uint64(vocab)) >> np.uint64(32)).astype(np.uint32)


def small_ints(seed: int, shape, lo: int, hi: int) -> np.ndarray:
    """float32 integers uniform in [lo, hi] (exact in FP32 and BF16 for small ranges)."""
    n = int(np.prod(shape))
    bits = splitmix64(seed, n) >> np.uint64(32)
    span = np.uint64(hi - lo + 1)
    vals = ((bits * span) >> np.uint64(32)).astype(np.int64) + lo
    return vals.astype(np.float32).reshape(shape)
