"""Seeded synthetic inputs for the benchmark configurations.

SplitMix64 (the generator of crates/llm/candle-llm/src/primitives/sampler.rs:27-52)
feeds a Box-Muller transform in f64; values are rounded once to f32. The same
bytes feed the CPU baseline and the GPU, so both sides see identical inputs.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int, offset: int = 0) -> np.ndarray:
    """Outputs offset .. offset+count-1 of the SplitMix64 stream started at `seed`."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + count + 1, dtype=np.uint64)
        z = np.uint64(seed) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal(seed: int, shape, std: float = 1.0, chunk: int = 1 << 24) -> np.ndarray:
    """N(0, std^2) f32 array of `shape` from SplitMix64(seed) + Box-Muller."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    pairs = (n + 1) // 2
    for p0 in range(0, pairs, chunk):
        p1 = min(pairs, p0 + chunk)
        r = splitmix64(seed, 2 * (p1 - p0), 2 * p0)
        u1 = ((r[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
        u2 = (r[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
        rad = np.sqrt(-2.0 * np.log(u1)) * std
        th = 2.0 * np.pi * u2
        z = np.empty(2 * (p1 - p0), dtype=np.float64)
        z[0::2] = rad * np.cos(th)
        z[1::2] = rad * np.sin(th)
        lo = 2 * p0
        hi = min(n, 2 * p1)
        out[lo:hi] = z[: hi - lo]
    return out.reshape(shape)


def _i64(v: int) -> int:
    """The int64 with the bits of the uint64 v."""
    return v - (1 << 64) if v >= 1 << 63 else v


def _srl(t, k: int):
    """Logical right shift of an int64 tensor read as uint64."""
    return (t >> k) & ((1 << (64 - k)) - 1)


def normal_torch(seed: int, shape, std: float = 1.0, device=None, chunk: int = 1 << 25):
    """normal() computed with torch on `device` (the large synthetic weights of configs 3-5, generated
    where they are used): the same SplitMix64 stream in int64 arithmetic (multiplication wraps mod 2^64,
    shifts are made logical), the same f64 Box-Muller, one rounding to f32. The values equal normal()'s
    wherever the device's f64 log / sqrt / cos / sin round like the host's before that f32 rounding."""
    import torch
    n = int(np.prod(shape))
    out = torch.empty(n, dtype=torch.float32, device=device)
    gold, m1, m2 = _i64(int(_GOLDEN)), _i64(int(_M1)), _i64(int(_M2))
    s = _i64(int(seed) & ((1 << 64) - 1))
    pairs = (n + 1) // 2
    for p0 in range(0, pairs, chunk):
        p1 = min(pairs, p0 + chunk)
        z = torch.arange(2 * p0 + 1, 2 * p1 + 1, dtype=torch.int64, device=device) * gold + s
        z = (z ^ _srl(z, 30)) * m1
        z = (z ^ _srl(z, 27)) * m2
        z = z ^ _srl(z, 31)
        z = _srl(z, 11).to(torch.float64)
        u1 = (z[0::2] + 1.0) * (1.0 / 9007199254740992.0)
        u2 = z[1::2] * (1.0 / 9007199254740992.0)
        del z
        rad = torch.sqrt(-2.0 * torch.log(u1)) * std
        th = (2.0 * np.pi) * u2
        v = torch.stack((rad * torch.cos(th), rad * torch.sin(th)), dim=1).reshape(-1)
        lo, hi = 2 * p0, min(n, 2 * p1)
        out[lo:hi] = v[: hi - lo].to(torch.float32)
    return out.reshape(shape)
