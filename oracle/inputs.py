"""Version-stable synthetic KV values (test infrastructure only).

A counter-based generator, so the same (seed, index) gives the same value on
any machine and numpy version: splitmix64 of (seed, counter) yields two
uniform doubles, Box-Muller turns them into one N(0,1) double, which is
rounded to float32 and then round-to-nearest-even to fp16 or bf16.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(x: np.ndarray) -> np.ndarray:
    """splitmix64 finaliser (Steele, Lea, Flood 2014) over uint64 arrays."""
    with np.errstate(over="ignore"):
        z = x + _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normal_f32(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n standard normal float32 values for counters offset .. offset+n-1."""
    ctr = np.arange(offset, offset + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        base = np.uint64(seed) * np.uint64(0xD1B54A32D192ED03)
        a = splitmix64(base ^ (ctr * np.uint64(2)))
        b = splitmix64(base ^ (ctr * np.uint64(2) + np.uint64(1)))
    # 53-bit uniforms in (0, 1] and [0, 1)
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)
    u2 = (b >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return z.astype(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16, returned as uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounding = ((u >> np.uint32(16)) & np.uint32(1)) + np.uint32(0x7FFF)
    with np.errstate(over="ignore"):
        r = (u + rounding) >> np.uint32(16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def normal_bits(seed: int, n: int, dtype: str, offset: int = 0) -> np.ndarray:
    """Raw 16-bit patterns of n N(0,1) values in 'fp16' or 'bf16'."""
    z = normal_f32(seed, n, offset)
    if dtype == "fp16":
        return z.astype(np.float16).view(np.uint16)
    if dtype == "bf16":
        return f32_to_bf16_bits(z)
    raise ValueError(f"unsupported dtype {dtype!r}")


def distinct_ids(seed: int, count: int, universe: int) -> np.ndarray:
    """`count` distinct ids from [0, universe), order randomised, seeded by
    splitmix64 keys (argsort of hashed counters = a random permutation)."""
    if count > universe:
        raise ValueError("more ids than the universe holds")
    keys = splitmix64(np.arange(universe, dtype=np.uint64) ^ splitmix64(np.full(1, seed, np.uint64)))
    return np.argsort(keys, kind="stable")[:count].astype(np.int64)


def run_ids(seed: int, count: int, universe: int, run: int) -> np.ndarray:
    """`count` distinct ids made of contiguous runs of length `run` with
    random, non-overlapping run starts (the fragmentation sweep)."""
    if count % run != 0 or universe % run != 0:
        raise ValueError("run must divide count and universe")
    slots = distinct_ids(seed, count // run, universe // run)
    return (slots[:, None] * run + np.arange(run, dtype=np.int64)[None, :]).reshape(-1)
