"""Seeded synthetic inputs for benchmarks and tests.

The reference ships no datasets or fixtures for its hot path, so inputs are
drawn from a deterministic host generator: SplitMix64 (Steele, Lea and
Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014) for
uniform draws, Box-Muller for normal ones, and Xavier-uniform bounds
U(+-sqrt(6 / (fan_in + fan_out))) for weights (the initialisation of
InitType::Xavier, runtime.rs:6-22).

Draw i of a stream seeded with s is mix(s + (i + 1) * 0x9E3779B97F4A7C15)
(mod 2^64), so every draw is computed independently and the whole array is
vectorised in numpy.  A uniform value takes the top 24 bits of a draw; a
normal pair takes the top 53 bits of two consecutive draws.  The values are
a pure function of (shape, seed, parameters).
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 21


def _draws(seed: int, start: int, count: int) -> np.ndarray:
    """SplitMix64 outputs start .. start + count - 1 of the stream `seed`."""
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform(shape, seed: int, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    """float32 values lo + (hi - lo) * u, u = k / 2^24 for a 24-bit draw k."""
    out = np.empty(shape, dtype=np.float32)
    flat = out.reshape(-1)
    for s in range(0, flat.size, _CHUNK):
        n = min(_CHUNK, flat.size - s)
        u = (_draws(seed, s, n) >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)
        flat[s:s + n] = (float(lo) + (float(hi) - float(lo)) * u).astype(np.float32)
    return out


def normal(shape, seed: int, mu: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    """float32 N(mu, sigma^2) by Box-Muller: element 2k is rad cos(2 pi u2)
    and element 2k + 1 is rad sin(2 pi u2) of the pair (u1, u2) taken from
    draws 2k and 2k + 1, rad = sqrt(-2 ln u1), u1 in (0, 1]."""
    out = np.empty(shape, dtype=np.float32)
    flat = out.reshape(-1)
    pairs = (flat.size + 1) // 2
    step = _CHUNK // 2
    for p in range(0, pairs, step):
        m = min(step, pairs - p)
        d = _draws(seed, 2 * p, 2 * m)
        u1 = ((d[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740993.0)
        u2 = (d[1::2] >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
        rad = np.sqrt(-2.0 * np.log(u1))
        ang = 2.0 * np.pi * u2
        pair = np.empty(2 * m, dtype=np.float64)
        pair[0::2] = mu + sigma * rad * np.cos(ang)
        pair[1::2] = mu + sigma * rad * np.sin(ang)
        e = min(2 * (p + m), flat.size)
        flat[2 * p:e] = pair[:e - 2 * p].astype(np.float32)
    return out


def xavier(fan_in: int, fan_out: int, seed: int) -> np.ndarray:
    """Xavier-uniform U(+-sqrt(6 / (fan_in + fan_out))) of shape [fan_in, fan_out]."""
    lim = float(np.sqrt(6.0 / (fan_in + fan_out)))
    return uniform((fan_in, fan_out), seed, -lim, lim)
