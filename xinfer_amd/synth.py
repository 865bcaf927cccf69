"""Seeded synthetic inputs for the INT4-G128-SYM path (numpy, host side).

Generator: SplitMix64 (Steele, Lea, Flood 2014) over a counter, one
independent stream per tensor; normals by Box-Muller.  Independent of any
C++ standard library, so the same seed gives the same bytes everywhere.

* weights: every nibble uniform on [-8, 7]: the packed bytes ARE the raw
  little-endian generator output (16 independent uniform nibbles per word),
  which is the two's-complement packing of tools/convert/qwen3_8_27b/
  convert.py:107-111.
* scales: fp16(|N(0, sigma)| / 7), one per (row, 128-k group).
* activations: fp16(N(0, 1)).
"""
from __future__ import annotations

import numpy as np

_M64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15

STREAM_W, STREAM_S, STREAM_X, STREAM_W2, STREAM_S2, STREAM_MISC = 1, 2, 3, 4, 5, 6


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _mix_int(z: int) -> int:
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def splitmix64(seed: int, stream: int, n: int, offset: int = 0) -> np.ndarray:
    """n outputs (uint64) of the SplitMix64 sequence for (seed, stream)."""
    start = _mix_int((seed * 0xD1B54A32D192ED03 + stream * GAMMA) & _M64)
    i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(start) + i * np.uint64(GAMMA)
        return _mix(z)


def uniform01(seed: int, stream: int, n: int) -> np.ndarray:
    """float64 in [0, 1) from the top 53 bits."""
    return (splitmix64(seed, stream, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normal(seed: int, stream: int, n: int) -> np.ndarray:
    """Box-Muller: z = sqrt(-2 ln(1 - u1)) cos(2 pi u2), u from consecutive pairs."""
    u = uniform01(seed, stream, 2 * n).reshape(n, 2)
    return np.sqrt(-2.0 * np.log1p(-u[:, 0])) * np.cos(2.0 * np.pi * u[:, 1])


def packed_weights(seed: int, N: int, K: int, stream: int = STREAM_W) -> np.ndarray:
    """uint8 [N, K/2]: uniform int4 nibbles, two per byte (low nibble = even k)."""
    nbytes = N * K // 2
    words = splitmix64(seed, stream, (nbytes + 7) // 8)
    return words.view(np.uint8)[:nbytes].reshape(N, K // 2).copy()


def scales(seed: int, N: int, K: int, sigma: float = 0.02, stream: int = STREAM_S,
           group_size: int = 128) -> np.ndarray:
    """fp16 bit patterns (uint16) [N, K/G] of |N(0, sigma)| / 7."""
    z = np.abs(normal(seed, stream, N * (K // group_size))) * sigma / 7.0
    return z.astype(np.float16).view(np.uint16).reshape(N, K // group_size)


def activations(seed: int, M: int, K: int, stream: int = STREAM_X) -> np.ndarray:
    """fp16 bit patterns (uint16) [M, K] of N(0, 1)."""
    return normal(seed, stream, M * K).astype(np.float16).view(np.uint16).reshape(M, K)
