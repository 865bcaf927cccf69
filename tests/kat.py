"""Input builders shared by the tests.

The integer-pattern fixtures are the reference's own known-answer inputs
(tests/test_ops_oracle.cpp); the reference drew X from std::mt19937 +
uniform_real_distribution, whose float mapping is implementation-defined,
so X here comes from the seeded SplitMix64 stream of xinfer_amd.synth.
"""
from __future__ import annotations

import numpy as np

from xinfer_amd import synth


def pattern_weights(N: int, K: int, lo_off: int, hi_off: int, p: int = 0) -> np.ndarray:
    """byte i = ((i + p + lo_off) & 15) | ((i + p + hi_off) & 15) << 4
    (test_ops_oracle.cpp:311-315, 405-409, 520-523, 617-620, 722-724)."""
    i = np.arange(N * (K // 2), dtype=np.int64)
    b = ((i + p + lo_off) & 15) | (((i + p + hi_off) & 15) << 4)
    return b.astype(np.uint8).reshape(N, K // 2)


def pattern_scales(N: int, K: int, base: float = 0.015, shift: int = 0,
                   p: int = 0, G: int = 128) -> np.ndarray:
    """scale i = half(base + 0.001 * ((i + p + shift) % 10)) (test_ops_oracle.cpp:307-309)."""
    from oracle import f32_to_f16
    i = np.arange(N * (K // G), dtype=np.int64)
    v = (np.float32(base) + ((i + p + shift) % 10).astype(np.float32) * np.float32(0.001))
    return f32_to_f16(v.astype(np.float32)).reshape(N, K // G)


def uniform_x(seed: int, M: int, K: int, lo: float = -1.0, hi: float = 1.0,
              stream: int = synth.STREAM_X) -> np.ndarray:
    u = synth.uniform01(seed, stream, M * K)
    return (lo + (hi - lo) * u).astype(np.float32).reshape(M, K)


def dense_dequant_np(W: np.ndarray, S_f32: np.ndarray, G: int = 128) -> np.ndarray:
    """Independent numpy formulation of the dequantised matrix, float64:
    sign-extend nibbles with int8 arithmetic shifts, interleave lo/hi."""
    N = W.shape[0]
    lo = (W.astype(np.int8) << 4) >> 4           # arithmetic shift sign-extends
    hi = W.astype(np.int8) >> 4
    q = np.empty((N, W.shape[1] * 2), np.float64)
    q[:, 0::2] = lo
    q[:, 1::2] = hi
    return q * np.repeat(S_f32.astype(np.float64), G, axis=1)


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
