"""CPU oracle for the INT4-G128-SYM projection path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker (or the
reported CPU baseline).  The shipped library (``xinfer_amd``,
``libxinfer_hip.so``) never calls it.

Thin numpy/ctypes wrapper over ``liboracle_int4.so`` (``int4_oracle.c``),
which restates the reference's CPU oracle loops:

* ``linear_int4``  -- tests/test_ops_oracle.cpp:319-348 (double accumulate)
* ``swiglu_int4``  -- tests/test_ops_oracle.cpp:626-669
* ``argmax``       -- tests/test_ops_oracle.cpp:926-933, src/ops/sampling.cpp:75-85
* ``dequant_int4`` -- tools/convert/qwen3_8_27b/convert.py:129-148
* ``quantize_int4``-- tools/convert/qwen3_8_27b/convert.py:93-119
* ``rmsnorm_f16``  -- src/ops/rmsnorm.cpp:45-78
* ``add_inplace_f16`` -- src/ops/elementwise.cpp:213-231
* ``crc64``        -- src/artifact/checksum.cpp:10-54 (one byte per step)
* ``f16``/``f32``  -- own IEEE binary16 conversion (round to nearest even)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_int4.so")
_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile the oracle with gcc (make -C oracle)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", _HERE],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_half_to_float.restype = ctypes.c_float
        L.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_float_to_half.restype = ctypes.c_uint16
        L.oracle_float_to_half.argtypes = [ctypes.c_float]
        L.oracle_half_to_float_n.argtypes = [_p, _p, _i64]
        L.oracle_float_to_half_n.argtypes = [_p, _p, _i64]
        L.oracle_nibble.restype = ctypes.c_int
        L.oracle_nibble.argtypes = [ctypes.c_uint8, ctypes.c_int]
        L.oracle_dequant_int4.argtypes = [_p, _p, _p, _i64, _i64, _i64]
        L.oracle_quantize_int4.argtypes = [_p, _p, _p, _i64, _i64, _i64]
        L.oracle_linear_int4.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64,
                                         _i64, ctypes.c_int]
        L.oracle_swiglu_int4.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64,
                                         _i64, _i64, ctypes.c_int]
        L.oracle_argmax.restype = ctypes.c_int64
        L.oracle_argmax.argtypes = [_p, _i64]
        L.oracle_top2_margin.restype = ctypes.c_float
        L.oracle_top2_margin.argtypes = [_p, _i64]
        L.oracle_rmsnorm_f16.argtypes = [_p, _p, _p, _i64, _i64, ctypes.c_float]
        L.oracle_add_inplace_f16.argtypes = [_p, _p, _i64]
        L.oracle_crc64.restype = ctypes.c_uint64
        L.oracle_crc64.argtypes = [_p, _i64]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def f16_to_f32(h) -> np.ndarray:
    """fp16 bit patterns (uint16) -> float32 values."""
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_half_to_float_n(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_f16(f) -> np.ndarray:
    """float32 values -> fp16 bit patterns (uint16), round to nearest even."""
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().oracle_float_to_half_n(_ptr(f), _ptr(out), f.size)
    return out


def nibble(byte: int, high: bool) -> int:
    return lib().oracle_nibble(byte, 1 if high else 0)


def dequant_int4(W, S, N, K, G=128) -> np.ndarray:
    W = _c(W, np.uint8)
    S = _c(S, np.uint16)
    out = np.empty((N, K), np.float32)
    lib().oracle_dequant_int4(_ptr(out), _ptr(W), _ptr(S), N, K, G)
    return out


def quantize_int4(w, G=128):
    w = _c(w, np.float32)
    N, K = w.shape
    W = np.empty((N, K // 2), np.uint8)
    S = np.empty((N, K // G), np.uint16)
    lib().oracle_quantize_int4(_ptr(W), _ptr(S), _ptr(w), N, K, G)
    return W, S


def linear_int4(X, W, S, M, N, K, G=128, bias=None, nthreads=1) -> np.ndarray:
    """X: float32 [M,K] (fp16 inputs: pass f16_to_f32(X_bits)). -> float32 [M,N]."""
    X = _c(X, np.float32)
    W = _c(W, np.uint8)
    S = _c(S, np.uint16)
    b = None if bias is None else _c(bias, np.float32)
    Y = np.zeros((M, N), np.float32)
    lib().oracle_linear_int4(_ptr(Y), _ptr(X), _ptr(W), _ptr(S), _ptr(b),
                             M, N, K, G, nthreads)
    return Y


def swiglu_int4(X, Wg, Sg, Wu, Su, M, N, K, G=128, nthreads=1) -> np.ndarray:
    X = _c(X, np.float32)
    Y = np.zeros((M, N), np.float32)
    lib().oracle_swiglu_int4(_ptr(Y), _ptr(X), _ptr(_c(Wg, np.uint8)),
                             _ptr(_c(Sg, np.uint16)), _ptr(_c(Wu, np.uint8)),
                             _ptr(_c(Su, np.uint16)), M, N, K, G, nthreads)
    return Y


def argmax(logits) -> int:
    x = _c(logits, np.float32).reshape(-1)
    return int(lib().oracle_argmax(_ptr(x), x.size))


def top2_margin(logits) -> float:
    x = _c(logits, np.float32).reshape(-1)
    return float(lib().oracle_top2_margin(_ptr(x), x.size))


def rmsnorm_f16(x_bits, weight, eps=1e-6) -> np.ndarray:
    """x_bits: uint16 [T, H] fp16 bit patterns -> uint16 [T, H]."""
    x = _c(x_bits, np.uint16)
    T, H = x.shape
    w = _c(weight, np.float32)
    out = np.zeros_like(x)
    lib().oracle_rmsnorm_f16(_ptr(out), _ptr(x), _ptr(w), T, H, float(eps))
    return out


def add_inplace_f16(a_bits, b_bits) -> np.ndarray:
    """Returns fp16(fp32(a) + fp32(b)) as uint16 (a copy; inputs untouched)."""
    a = np.array(a_bits, np.uint16, copy=True)
    b = _c(b_bits, np.uint16)
    lib().oracle_add_inplace_f16(_ptr(a), _ptr(b), a.size)
    return a


def crc64(data) -> int:
    """CRC-64/ECMA-182 (reflected) of bytes / a uint8 array."""
    a = np.frombuffer(bytes(data), np.uint8) if isinstance(data, (bytes, bytearray, memoryview)) \
        else _c(np.asarray(data).reshape(-1).view(np.uint8), np.uint8)
    return int(lib().oracle_crc64(_ptr(a), a.size))


# ------------------------------------------------------------------------
# Reference artifact code built from /root/reference (oracle/_ref/artifact_ref):
# the reference's own writer / reader / CRC, driven by ref_artifact_driver.cpp.
_REF_TOOL = os.path.join(_HERE, "_ref", "artifact_ref")


def ref_artifact_tool():
    """Path of the reference-built artifact tool, or None when absent."""
    return _REF_TOOL if os.path.exists(_REF_TOOL) else None
