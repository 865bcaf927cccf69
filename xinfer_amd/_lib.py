"""ctypes binding of libxinfer_hip.so (the C-ABI in include/xinfer_hip/xinfer_ops.h).

Loading fails loudly when the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libxinfer_hip.so")

XINFER_OK = 0
XINFER_ERR_INVALID_ARG = -1
XINFER_ERR_UNSUPPORTED = -2
XINFER_ERR_MISALIGNED = -3
XINFER_ERR_HIP = -4
XINFER_ERR_SCRATCH = -5

# Every symbol include/xinfer_hip/xinfer_ops.h declares.
EXPORTS = (
    "xinfer_status_string",
    "xinfer_version",
    "xinfer_linear_int4_f16",
    "xinfer_linear_int4_f16_f32out",
    "xinfer_linear_int4_f32",
    "xinfer_linear_int4_naive_f32",
    "xinfer_linear_int4_fused_f16",
    "xinfer_linear_int4_fused_f32",
    "xinfer_mlp_gate_up_swiglu_int4_f16",
    "xinfer_mlp_gate_up_swiglu_int4_f32",
    "xinfer_argmax_scratch_bytes",
    "xinfer_argmax_f32",
    "xinfer_lm_head_argmax_scratch_bytes",
    "xinfer_lm_head_argmax_int4",
    "xinfer_dequant_int4_f32",
)


class XinferError(RuntimeError):
    def __init__(self, fn: str, status: int):
        self.status = status
        name = _lib.xinfer_status_string(status).decode() if _lib else str(status)
        super().__init__(f"{fn} failed: {name} ({status})")


class FusedDesc(ctypes.Structure):
    """Mirror of ``xinfer_fused_desc`` (reference FusedProjectionDesc, src/ops/linear.h:66-72)."""
    _fields_ = [("Y", ctypes.c_void_p), ("W_int4", ctypes.c_void_p),
                ("scales", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("N", ctypes.c_int64)]


_lib = None
_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_sz = ctypes.c_size_t


def load_library(path: str = None):
    """Load libxinfer_hip.so.  torch is imported first so the library binds to
    the HIP runtime torch already loaded (same soname)."""
    global _lib
    if _lib is not None:
        return _lib
    # XINFER_HIP_LIB selects another build of the same library (tuning runs)
    path = path or os.environ.get("XINFER_HIP_LIB") or LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m xinfer_amd.build` "
            "(there is no CPU fallback for this path)")
    import torch  # noqa: F401  (binds libamdhip64 before dlopen)
    L = ctypes.CDLL(path)
    for name in EXPORTS:
        getattr(L, name)  # AttributeError if a declared symbol is missing
    L.xinfer_status_string.restype = ctypes.c_char_p
    L.xinfer_status_string.argtypes = [ctypes.c_int]
    L.xinfer_version.restype = ctypes.c_char_p
    L.xinfer_version.argtypes = []
    lin = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32]
    for n in ("xinfer_linear_int4_f16", "xinfer_linear_int4_f16_f32out",
              "xinfer_linear_int4_f32", "xinfer_linear_int4_naive_f32"):
        getattr(L, n).argtypes = lin
        getattr(L, n).restype = ctypes.c_int
    for n in ("xinfer_linear_int4_fused_f16", "xinfer_linear_int4_fused_f32"):
        getattr(L, n).argtypes = [_p, _p, ctypes.POINTER(FusedDesc), _i32, _i64, _i64, _i32]
        getattr(L, n).restype = ctypes.c_int
    for n in ("xinfer_mlp_gate_up_swiglu_int4_f16", "xinfer_mlp_gate_up_swiglu_int4_f32"):
        getattr(L, n).argtypes = [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32]
        getattr(L, n).restype = ctypes.c_int
    L.xinfer_argmax_scratch_bytes.argtypes = [_i64, _i64]
    L.xinfer_argmax_scratch_bytes.restype = _sz
    L.xinfer_argmax_f32.argtypes = [_p, _p, _i64, _i64, _p, _p, _sz]
    L.xinfer_argmax_f32.restype = ctypes.c_int
    L.xinfer_lm_head_argmax_scratch_bytes.argtypes = [_i64, _i64, _i64]
    L.xinfer_lm_head_argmax_scratch_bytes.restype = _sz
    L.xinfer_lm_head_argmax_int4.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32,
                                             _p, _sz]
    L.xinfer_lm_head_argmax_int4.restype = ctypes.c_int
    L.xinfer_dequant_int4_f32.argtypes = [_p, _p, _p, _p, _i64, _i64, _i32]
    L.xinfer_dequant_int4_f32.restype = ctypes.c_int
    _lib = L
    return L


def check(fn: str, status: int) -> None:
    if status != XINFER_OK:
        raise XinferError(fn, status)
