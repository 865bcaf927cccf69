"""ctypes binding of libxinfer_hip.so (the C-ABI in include/xinfer_hip/xinfer_ops.h and
include/xinfer_hip/xinfer_artifact.h).

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
XINFER_ERR_IO = -6
XINFER_ERR_CHECKSUM = -7

# Every symbol include/xinfer_hip/*.h declares.
EXPORTS = (
    "xinfer_status_string",
    "xinfer_version",
    "xinfer_stream_release",
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
    "xinfer_lm_head_argmax_int4_noalloc",
    "xinfer_dequant_int4_f32",
    "xinfer_rmsnorm_f16",
    "xinfer_add_inplace_f16",
    "xinfer_rmsnorm_projection_workspace_bytes",
    "xinfer_rmsnorm_linear_int4_fused_f16",
    "xinfer_rmsnorm_mlp_gate_up_swiglu_int4_f16",
    "xinfer_linear_int4_residual_f16",
    # xinfer_artifact.h
    "xinfer_crc64",
    "xinfer_crc64_file",
    "xinfer_crc64_device_scratch_bytes",
    "xinfer_crc64_device",
    "xinfer_artifact_open",
    "xinfer_artifact_close",
    "xinfer_artifact_header",
    "xinfer_artifact_footer",
    "xinfer_artifact_metadata_json",
    "xinfer_artifact_section_count",
    "xinfer_artifact_section_at",
    "xinfer_artifact_section_by_name",
    "xinfer_artifact_read_section",
    "xinfer_artifact_validate_checksum",
    "xinfer_artifact_upload_section",
    "xinfer_artifact_load_linear",
)


class XinferError(RuntimeError):
    def __init__(self, fn: str, status: int):
        self.status = status
        name = _lib.xinfer_status_string(status).decode() if _lib else str(status)
        super().__init__(f"{fn} failed: {name} ({status})")


class FileHeader(ctypes.Structure):
    """Mirror of ``xinfer_file_header`` (reference FileHeader, src/artifact/container.h:35-47)."""
    _pack_ = 1
    _fields_ = [("magic", ctypes.c_uint8 * 8), ("format_version", ctypes.c_uint32),
                ("header_size", ctypes.c_uint32), ("flags", ctypes.c_uint32),
                ("section_count", ctypes.c_uint32), ("metadata_offset", ctypes.c_uint64),
                ("metadata_size", ctypes.c_uint64), ("section_table_offset", ctypes.c_uint64),
                ("section_table_size", ctypes.c_uint64), ("total_file_size", ctypes.c_uint64)]


class SectionInfo(ctypes.Structure):
    """Mirror of ``xinfer_section_info`` (reference SectionEntry, src/artifact/container.h:50-58)."""
    _pack_ = 1
    _fields_ = [("name", ctypes.c_char * 96), ("type_tag", ctypes.c_uint32),
                ("flags", ctypes.c_uint32), ("offset", ctypes.c_uint64),
                ("size", ctypes.c_uint64), ("checksum", ctypes.c_uint64)]


class LinearWeightViewC(ctypes.Structure):
    """Mirror of ``xinfer_linear_weight_view`` (reference LinearWeightView, weights.h:13-23)."""
    _fields_ = [("d_weights_int4", ctypes.c_void_p), ("d_scales", ctypes.c_void_p),
                ("in_features", ctypes.c_int64), ("out_features", ctypes.c_int64),
                ("group_size", ctypes.c_int32)]


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
    L.xinfer_stream_release.restype = ctypes.c_int
    L.xinfer_stream_release.argtypes = [_p]
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
    L.xinfer_lm_head_argmax_int4_noalloc.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32]
    L.xinfer_lm_head_argmax_int4_noalloc.restype = ctypes.c_int
    L.xinfer_dequant_int4_f32.argtypes = [_p, _p, _p, _p, _i64, _i64, _i32]
    L.xinfer_dequant_int4_f32.restype = ctypes.c_int
    f32 = ctypes.c_float
    L.xinfer_rmsnorm_f16.argtypes = [_p, _p, _p, _p, _i64, _i64, f32]
    L.xinfer_rmsnorm_f16.restype = ctypes.c_int
    L.xinfer_add_inplace_f16.argtypes = [_p, _p, _p, _i64]
    L.xinfer_add_inplace_f16.restype = ctypes.c_int
    L.xinfer_rmsnorm_projection_workspace_bytes.argtypes = [_i64, _i64]
    L.xinfer_rmsnorm_projection_workspace_bytes.restype = _sz
    L.xinfer_rmsnorm_linear_int4_fused_f16.argtypes = [_p, _p, _p, f32, ctypes.POINTER(FusedDesc), _i32,
                                                       _i64, _i64, _i32, _p, _sz]
    L.xinfer_rmsnorm_linear_int4_fused_f16.restype = ctypes.c_int
    L.xinfer_rmsnorm_mlp_gate_up_swiglu_int4_f16.argtypes = [_p, _p, _p, _p, f32, _p, _p, _p, _p,
                                                             _i64, _i64, _i64, _i32, _p, _sz]
    L.xinfer_rmsnorm_mlp_gate_up_swiglu_int4_f16.restype = ctypes.c_int
    L.xinfer_linear_int4_residual_f16.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32]
    L.xinfer_linear_int4_residual_f16.restype = ctypes.c_int
    _bind_artifact(L)
    _lib = L
    return L


def _bind_artifact(L) -> None:
    u64 = ctypes.c_uint64
    cp = ctypes.c_char_p
    L.xinfer_crc64.argtypes = [_p, _sz]
    L.xinfer_crc64.restype = u64
    L.xinfer_crc64_file.argtypes = [cp, u64]
    L.xinfer_crc64_file.restype = u64
    L.xinfer_crc64_device_scratch_bytes.argtypes = [_sz]
    L.xinfer_crc64_device_scratch_bytes.restype = _sz
    L.xinfer_crc64_device.argtypes = [_p, _p, _sz, _p, _p, _sz]
    L.xinfer_crc64_device.restype = ctypes.c_int
    L.xinfer_artifact_open.argtypes = [cp, ctypes.POINTER(_p), _p, _sz]
    L.xinfer_artifact_open.restype = ctypes.c_int
    L.xinfer_artifact_close.argtypes = [_p]
    L.xinfer_artifact_close.restype = None
    L.xinfer_artifact_header.argtypes = [_p, ctypes.POINTER(FileHeader)]
    L.xinfer_artifact_header.restype = ctypes.c_int
    L.xinfer_artifact_footer.argtypes = [_p, ctypes.POINTER(u64)]
    L.xinfer_artifact_footer.restype = ctypes.c_int
    L.xinfer_artifact_metadata_json.argtypes = [_p, ctypes.POINTER(_sz)]
    L.xinfer_artifact_metadata_json.restype = _p
    L.xinfer_artifact_section_count.argtypes = [_p]
    L.xinfer_artifact_section_count.restype = _i32
    L.xinfer_artifact_section_at.argtypes = [_p, _i32, ctypes.POINTER(SectionInfo)]
    L.xinfer_artifact_section_at.restype = ctypes.c_int
    L.xinfer_artifact_section_by_name.argtypes = [_p, cp, ctypes.POINTER(SectionInfo)]
    L.xinfer_artifact_section_by_name.restype = ctypes.c_int
    L.xinfer_artifact_read_section.argtypes = [_p, cp, _p, _sz, _p, _sz]
    L.xinfer_artifact_read_section.restype = ctypes.c_int
    L.xinfer_artifact_validate_checksum.argtypes = [_p, _p, _sz]
    L.xinfer_artifact_validate_checksum.restype = ctypes.c_int
    L.xinfer_artifact_upload_section.argtypes = [_p, cp, _p, _p, _sz, ctypes.c_int, _p, _sz]
    L.xinfer_artifact_upload_section.restype = ctypes.c_int
    L.xinfer_artifact_load_linear.argtypes = [_p, cp, _i64, _i64, _i32, _p,
                                              ctypes.POINTER(LinearWeightViewC), _p, _sz]
    L.xinfer_artifact_load_linear.restype = ctypes.c_int


def check(fn: str, status: int) -> None:
    if status != XINFER_OK:
        raise XinferError(fn, status)
