"""Python mirror of the reference's ``xinfer::ops`` projection entry points.

Same names, argument order and meaning as src/ops/linear.h and
src/ops/sampling.h, with torch device tensors in place of raw USM pointers
and the current torch stream in place of ``sycl::queue&``.  Every call goes
through the C-ABI of libxinfer_hip.so; nothing here computes on the CPU.
Status codes other than XINFER_OK raise ``XinferError``; shapes <= 0 are a
no-op, as in the reference (src/ops/linear.cpp:176).
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from ._lib import FusedDesc, check, load_library


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(stream=None):
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else stream


def linear_int4(Y: torch.Tensor, X: torch.Tensor, W_int4: torch.Tensor,
                scales: torch.Tensor, bias: Optional[torch.Tensor], M: int, N: int,
                K: int, group_size: int = 128, stream=None) -> None:
    """Y = X * dequant(W)^T (+ bias).  Overloads by dtype like src/ops/linear.h:30-63:
    (fp16 Y, fp16 X), (fp32 Y, fp16 X), (fp32 Y, fp32 X)."""
    L = load_library()
    args = (_stream(stream), _ptr(Y), _ptr(X), _ptr(W_int4), _ptr(scales), _ptr(bias),
            M, N, K, group_size)
    if X.dtype == torch.float16 and Y.dtype == torch.float16:
        check("linear_int4", L.xinfer_linear_int4_f16(*args))
    elif X.dtype == torch.float16 and Y.dtype == torch.float32:
        check("linear_int4", L.xinfer_linear_int4_f16_f32out(*args))
    elif X.dtype == torch.float32 and Y.dtype == torch.float32:
        check("linear_int4", L.xinfer_linear_int4_f32(*args))
    else:
        raise TypeError(f"no linear_int4 overload for X {X.dtype}, Y {Y.dtype}")


def linear_int4_naive(Y, X, W_int4, scales, bias, M, N, K, group_size=128, stream=None):
    """src/ops/linear.h:159-168 (fp32 in/out, one thread per output)."""
    L = load_library()
    check("linear_int4_naive", L.xinfer_linear_int4_naive_f32(
        _stream(stream), _ptr(Y), _ptr(X), _ptr(W_int4), _ptr(scales), _ptr(bias),
        M, N, K, group_size))


class FusedProjectionDesc:
    """src/ops/linear.h:66-81: {Y, W_int4, scales, bias, N}."""

    def __init__(self, Y, W_int4, scales, bias=None, N=0):
        self.Y, self.W_int4, self.scales, self.bias, self.N = Y, W_int4, scales, bias, N


def linear_int4_fused(X: torch.Tensor, descs: Sequence[FusedProjectionDesc], num_descs: int,
                      M: int, K: int, group_size: int = 128, stream=None) -> None:
    """src/ops/linear.h:97-111: up to 4 projections over one X in one launch."""
    L = load_library()
    arr = (FusedDesc * max(1, num_descs))()
    for i in range(min(num_descs, len(descs))):
        d = descs[i]
        arr[i] = FusedDesc(_ptr(d.Y), _ptr(d.W_int4), _ptr(d.scales), _ptr(d.bias), d.N)
    fn = L.xinfer_linear_int4_fused_f16 if X.dtype == torch.float16 else \
        L.xinfer_linear_int4_fused_f32
    check("linear_int4_fused", fn(_stream(stream), _ptr(X), arr, num_descs, M, K, group_size))


def mlp_gate_up_swiglu_int4(Y, X, W_gate, scales_gate, W_up, scales_up, M, N, K,
                            group_size=128, stream=None) -> None:
    """src/ops/linear.h:117-139: Y = silu(X Wg^T) * (X Wu^T)."""
    L = load_library()
    fn = L.xinfer_mlp_gate_up_swiglu_int4_f16 if X.dtype == torch.float16 else \
        L.xinfer_mlp_gate_up_swiglu_int4_f32
    check("mlp_gate_up_swiglu_int4", fn(_stream(stream), _ptr(Y), _ptr(X), _ptr(W_gate),
                                        _ptr(scales_gate), _ptr(W_up), _ptr(scales_up),
                                        M, N, K, group_size))


def argmax_scratch_size(vocab_size: int, rows: int = 1) -> int:
    """Bytes of scratch for argmax (src/ops/sampling.h:13-17 counted elements)."""
    return int(load_library().xinfer_argmax_scratch_bytes(vocab_size, rows))


def argmax_rows(logits: torch.Tensor, out_ids: torch.Tensor, vocab_size: int, rows: int,
                scratch: Optional[torch.Tensor] = None, stream=None) -> None:
    """Asynchronous batched argmax: out_ids (int64, device) [rows]."""
    L = load_library()
    nbytes = 0 if scratch is None else scratch.numel() * scratch.element_size()
    check("argmax", L.xinfer_argmax_f32(_stream(stream), _ptr(logits), vocab_size, rows,
                                        _ptr(out_ids), _ptr(scratch), nbytes))


def argmax(logits: torch.Tensor, vocab_size: int, scratch: Optional[torch.Tensor] = None,
           stream=None) -> int:
    """src/ops/sampling.h:22-26: blocking greedy argmax of one row -> token id."""
    out = torch.empty(1, dtype=torch.int64, device=logits.device)
    argmax_rows(logits, out, vocab_size, 1, scratch, stream)
    return int(out.item())


def lm_head_argmax_scratch_size(M: int, N: int, K: int) -> int:
    return int(load_library().xinfer_lm_head_argmax_scratch_bytes(M, N, K))


def lm_head_argmax_int4(ids: torch.Tensor, logits: Optional[torch.Tensor], X, W_int4, scales,
                        M, N, K, group_size=128, scratch: Optional[torch.Tensor] = None,
                        stream=None) -> None:
    """LM-head GEMV + per-row argmax in one pass (forward.cpp:304-307 + 596)."""
    L = load_library()
    nbytes = 0 if scratch is None else scratch.numel() * scratch.element_size()
    check("lm_head_argmax_int4", L.xinfer_lm_head_argmax_int4(
        _stream(stream), _ptr(ids), _ptr(logits), _ptr(X), _ptr(W_int4), _ptr(scales),
        M, N, K, group_size, _ptr(scratch), nbytes))


def dequant_int4(out: torch.Tensor, W_int4, scales, N, K, group_size=128, stream=None) -> None:
    """Device dequantisation (convert.py:129-148 semantics), fp32 [N][K]."""
    L = load_library()
    check("dequant_int4", L.xinfer_dequant_int4_f32(_stream(stream), _ptr(out), _ptr(W_int4),
                                                    _ptr(scales), N, K, group_size))


# ---- operations on either side of the projections (forward.cpp:112-125, 229, 270-290)

def rmsnorm(out: torch.Tensor, inp: torch.Tensor, weight: torch.Tensor, num_tokens: int,
            hidden_size: int, eps: float = 1e-6, stream=None) -> None:
    """src/ops/rmsnorm.h:17-23 (fp16 in/out, fp32 weight)."""
    L = load_library()
    check("rmsnorm", L.xinfer_rmsnorm_f16(_stream(stream), _ptr(out), _ptr(inp), _ptr(weight),
                                          num_tokens, hidden_size, float(eps)))


def add_inplace(a: torch.Tensor, b: torch.Tensor, num_elements: int, stream=None) -> None:
    """src/ops/elementwise.h:22 (fp16): a = fp16(fp32(a) + fp32(b))."""
    L = load_library()
    check("add_inplace", L.xinfer_add_inplace_f16(_stream(stream), _ptr(a), _ptr(b), num_elements))


def rmsnorm_projection_workspace_size(M: int, K: int) -> int:
    """Bytes of workspace the RMSNorm + projection calls need (0 at M = 1)."""
    return int(load_library().xinfer_rmsnorm_projection_workspace_bytes(M, K))


def _norm_workspace(X: torch.Tensor, M: int, K: int, workspace: Optional[torch.Tensor]):
    """The caller's workspace, or a fresh torch buffer when none was given."""
    if workspace is None:
        need = rmsnorm_projection_workspace_size(M, K)
        if need:
            workspace = torch.empty(need, dtype=torch.uint8, device=X.device)
    nbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    return _ptr(workspace), nbytes


def rmsnorm_linear_int4_fused(X: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                              descs: Sequence[FusedProjectionDesc], num_descs: int, M: int, K: int,
                              group_size: int = 128, workspace: Optional[torch.Tensor] = None,
                              stream=None) -> None:
    """rmsnorm(X) then linear_int4_fused (one launch where the kernel taking
    the shape applies the norm while it stages X; otherwise the normalised
    rows go through `workspace`, allocated here when not given at M >= 2)."""
    L = load_library()
    ws, nws = _norm_workspace(X, M, K, workspace)
    arr = (FusedDesc * max(1, num_descs))()
    for i in range(min(num_descs, len(descs))):
        d = descs[i]
        arr[i] = FusedDesc(_ptr(d.Y), _ptr(d.W_int4), _ptr(d.scales), _ptr(d.bias), d.N)
    check("rmsnorm_linear_int4_fused", L.xinfer_rmsnorm_linear_int4_fused_f16(
        _stream(stream), _ptr(X), _ptr(norm_weight), float(eps), arr, num_descs, M, K, group_size,
        ws, nws))


def rmsnorm_mlp_gate_up_swiglu_int4(Y, X, norm_weight, eps, W_gate, scales_gate, W_up, scales_up,
                                    M, N, K, group_size=128, workspace=None, stream=None) -> None:
    """rmsnorm(X) then mlp_gate_up_swiglu_int4 (workspace as rmsnorm_linear_int4_fused)."""
    L = load_library()
    ws, nws = _norm_workspace(X, M, K, workspace)
    check("rmsnorm_mlp_gate_up_swiglu_int4", L.xinfer_rmsnorm_mlp_gate_up_swiglu_int4_f16(
        _stream(stream), _ptr(Y), _ptr(X), _ptr(norm_weight), float(eps), _ptr(W_gate), _ptr(scales_gate),
        _ptr(W_up), _ptr(scales_up), M, N, K, group_size, ws, nws))


def linear_int4_residual(residual: torch.Tensor, X, W_int4, scales, bias, M, N, K, group_size=128,
                         stream=None) -> None:
    """residual += linear_int4(X) with the rounding of linear_int4 + add_inplace."""
    L = load_library()
    check("linear_int4_residual", L.xinfer_linear_int4_residual_f16(
        _stream(stream), _ptr(residual), _ptr(X), _ptr(W_int4), _ptr(scales), _ptr(bias), M, N, K,
        group_size))


def stream_release(stream) -> None:
    """Give back a stream's split-K slot and argmax scratch (no reference
    counterpart; for callers that destroy streams)."""
    L = load_library()
    check("stream_release", L.xinfer_stream_release(_stream(stream)))
