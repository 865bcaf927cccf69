"""Helpers for the GPU parity tests: numpy <-> torch device tensors."""
import os

import numpy as np


def dev():
    import torch
    return torch.device("cuda:0")


def to_dev(a: np.ndarray, kind: str = None):
    """Upload a numpy array.  kind='f16' reinterprets uint16 bit patterns as fp16."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if kind == "f16":
        t = t.view(torch.float16)
    return t.to(dev())


def f16_dev(bits: np.ndarray):
    return to_dev(np.ascontiguousarray(bits, np.uint16), "f16")


def to_np(t) -> np.ndarray:
    import torch
    t = t.detach().cpu()
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def check_f16_tol(y_bits: np.ndarray, ref: np.ndarray, max_abs=1e-2, max_rel_l2=1e-3):
    """BASELINE tolerance for fp16 outputs against the FP32-accumulate oracle."""
    import oracle
    from tests import kat
    y = oracle.f16_to_f32(y_bits).astype(np.float64)
    err = np.abs(y - ref).max()
    rl2 = kat.rel_l2(y, ref)
    assert err <= max_abs and rl2 <= max_rel_l2, f"max_abs {err:.3e} rel_l2 {rl2:.3e}"
    return err, rl2
