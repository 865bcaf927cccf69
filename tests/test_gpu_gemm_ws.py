"""Parity of the producer/consumer prefill GEMM (gemm_ws_int4.hip) against
the oracle at the BASELINE fp16 bound (max abs <= 1e-2, rel-L2 <= 1e-3).
The default routing sends only shapes that fill the CUs to it (config 4);
a child process with XINFER_GEMM_WS=1 forces it for ragged shapes: M and N
off the 256 x 136 block (a partial last row block, N below one block and
not a multiple of 8, partial last column blocks), bias, the residual form,
and an output view 2 bytes past a 16-byte boundary (the per-element store
path instead of 16-byte stores)."""
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from tests import kat
from tests.gpu_util import check_f16_tol, cpu_threads, f16_dev, to_dev, to_np
from xinfer_amd import synth

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


_CHILD = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import oracle
from tests import kat
from xinfer_amd import synth, ops
dev = torch.device("cuda:0")
def f16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.float16).to(dev)
def bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)
shapes = [(17, 272, 1024), (128, 544, 1024), (130, 300, 2048), (200, 560, 1024), (257, 1000, 3072),
          (64, 17, 1024), (512, 4352, 2048), (300, 408, 1024), (512, 136, 5120)]
for (M, N, K) in shapes:
    print("case", M, N, K, flush=True)
    W, S, Xb = synth.packed_weights(M + N, N, K), synth.scales(M + N, N, K), synth.activations(M, M, K)
    bias = np.linspace(-1, 1, N).astype(np.float32)
    dW, dS, dX = torch.from_numpy(W).to(dev), f16(S), f16(Xb)
    X = oracle.f16_to_f32(Xb)
    Y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    ops.linear_int4(Y, dX, dW, dS, torch.from_numpy(bias).to(dev), M, N, K)
    ref = oracle.linear_int4(X, W, S, M, N, K, bias=bias, nthreads=8)
    y = oracle.f16_to_f32(bits(Y)).astype(np.float64)
    err, rl2 = float(np.abs(y - ref).max()), kat.rel_l2(y, ref)
    assert err <= 1e-2 and rl2 <= 1e-3, (M, N, K, err, rl2)
    # residual form: R = fp16(R + fp16(linear))
    R0 = oracle.f32_to_f16(np.random.default_rng(M).normal(0, 1, (M, N)).astype(np.float32))
    R = f16(R0)
    ops.linear_int4_residual(R, dX, dW, dS, None, M, N, K)
    Yp = torch.empty((M, N), dtype=torch.float16, device=dev)
    ops.linear_int4(Yp, dX, dW, dS, None, M, N, K)
    want = (Yp.float() + f16(R0).float()).half()
    assert torch.equal(R, want), (M, N, K)
    # an output view 2 bytes past a 16-byte boundary
    Yb = torch.full((M * N + 8,), float("nan"), dtype=torch.float16, device=dev)
    Yo = Yb[1:1 + M * N].view(M, N)
    ops.linear_int4(Yo, dX, dW, dS, torch.from_numpy(bias).to(dev), M, N, K)
    assert torch.equal(Yo, Y), (M, N, K, "offset view")
    assert torch.isnan(Yb[0]) and torch.isnan(Yb[1 + M * N:]).all(), (M, N, K, "outside the view")
    print("ok", M, N, K, err, rl2, flush=True)
print("ws child ok")
"""


def test_ws_forced_ragged_shapes():
    env = dict(os.environ, XINFER_GEMM_WS="1")
    r = subprocess.run([sys.executable, "-c", _CHILD, ROOT], capture_output=True, text=True, timeout=600,
                       cwd=ROOT, env=env)
    print(r.stdout[-3000:], r.stderr[-3000:])
    assert r.returncode == 0, r.stderr[-3000:]
    assert "ws child ok" in r.stdout


def test_ws_config4_all_rows():
    """Config 4 (M = 512, N = 17408, K = 5120) on its default route, every row
    against the oracle."""
    import torch
    from xinfer_amd import ops
    M, N, K = 512, 17408, 5120
    print("case cfg4 all rows", flush=True)
    W, S, Xb = synth.packed_weights(0, N, K), synth.scales(0, N, K), synth.activations(0, M, K)
    Y = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    ops.linear_int4(Y, f16_dev(Xb), to_dev(W), f16_dev(S), None, M, N, K)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
    print(check_f16_tol(to_np(Y), ref))
