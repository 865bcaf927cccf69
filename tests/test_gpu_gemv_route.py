"""The decode GEMV on shapes the row-pair kernels take by default (M = 1,
even N, K a multiple of 1024 in 4096-6144, and M = 1 long K): a child
process with XINFER_PAIR_MIN_ROWS and XINFER_PAIRM=0 keeps them on the GEMV
(the route a caller selects with those tuning variables), checked against
the oracle at the BASELINE bound, fp32 outputs at the reference's 1e-4;
and norm + projection at M = 2 / 3 on the routes left without the dot2
kernel."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_CHILD = r"""
import sys
sys.path.insert(0, sys.argv[1])
import numpy as np, torch
import oracle
from tests.gpu_util import check_f16_tol, cpu_threads, f16_dev, to_dev, to_np
from xinfer_amd import ops, synth
from xinfer_amd._lib import load_library
load_library()
for (N, K) in ((34816, 5120), (6144, 4096), (4096, 6144), (5120, 17408)):
    print("case", N, K, flush=True)
    W, S, Xb = synth.packed_weights(N, N, K), synth.scales(N, N, K), synth.activations(K, 1, K)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, 1, N, K, nthreads=cpu_threads())
    Y = torch.full((1, N), float("nan"), dtype=torch.float16, device="cuda")
    ops.linear_int4(Y, f16_dev(Xb), to_dev(W), f16_dev(S), None, 1, N, K)
    print(check_f16_tol(to_np(Y), ref))
    Yf = torch.full((1, N), float("nan"), dtype=torch.float32, device="cuda")
    ops.linear_int4(Yf, f16_dev(Xb), to_dev(W), f16_dev(S), None, 1, N, K)
    assert np.abs(to_np(Yf) - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
N, K = 17408, 5120
Wg, Wu = synth.packed_weights(8, N, K), synth.packed_weights(8, N, K, synth.STREAM_W2)
Sg, Su = synth.scales(8, N, K), synth.scales(8, N, K, stream=synth.STREAM_S2)
Xb = synth.activations(9, 1, K)
Y = torch.full((1, N), float("nan"), dtype=torch.float16, device="cuda")
ops.mlp_gate_up_swiglu_int4(Y, f16_dev(Xb), to_dev(Wg), f16_dev(Sg), to_dev(Wu), f16_dev(Su), 1, N, K)
ref = oracle.swiglu_int4(oracle.f16_to_f32(Xb), Wg, Sg, Wu, Su, 1, N, K, nthreads=cpu_threads())
print(check_f16_tol(to_np(Y), ref))
# norm + projection at M = 2 / 3 off the dot2 kernel: the GEMV's norm
# prologue (M = 2) and the norm kernel first (M = 3)
nw = np.linspace(0.5, 1.5, K).astype(np.float32)
for M in (2, 3):
    print("case norm", M, flush=True)
    Xb = synth.activations(20 + M, M, K)
    xn = oracle.f16_to_f32(oracle.rmsnorm_f16(Xb, nw, 1e-6))
    Y = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    ops.rmsnorm_mlp_gate_up_swiglu_int4(Y, f16_dev(Xb), to_dev(nw), 1e-6, to_dev(Wg), f16_dev(Sg), to_dev(Wu),
                                        f16_dev(Su), M, N, K)
    print(check_f16_tol(to_np(Y), oracle.swiglu_int4(xn, Wg, Sg, Wu, Su, M, N, K, nthreads=cpu_threads())))
    Nq = 12288
    Wq, Sq = synth.packed_weights(30, Nq, K), synth.scales(30, Nq, K)
    Yq = torch.full((M, Nq), float("nan"), dtype=torch.float16, device="cuda")
    ops.rmsnorm_linear_int4_fused(f16_dev(Xb), to_dev(nw), 1e-6,
                                  [ops.FusedProjectionDesc(Yq, to_dev(Wq), f16_dev(Sq), None, Nq)], 1, M, K)
    print(check_f16_tol(to_np(Yq), oracle.linear_int4(xn, Wq, Sq, M, Nq, K, nthreads=cpu_threads())))
print("gemv child ok")
"""


def test_gemv_route_on_row_pair_shapes():
    env = dict(os.environ, XINFER_PAIR_MIN_ROWS="1000000000", XINFER_PAIRM="0")
    r = subprocess.run([sys.executable, "-c", _CHILD, ROOT], capture_output=True, text=True, timeout=600,
                       cwd=ROOT, env=env)
    print(r.stdout[-3000:], r.stderr[-3000:])
    assert r.returncode == 0, r.stderr[-3000:]
    assert "gemv child ok" in r.stdout
