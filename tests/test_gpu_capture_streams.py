"""The projection entry points allocate nothing and never synchronise, so
(1) the very first call of a process can be captured into a graph, and
(2) calls on different streams may overlap.

(1) runs in a fresh child process: the library is loaded and its first call
ever -- a small-batch projection that splits K over blocks (M = 4,
K = 17408, N = 5120, the down projection of config 2) -- is made inside
torch.cuda.graph capture (capture_error_mode "global": any allocation or
device synchronisation inside the call fails the capture).  Replays are
compared with the oracle.
(2) enqueues M = 8 launches of that shape on two (then forty) streams without
synchronising in between; every result must be bit-identical to a solo run
and within the fp32-output bound of the oracle.  Forty streams exceed the
library's 32 split-K slots per device: the extra streams plan without the
cross-block split (another summation order, so other bits than the solo
run), and every one of their results must match the oracle and each other."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from tests import kat
from tests.gpu_util import cpu_threads, f16_dev, to_dev, to_np
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


def _check_f32(y, ref):
    err = np.abs(y - ref).max()
    assert err <= 1e-4 * max(1.0, np.abs(ref).max()) and kat.rel_l2(y, ref) <= 1e-4, err


_CHILD = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import oracle
from xinfer_amd import synth, ops
M, N, K = 4, 5120, 17408
W, S, Xb = synth.packed_weights(5, N, K), synth.scales(5, N, K), synth.activations(5, M, K)
dev = torch.device("cuda:0")
dW = torch.from_numpy(W).to(dev)
dS = torch.from_numpy(S.view(np.int16)).view(torch.float16).to(dev)
dX = torch.from_numpy(Xb.view(np.int16)).view(torch.float16).to(dev)
Y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
s = torch.cuda.Stream()
with torch.cuda.stream(s):
    with torch.cuda.graph(g, stream=s, capture_error_mode="global"):
        ops.linear_int4(Y, dX, dW, dS, None, M, N, K)   # the library's first call
torch.cuda.synchronize()
ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=8)
first = None
for rep in range(3):
    Y.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    y = Y.cpu().numpy()
    err = float(np.abs(y - ref).max())
    assert err <= 1e-4 * max(1.0, float(np.abs(ref).max())), (rep, err)
    if first is None:
        first = y.copy()
    assert np.array_equal(first.view(np.uint32), y.view(np.uint32)), rep
print("first-call capture ok", err)
"""


def test_first_call_captured_in_fresh_process():
    print("case first-call capture M=4 N=5120 K=17408", flush=True)
    r = subprocess.run([sys.executable, "-c", _CHILD, ROOT], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    print(r.stdout[-2000:], r.stderr[-3000:])
    assert r.returncode == 0, r.stderr[-3000:]
    assert "first-call capture ok" in r.stdout


@pytest.mark.parametrize("nstreams", [2, 40])
def test_concurrent_streams_small_batch(nstreams):
    import torch
    from xinfer_amd import ops
    M, N, K = 8, 5120, 17408
    reps = 6 if nstreams <= 2 else 3
    print("case streams", nstreams, "M", M, "N", N, "K", K, flush=True)
    ins = []
    for i in range(nstreams):
        W, S, Xb = synth.packed_weights(40 + i, N, K), synth.scales(40 + i, N, K), synth.activations(40 + i, M, K)
        ins.append((W, S, Xb, to_dev(W), f16_dev(S), f16_dev(Xb)))
    # solo runs on the current stream (the reference bits of each input)
    solo = []
    for (_, _, _, dW, dS, dX) in ins:
        Y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        ops.linear_int4(Y, dX, dW, dS, None, M, N, K)
        torch.cuda.synchronize()
        solo.append(to_np(Y).copy())
    refs = [oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
            for (W, S, Xb) in (x[:3] for x in ins)]
    for i in range(nstreams):
        _check_f32(solo[i], refs[i])
    # raw HIP streams (torch's pool hands out at most 32 distinct streams per
    # priority, so 40 torch streams would repeat handles)
    hip = ctypes.CDLL("libamdhip64.so")
    handles = []
    for _ in range(nstreams):
        h = ctypes.c_void_p()
        assert hip.hipStreamCreate(ctypes.byref(h)) == 0
        handles.append(h.value)
    assert len(set(handles)) == nstreams
    streams = handles
    outs = [[torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda") for _ in range(reps)]
            for _ in range(nstreams)]
    torch.cuda.synchronize()
    for r in range(reps):  # interleaved: every stream has work queued while the others run
        for i, st in enumerate(streams):
            _, _, _, dW, dS, dX = ins[i]
            ops.linear_int4(outs[i][r], dX, dW, dS, None, M, N, K, stream=st)
    torch.cuda.synchronize()
    exact = 0
    for i in range(nstreams):
        first = to_np(outs[i][0])
        _check_f32(first, refs[i])
        for r in range(1, reps):
            assert np.array_equal(to_np(outs[i][r]).view(np.uint32), first.view(np.uint32)), (i, r)
        exact += np.array_equal(first.view(np.uint32), solo[i].view(np.uint32))
    print("streams with the solo run's bits:", exact, "of", nstreams)
    if nstreams <= 2:  # both streams hold a split-K slot: the solo plan
        assert exact == nstreams
    else:  # more streams than slots: some ran the plan without the cross-block split
        assert exact < nstreams
    # giving the slots back lets new streams take them: after the release a
    # fresh stream runs the split-K plan again (the solo run's bits)
    for h in handles:
        ops.stream_release(h)
        assert hip.hipStreamDestroy(ctypes.c_void_p(h)) == 0
    h = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(h)) == 0
    _, _, _, dW, dS, dX = ins[0]
    Y = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    ops.linear_int4(Y, dX, dW, dS, None, M, N, K, stream=h.value)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(Y).view(np.uint32), solo[0].view(np.uint32))
    ops.stream_release(h.value)
    assert hip.hipStreamDestroy(h) == 0
