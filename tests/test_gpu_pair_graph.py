"""The row-pair kernels (M = 1 plain / SwiGLU / fused RMSNorm, M = 2 SwiGLU
in the dot2 form, M = 1 long K over four waves) captured into a HIP graph:
every replay, with eager launches and synchronisations in between, gives
the bits of the eager call, which is itself held to the oracle's bound in
test_gpu_parity.py / test_gpu_fusion.py.  The kernels clear no memory and
allocate nothing, so nothing in them depends on the replay count."""
import numpy as np
import pytest

from tests.gpu_util import f16_dev, to_dev, to_np
from xinfer_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xinfer_amd import _lib
    _lib.load_library()
    yield
    torch.cuda.synchronize()


def _check_replays(fn, outs):
    import torch
    fn()
    torch.cuda.synchronize()
    want = [to_np(o).copy() for o in outs]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        fn()  # eager work between the replays
        torch.cuda.synchronize()
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert np.array_equal(to_np(o).view(np.uint16), w.view(np.uint16)), rep


@pytest.mark.parametrize("M", [1, 2])
def test_pair_swiglu_graph(M):
    import torch
    from xinfer_amd import ops
    print("case swiglu", M, flush=True)
    N, K = 17408, 5120
    Wg, Wu = to_dev(synth.packed_weights(1, N, K)), to_dev(synth.packed_weights(2, N, K))
    Sg, Su = f16_dev(synth.scales(1, N, K)), f16_dev(synth.scales(2, N, K))
    X = f16_dev(synth.activations(3, M, K))
    Y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    _check_replays(lambda: ops.mlp_gate_up_swiglu_int4(Y, X, Wg, Sg, Wu, Su, M, N, K), [Y])


def test_pair_norm_qkv_and_long_k_graph():
    import torch
    from xinfer_amd import ops
    print("case norm+qkv, long K", flush=True)
    K, Ns = 5120, (12288, 1024, 1024)
    X = f16_dev(synth.activations(4, 1, K))
    nw = to_dev(np.linspace(0.5, 1.5, K).astype(np.float32))
    Ys = [torch.empty((1, N), dtype=torch.float16, device="cuda") for N in Ns]
    Ws = [(to_dev(synth.packed_weights(10 + i, N, K)), f16_dev(synth.scales(10 + i, N, K))) for i, N in enumerate(Ns)]

    def qkv():
        ds = [ops.FusedProjectionDesc(Y, W, S, None, N) for Y, (W, S), N in zip(Ys, Ws, Ns)]
        ops.rmsnorm_linear_int4_fused(X, nw, 1e-6, ds, 3, 1, K)
    _check_replays(qkv, Ys)
    N2, K2 = 5120, 17408  # down projection at M = 1: K over four waves
    W2, S2 = to_dev(synth.packed_weights(20, N2, K2)), f16_dev(synth.scales(20, N2, K2))
    X2 = f16_dev(synth.activations(21, 1, K2))
    Y2 = torch.empty((1, N2), dtype=torch.float16, device="cuda")
    _check_replays(lambda: ops.linear_int4(Y2, X2, W2, S2, None, 1, N2, K2), [Y2])
