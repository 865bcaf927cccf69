"""xinfer_lm_head_argmax_int4_noalloc (candidates in a static device array)
against xinfer_lm_head_argmax_int4 with caller scratch, through the C-ABI:
ids and logits bit-identical on two calls in a row, the second smaller, and
ids exact against the oracle."""
import numpy as np
import pytest

import oracle
from tests.gpu_util import cpu_threads, f16_dev, to_dev, to_np
from xinfer_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.synchronize()


def _lib():
    from xinfer_amd import _lib as xl
    return xl.load_library()


def _run(L, M, N, K, seed):
    import torch
    print("case noalloc lm-head M", M, "N", N, "K", K, flush=True)
    W, S, Xb = synth.packed_weights(seed, N, K), synth.scales(seed, N, K, 0.01), synth.activations(seed, M, K)
    dW, dS, dX = to_dev(W), f16_dev(S), f16_dev(Xb)
    st = torch.cuda.current_stream().cuda_stream
    ids_a = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    lg_a = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    rc = L.xinfer_lm_head_argmax_int4_noalloc(st, ids_a.data_ptr(), lg_a.data_ptr(), dX.data_ptr(),
                                              dW.data_ptr(), dS.data_ptr(), M, N, K, 128)
    assert rc == 0, rc
    nbytes = L.xinfer_lm_head_argmax_scratch_bytes(M, N, K)
    scr = torch.empty(max(8, nbytes), dtype=torch.uint8, device="cuda")
    ids_b = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    lg_b = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    rc = L.xinfer_lm_head_argmax_int4(st, ids_b.data_ptr(), lg_b.data_ptr(), dX.data_ptr(), dW.data_ptr(),
                                      dS.data_ptr(), M, N, K, 128, scr.data_ptr(), scr.numel())
    assert rc == 0, rc
    torch.cuda.synchronize()
    assert np.array_equal(to_np(ids_a), to_np(ids_b))
    assert np.array_equal(to_np(lg_a).view(np.uint32), to_np(lg_b).view(np.uint32))
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
    for m in range(M):
        assert int(to_np(ids_a)[m]) == oracle.argmax(ref[m]), m


def test_noalloc_lm_head_matches_scratch_entry_point():
    L = _lib()
    _run(L, 8, 151936, 5120, 0)   # config 3 at M = 8 (small-batch kernel, 2 launches)
    _run(L, 1, 32768, 4096, 1)    # then a smaller call: M = 1 GEMV plan, fewer candidates
