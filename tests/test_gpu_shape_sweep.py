"""GPU parity over seeded random shapes: every entry point against the CPU
oracle on shapes no hand-picked case covers, so the launch planners'
branches (k-slices, waves per tile, blocks per CU, LDS caps, descriptor
rounding, the GEMV / small-batch / GEMM split by M) are all exercised.
Tolerances as in test_gpu_parity.py (BASELINE bound for fp16 outputs; the
reference's fp32-output bound, the fp16 one where the MFMA GEMM rounds q*s);
argmax ids equal the first max of the kernel's own logits, and the oracle's
id whenever the oracle's top-two margin exceeds 1e-3."""
import numpy as np
import pytest

import oracle
from tests import kat
from tests.gpu_util import check_f16_tol, cpu_threads, f16_dev, to_dev, to_np
from xinfer_amd import synth

pytestmark = pytest.mark.gpu

KINDS = ("lin16", "lin32", "swiglu", "fused", "resid", "argmax")
NCASES = 48
MAX_MACS = 3e8  # keeps each oracle call well under a second


def _cases():
    rng = np.random.default_rng(20260101)
    m_pool = ([1] * 6 + [2] * 4 + list(range(3, 9)) + list(range(9, 17, 2)) +
              [int(x) for x in rng.integers(17, 129, 3)] + [int(x) for x in rng.integers(129, 601, 2)])
    out = []
    for i in range(NCASES):
        kind = KINDS[i % len(KINDS)]
        M = int(rng.choice(m_pool))
        if kind == "argmax":
            M = min(M, 8)
        K = 128 * int(rng.integers(1, 141))
        N = int(rng.integers(1, 5001))
        while M * N * K > MAX_MACS and N > 1:
            N = max(1, N // 2)
        out.append((i, kind, M, N, K))
    return out


CASES = _cases()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xinfer_amd import _lib
    _lib.load_library()
    yield
    torch.cuda.synchronize()


def _empty(shape, dtype):
    import torch
    return torch.full(shape, float("nan"), dtype=dtype, device="cuda")


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}-M{c[2]}-N{c[3]}-K{c[4]}")
def test_random_shape(case):
    import torch
    from xinfer_amd import ops
    i, kind, M, N, K = case
    print("case", case, flush=True)
    nt = cpu_threads()
    Xb = synth.activations(100 + i, M, K)
    X = oracle.f16_to_f32(Xb)
    dX = f16_dev(Xb)
    if kind in ("lin16", "lin32", "resid"):
        W, S = synth.packed_weights(100 + i, N, K), synth.scales(100 + i, N, K)
        ref = oracle.linear_int4(X, W, S, M, N, K, nthreads=nt)
        if kind == "lin32":
            Y = _empty((M, N), torch.float32)
            ops.linear_int4(Y, dX, to_dev(W), f16_dev(S), None, M, N, K)
            y = to_np(Y)
            err = np.abs(y - ref).max()
            if M > 16:  # the MFMA GEMM rounds q*s to fp16: the fp16-output bound
                assert err <= 1e-2 and kat.rel_l2(y, ref) <= 1e-3, err
            else:       # fp16-in / fp32-out bound of test_ops_oracle.cpp:781
                assert err <= 1e-4 * max(1.0, np.abs(ref).max()) and kat.rel_l2(y, ref) <= 1e-4, err
            return
        if kind == "lin16":
            Y = _empty((M, N), torch.float16)
            ops.linear_int4(Y, dX, to_dev(W), f16_dev(S), None, M, N, K)
            print(check_f16_tol(to_np(Y), ref))
            return
        r0 = synth.activations(200 + i, M, N)  # residual stream, fp16
        R = f16_dev(r0)
        ops.linear_int4_residual(R, dX, to_dev(W), f16_dev(S), None, M, N, K)
        print(check_f16_tol(to_np(R), oracle.f16_to_f32(r0).astype(np.float64) + ref))
        return
    if kind == "swiglu":
        # scales |N(0, 0.01)|/7 keep SiLU(g)*u small enough for the 1e-2 bound at long K
        Wg, Sg = synth.packed_weights(100 + i, N, K), synth.scales(100 + i, N, K, 0.01)
        Wu, Su = synth.packed_weights(300 + i, N, K), synth.scales(300 + i, N, K, 0.01)
        Y = _empty((M, N), torch.float16)
        ops.mlp_gate_up_swiglu_int4(Y, dX, to_dev(Wg), f16_dev(Sg), to_dev(Wu), f16_dev(Su), M, N, K)
        ref = oracle.swiglu_int4(X, Wg, Sg, Wu, Su, M, N, K, nthreads=nt)
        print(check_f16_tol(to_np(Y), ref))
        return
    if kind == "fused":
        rng = np.random.default_rng(i)
        nd = int(rng.integers(2, 5))
        Ns = [max(1, int(N * f)) for f in rng.dirichlet(np.ones(nd))]
        descs, outs, refs = [], [], []
        for p, Np in enumerate(Ns):
            W, S = synth.packed_weights(400 + 4 * i + p, Np, K), synth.scales(400 + 4 * i + p, Np, K)
            refs.append(oracle.linear_int4(X, W, S, M, Np, K, nthreads=nt))
            Y = _empty((M, Np), torch.float16)
            outs.append(Y)
            descs.append(ops.FusedProjectionDesc(Y, to_dev(W), f16_dev(S), None, Np))
        print("descs", Ns, flush=True)
        ops.linear_int4_fused(dX, descs, nd, M, K)
        for Y, ref in zip(outs, refs):
            print(check_f16_tol(to_np(Y), ref))
        return
    # argmax: LM-head path, ids exact against the oracle's logits
    W, S = synth.packed_weights(100 + i, N, K), synth.scales(100 + i, N, K, 0.01)
    ref = oracle.linear_int4(X, W, S, M, N, K, nthreads=nt)
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    logits = _empty((M, N), torch.float32)
    ops.lm_head_argmax_int4(ids, logits, dX, to_dev(W), f16_dev(S), M, N, K)
    got, lg = to_np(ids), to_np(logits)
    for m in range(M):
        assert got[m] == oracle.argmax(lg[m])           # first max of its own logits
        if oracle.top2_margin(ref[m]) > 1e-3:            # clear winner: same as the oracle
            assert got[m] == oracle.argmax(ref[m])
    assert np.abs(lg - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
