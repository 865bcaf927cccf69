"""GPU parity of the decode-layer fusions around the projection kernels:
the RMSNorm prologue (src/ops/rmsnorm.cpp:45-78 applied to X while it is
staged, forward.cpp:112-125 / 237-247 / 273-281), the residual-add epilogue
(forward.cpp:229 / 270 / 284-290: o_proj / down_proj then add_inplace) and
the standalone rmsnorm / add_inplace ops they replace.

Bounds: standalone rmsnorm within one fp16 ulp of the oracle (the FP32 sum
of squares is taken in another order); fused projections fp16 max abs
<= 1e-2 and relative L2 <= 1e-3 against the oracle's linear(rmsnorm(X));
the residual epilogue bit-exact against linear_int4 followed by add_inplace
(it is the same two roundings); add_inplace bit-exact."""
import numpy as np
import pytest

import oracle
from tests.gpu_util import check_f16_tol, cpu_threads, f16_dev, to_dev, to_np
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


def _ops():
    from xinfer_amd import ops
    return ops


def _empty(shape, dtype):
    import torch
    return torch.full(shape, float("nan"), dtype=dtype, device="cuda")


def _bits(t):
    return to_np(t).view(np.uint16)


def _norm_w(seed, K, lo=0.0, hi=2.0):
    """U(0, 2) as in tests/test_ops_oracle.cpp:61-62; the projection tests use
    U(0.5, 1.5) so that outputs keep the magnitude of the unfused tests (an
    fp16 output above 32 rounds by up to 0.0156, beyond the 1e-2 bound)."""
    rng = np.random.default_rng(seed)
    return rng.uniform(lo, hi, K).astype(np.float32)


def _xin(seed, M, K, scale=1.0):
    rng = np.random.default_rng(seed)
    return oracle.f32_to_f16(rng.uniform(-scale, scale, (M, K)).astype(np.float32))


@pytest.mark.parametrize("T,H", [(4, 5120), (1, 128), (7, 17408), (3, 1000), (300, 5120), (2, 1001), (5, 24)])
def test_rmsnorm_vs_oracle(T, H):
    import torch
    ops = _ops()
    print("case", T, H, flush=True)
    x, w = _xin(T + H, T, H, 3.0), _norm_w(H, H)
    out = _empty((T, H), torch.float16)
    ops.rmsnorm(out, f16_dev(x), to_dev(w), T, H, 1e-6)
    got = oracle.f16_to_f32(_bits(out)).astype(np.float64)
    ref = oracle.f16_to_f32(oracle.rmsnorm_f16(x, w, 1e-6)).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert (np.abs(got - ref) <= ulp).all(), np.abs(got - ref).max()


def test_add_inplace_bit_exact():
    import torch
    ops = _ops()
    for n in (1, 7, 4096, 1_000_003):
        rng = np.random.default_rng(n)
        a = oracle.f32_to_f16(rng.normal(0, 4, n).astype(np.float32))
        b = oracle.f32_to_f16(rng.normal(0, 4, n).astype(np.float32))
        da = f16_dev(a)
        ops.add_inplace(da, f16_dev(b), n)
        assert np.array_equal(_bits(da), oracle.add_inplace_f16(a, b)), n


def _ref_linear_after_norm(x, w, W, S, M, N, K, bias=None):
    xn = oracle.f16_to_f32(oracle.rmsnorm_f16(x, w, 1e-6))
    return oracle.linear_int4(xn, W, S, M, N, K, bias=bias, nthreads=cpu_threads())


@pytest.mark.parametrize("M", [1, 2, 3, 4, 6, 8])
def test_rmsnorm_fused_qkv_descs(M):
    """Qwen3.5-27B full-attention shape (q 12288, k 1024, v 1024 at K 5120)
    with the input norm fused into the projection launch."""
    import torch
    ops = _ops()
    K, Ns = 5120, (12288, 1024, 1024)
    x, w = _xin(60 + M, M, K, 2.0), _norm_w(61, K, 0.5, 1.5)
    dX, dw = f16_dev(x), to_dev(w)
    descs, refs, outs = [], [], []
    for p, N in enumerate(Ns):
        W, S = synth.packed_weights(70 + p, N, K), synth.scales(70 + p, N, K)
        bias = np.linspace(-1, 1, N).astype(np.float32) if p == 2 else None
        refs.append(_ref_linear_after_norm(x, w, W, S, M, N, K, bias))
        Y = _empty((M, N), torch.float16)
        outs.append(Y)
        descs.append(ops.FusedProjectionDesc(Y, to_dev(W), f16_dev(S),
                                             None if bias is None else to_dev(bias), N))
    ops.rmsnorm_linear_int4_fused(dX, dw, 1e-6, descs, 3, M, K)
    for Y, ref in zip(outs, refs):
        print(check_f16_tol(to_np(Y), ref))
    assert np.array_equal(_bits(dX), x)          # the input itself is not normalised in place


@pytest.mark.parametrize("M", [2, 3, 4])
def test_rmsnorm_fused_short_rows(M):
    """4096 output rows over three descriptors: the norm in the GEMV's staging
    at M = 2, in the dot2 kernel's at M = 3, the norm kernel first at M = 4."""
    import torch
    ops = _ops()
    K, Ns = 5120, (2048, 1024, 1024)
    print("case", M, flush=True)
    x, w = _xin(300 + M, M, K, 2.0), _norm_w(301, K, 0.5, 1.5)
    descs, refs, outs = [], [], []
    for p, N in enumerate(Ns):
        W, S = synth.packed_weights(310 + p, N, K), synth.scales(310 + p, N, K)
        refs.append(_ref_linear_after_norm(x, w, W, S, M, N, K))
        Y = _empty((M, N), torch.float16)
        outs.append(Y)
        descs.append(ops.FusedProjectionDesc(Y, to_dev(W), f16_dev(S), None, N))
    ops.rmsnorm_linear_int4_fused(f16_dev(x), to_dev(w), 1e-6, descs, 3, M, K)
    for Y, ref in zip(outs, refs):
        print(check_f16_tol(to_np(Y), ref))


@pytest.mark.parametrize("M,N,K", [(1, 17408, 5120), (2, 17408, 5120), (3, 17408, 5120), (4, 17408, 5120), (8, 1000, 1024), (3, 640, 17408),
                                   (1, 640, 17408), (2, 640, 17408), (2, 4096, 5120), (1, 2048, 4096), (1, 4096, 6144),
                                   (8, 17408, 5120), (4, 2048, 6144), (8, 640, 4096),
                                   (8, 1024, 6144), (5, 2048, 5120), (7, 4096, 4096), (3, 1024, 5120)])
def test_rmsnorm_fused_swiglu(M, N, K):
    import torch
    from scipy.special import expit
    ops = _ops()
    print("case", M, N, K, flush=True)
    Wg, Wu = synth.packed_weights(8, N, K), synth.packed_weights(8, N, K, synth.STREAM_W2)
    Sg, Su = synth.scales(8, N, K), synth.scales(8, N, K, stream=synth.STREAM_S2)
    x, w = _xin(90 + M, M, K, 2.0), _norm_w(K, K, 0.5, 1.5)
    Y = _empty((M, N), torch.float16)
    ops.rmsnorm_mlp_gate_up_swiglu_int4(Y, f16_dev(x), to_dev(w), 1e-6, to_dev(Wg), f16_dev(Sg),
                                        to_dev(Wu), f16_dev(Su), M, N, K)
    xn = oracle.f16_to_f32(oracle.rmsnorm_f16(x, w, 1e-6))
    ref = oracle.swiglu_int4(xn, Wg, Sg, Wu, Su, M, N, K, nthreads=cpu_threads())
    print(check_f16_tol(to_np(Y), ref))
    assert expit is not None


@pytest.mark.parametrize("M", [9, 64])
def test_rmsnorm_fused_prefill_rows(M):
    """Beyond decode sizes the norm runs as its own kernel into a library
    buffer that the projection (GEMM path) reads; same results."""
    import torch
    ops = _ops()
    K, Ns = 1024, (256, 128)
    x, w = _xin(200 + M, M, K, 2.0), _norm_w(3, K, 0.5, 1.5)
    descs, refs, outs = [], [], []
    for p, N in enumerate(Ns):
        W, S = synth.packed_weights(80 + p, N, K), synth.scales(80 + p, N, K)
        refs.append(_ref_linear_after_norm(x, w, W, S, M, N, K))
        Y = _empty((M, N), torch.float16)
        outs.append(Y)
        descs.append(ops.FusedProjectionDesc(Y, to_dev(W), f16_dev(S), None, N))
    ops.rmsnorm_linear_int4_fused(f16_dev(x), to_dev(w), 1e-6, descs, 2, M, K)
    for Y, ref in zip(outs, refs):
        print(check_f16_tol(to_np(Y), ref))
    Wg, Wu = synth.packed_weights(8, 256, K), synth.packed_weights(8, 256, K, synth.STREAM_W2)
    Sg, Su = synth.scales(8, 256, K), synth.scales(8, 256, K, stream=synth.STREAM_S2)
    Y = _empty((M, 256), torch.float16)
    ops.rmsnorm_mlp_gate_up_swiglu_int4(Y, f16_dev(x), to_dev(w), 1e-6, to_dev(Wg), f16_dev(Sg),
                                        to_dev(Wu), f16_dev(Su), M, 256, K)
    xn = oracle.f16_to_f32(oracle.rmsnorm_f16(x, w, 1e-6))
    print(check_f16_tol(to_np(Y), oracle.swiglu_int4(xn, Wg, Sg, Wu, Su, M, 256, K)))


@pytest.mark.parametrize("M,N,K", [(1, 5120, 6144), (1, 5120, 17408), (4, 5120, 17408), (3, 5120, 6144),
                                   (4, 5120, 6144), (8, 333, 1024), (64, 1000, 2048), (512, 2048, 1024)])
def test_residual_epilogue_bit_exact(M, N, K):
    """residual += o_proj(X) in one launch gives the bits of o_proj into a
    fp16 buffer followed by add_inplace (forward.cpp:229 / 284-290)."""
    import torch
    ops = _ops()
    print("case", M, N, K, flush=True)
    W, S = synth.packed_weights(M + N, N, K), synth.scales(M + N, N, K)
    Xb = synth.activations(M + K, M, K)
    r0 = _xin(5 + M, M, N, 4.0)
    bias = np.linspace(-0.5, 0.5, N).astype(np.float32)
    dW, dS, dX = to_dev(W), f16_dev(S), f16_dev(Xb)
    for b in (None, bias):
        db = None if b is None else to_dev(b)
        Y = _empty((M, N), torch.float16)
        ops.linear_int4(Y, dX, dW, dS, db, M, N, K)
        want = f16_dev(r0)
        ops.add_inplace(want, Y, M * N)
        got = f16_dev(r0)
        ops.linear_int4_residual(got, dX, dW, dS, db, M, N, K)
        assert np.array_equal(_bits(got), _bits(want)), (M, N, K, b is None)
    # and within the usual bound of the oracle's fp32 result + residual
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, bias=bias,
                             nthreads=cpu_threads()) + oracle.f16_to_f32(r0)
    err = np.abs(oracle.f16_to_f32(_bits(got)) - ref).max()
    assert err <= 1e-2 * max(1.0, np.abs(ref).max() / 8), err
