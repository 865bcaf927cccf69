"""GPU parity: the HIP kernels (through the C-ABI) against the CPU oracle on
identical inputs.  Tolerances: the reference's own per-case bounds for its
known-answer fixtures (tests/test_ops_oracle.cpp), and the BASELINE bound
for fp16 outputs (max abs <= 1e-2, relative L2 <= 1e-3); argmax ids and
dequantised weights bit-exact."""
import glob
import os

import numpy as np
import pytest

import oracle
from tests import kat
from tests.gpu_util import check_f16_tol, cpu_threads, f16_dev, to_dev, to_np
from xinfer_amd import synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


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


# ------------------------------------------- reference known-answer cases ----

def test_golden_linear_fixtures():
    import torch
    ops = _ops()
    for f in sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))):
        z = np.load(f, allow_pickle=False)
        if str(z["kind"]) != "linear":
            continue
        M, N, K = (int(v) for v in z["shape"])
        print("case", os.path.basename(f), flush=True)
        W, S = to_dev(z["W"]), f16_dev(z["S"])
        if bool(z["x_f16"]):
            X = f16_dev(oracle.f32_to_f16(z["X"]))
            Yh = _empty((M, N), torch.float16)
            ops.linear_int4(Yh, X, W, S, None, M, N, K)
            y = oracle.f16_to_f32(to_np(Yh))
            assert np.abs(y - z["Y"]).max() <= 5e-3          # test_ops_oracle.cpp:768
            Yf = _empty((M, N), torch.float32)
            ops.linear_int4(Yf, X, W, S, None, M, N, K)
            assert np.abs(to_np(Yf) - z["Y"]).max() <= 1e-4  # :781
        Yf = _empty((M, N), torch.float32)
        ops.linear_int4(Yf, to_dev(z["X"]), W, S, None, M, N, K)
        tol = 1e-3 if N == 48 else 1e-4                        # :459 split-K, :356
        assert np.abs(to_np(Yf) - z["Y"]).max() <= tol, f


def test_reference_linear_m2_k5120_n2048_f32_and_naive():
    import torch
    ops = _ops()
    M, N, K = 2, 2048, 5120                                   # test_ops_oracle.cpp:290-369
    W = kat.pattern_weights(N, K, 3, 7)
    S = kat.pattern_scales(N, K)
    X = kat.uniform_x(46, M, K)
    ref = oracle.linear_int4(X, W, S, M, N, K, nthreads=cpu_threads())
    dW, dS, dX = to_dev(W), f16_dev(S), to_dev(X)
    Y = _empty((M, N), torch.float32)
    ops.linear_int4(Y, dX, dW, dS, None, M, N, K)
    assert np.abs(to_np(Y) - ref).max() <= 1e-4
    Y2 = _empty((M, N), torch.float32)
    ops.linear_int4_naive(Y2, dX, dW, dS, None, M, N, K)
    assert np.abs(to_np(Y2) - ref).max() <= 1e-4


@pytest.mark.parametrize("xdtype", ["f32", "f16"])
def test_reference_fused_four_projections(xdtype):
    import torch
    ops = _ops()
    M, K, Ns = 1, 512, (128, 64, 48, 48)                      # test_ops_oracle.cpp:499-599
    X = kat.uniform_x(49, M, K)
    if xdtype == "f16":
        X = oracle.f16_to_f32(oracle.f32_to_f16(X))
        dX = f16_dev(oracle.f32_to_f16(X))
        ydt = torch.float16
    else:
        dX = to_dev(X)
        ydt = torch.float32
    descs, refs, outs = [], [], []
    for p, N in enumerate(Ns):
        W = kat.pattern_weights(N, K, 3, 7, p)
        S = kat.pattern_scales(N, K, p=p)
        refs.append(oracle.linear_int4(X, W, S, M, N, K))
        Y = _empty((M, N), ydt)
        outs.append(Y)
        descs.append(ops.FusedProjectionDesc(Y, to_dev(W), f16_dev(S), None, N))
    ops.linear_int4_fused(dX, descs, 4, M, K)
    for Y, ref in zip(outs, refs):
        if xdtype == "f16":
            assert np.abs(oracle.f16_to_f32(to_np(Y)) - ref).max() <= 5e-3
        else:
            assert np.abs(to_np(Y) - ref).max() <= 1e-4


@pytest.mark.parametrize("xdtype", ["f32", "f16"])
def test_reference_swiglu(xdtype):
    import torch
    ops = _ops()
    z = np.load(os.path.join(GOLDEN, "swiglu_m1_n256_k512.npz"), allow_pickle=False)
    M, N, K = (int(v) for v in z["shape"])
    X = z["X"]
    if xdtype == "f16":
        X = oracle.f16_to_f32(oracle.f32_to_f16(X))
        ref = oracle.swiglu_int4(X, z["W"], z["S"], z["W2"], z["S2"], M, N, K)
        Y = _empty((M, N), torch.float16)
        ops.mlp_gate_up_swiglu_int4(Y, f16_dev(oracle.f32_to_f16(X)), to_dev(z["W"]),
                                    f16_dev(z["S"]), to_dev(z["W2"]), f16_dev(z["S2"]), M, N, K)
        assert np.abs(oracle.f16_to_f32(to_np(Y)) - ref).max() <= 5e-3
    else:
        Y = _empty((M, N), torch.float32)
        ops.mlp_gate_up_swiglu_int4(Y, to_dev(X), to_dev(z["W"]), f16_dev(z["S"]),
                                    to_dev(z["W2"]), f16_dev(z["S2"]), M, N, K)
        assert np.abs(to_np(Y) - z["Y"]).max() <= 1e-4       # test_ops_oracle.cpp:695


def test_reference_argmax_planted():
    ops = _ops()
    x = kat.uniform_x(48, 1, 248320, -100.0, 100.0)[0]       # test_ops_oracle.cpp:911-947
    x[123456] = 999.0
    assert ops.argmax(to_dev(x), 248320) == oracle.argmax(x) == 123456
    z = np.load(os.path.join(GOLDEN, "argmax_v8192.npz"), allow_pickle=False)
    assert ops.argmax(to_dev(z["X"]), 8192) == int(z["Y"])


def test_dequant_bit_exact():
    import torch
    ops = _ops()
    for (N, K) in ((16, 512), (6144, 5120)):
        W = synth.packed_weights(0, N, K)
        S = synth.scales(0, N, K)
        out = _empty((N, K), torch.float32)
        ops.dequant_int4(out, to_dev(W), f16_dev(S), N, K)
        ref = oracle.dequant_int4(W, S, N, K)
        assert np.array_equal(to_np(out).view(np.uint32), ref.view(np.uint32))


# --------------------------------------------------- BASELINE configs ----

def _linear_case(M, N, K, seed=0, sigma=0.02, out="f16", sample_rows=None):
    import torch
    ops = _ops()
    W = synth.packed_weights(seed, N, K)
    S = synth.scales(seed, N, K, sigma)
    Xb = synth.activations(seed, M, K)
    X = oracle.f16_to_f32(Xb)
    ydt = torch.float16 if out == "f16" else torch.float32
    Y = _empty((M, N), ydt)
    ops.linear_int4(Y, f16_dev(Xb), to_dev(W), f16_dev(S), None, M, N, K)
    y = to_np(Y)
    rows = np.arange(M) if sample_rows is None else np.asarray(sample_rows)
    ref = oracle.linear_int4(X[rows], W, S, len(rows), N, K, nthreads=cpu_threads())
    y = y[rows]
    if out == "f16":
        return check_f16_tol(y, ref)
    # fp32 outputs: the reference's fp16-in/fp32-out bound (test_ops_oracle.cpp:781)
    err = np.abs(y - ref).max()
    assert err <= 1e-4 * max(1.0, np.abs(ref).max()) and kat.rel_l2(y, ref) <= 1e-4, err
    return err, kat.rel_l2(y, ref)


def test_cfg0_qproj_m1():
    print(_linear_case(1, 6144, 5120))


def test_north_star_gemv_m1_n34816():
    print(_linear_case(1, 34816, 5120))


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_cfg2_down_proj_small_batch(M):
    print(_linear_case(M, 5120, 17408))


@pytest.mark.parametrize("M", [3, 5, 6, 7])
def test_ragged_batch(M):
    print(_linear_case(M, 1000, 1536, seed=M))


@pytest.mark.parametrize("N,K", [(1, 128), (3, 384), (7, 640), (48, 5120), (129, 1152), (513, 3200)])
def test_ragged_shapes_m1(N, K):
    print(_linear_case(1, N, K, seed=N))
    print(_linear_case(2, N, K, seed=N, out="f32"))


# Long K: the M <= 2 GEMV stages X in more than 64 KB of LDS (one 8-wave
# block per CU); past three staging rounds it stages in a loop; past 159 KB
# M = 2 runs the small-batch kernel.
@pytest.mark.parametrize("M,N,K", [(1, 520, 40960), (1, 300, 74240), (2, 260, 30720), (2, 200, 40960)])
def test_long_k_large_lds(M, N, K):
    print(_linear_case(M, N, K, seed=K % 97))


def test_long_k_swiglu_m1():
    import torch
    ops = _ops()
    M, N, K = 1, 264, 40960
    # scales |N(0, 0.005)|/7 keep |y| below 4 at this K (with config 1's 0.02
    # the outputs reach ~36, where fp16 spacing alone exceeds the 1e-2 bound)
    W = synth.packed_weights(3, 2 * N, K)
    S = synth.scales(3, 2 * N, K, 0.005)
    Xb = synth.activations(3, M, K)
    dW, dS = to_dev(W), f16_dev(S)
    Y = _empty((M, N), torch.float16)
    ops.mlp_gate_up_swiglu_int4(Y, f16_dev(Xb), dW[:N], dS[:N], dW[N:], dS[N:], M, N, K)
    ref = oracle.swiglu_int4(oracle.f16_to_f32(Xb), W[:N], S[:N], W[N:], S[N:], M, N, K,
                             nthreads=cpu_threads())
    print(check_f16_tol(to_np(Y), ref))


# M = 1 launches of at least 32768 rows (K = 4096..6144) run the row-pair
# kernel: bias, fp32 output, the residual epilogue, several descriptors, and
# an odd N (left to the GEMV).
@pytest.mark.parametrize("N,K,out", [(32768, 4096, "f16"), (34816, 6144, "f32"), (33000, 5120, "f16"),
                                     (32769, 5120, "f16")])
def test_pair_kernel_shapes(N, K, out):
    print(_linear_case(1, N, K, seed=N % 89, out=out))


def test_pair_kernel_bias_residual_descs():
    import torch
    ops = _ops()
    K = 5120
    Xb = synth.activations(21, 1, K)
    X = oracle.f16_to_f32(Xb)
    # bias + residual on one 32768-row projection
    N = 32768
    W, S = synth.packed_weights(21, N, K), synth.scales(21, N, K)
    bias = np.linspace(-0.5, 0.5, N).astype(np.float32)
    r0 = synth.activations(22, 1, N)
    R = f16_dev(r0)
    ops.linear_int4_residual(R, f16_dev(Xb), to_dev(W), f16_dev(S), to_dev(bias), 1, N, K)
    ref = oracle.linear_int4(X, W, S, 1, N, K, bias=bias, nthreads=cpu_threads())
    print(check_f16_tol(to_np(R), oracle.f16_to_f32(r0).astype(np.float64) + ref))
    # four descriptors, 33792 rows together, pair boundaries inside each
    Ns = (12288, 10240, 6146, 5118)
    descs, outs, refs = [], [], []
    for p, Np in enumerate(Ns):
        Wp, Sp = synth.packed_weights(30 + p, Np, K), synth.scales(30 + p, Np, K)
        refs.append(oracle.linear_int4(X, Wp, Sp, 1, Np, K, nthreads=cpu_threads()))
        Y = _empty((1, Np), torch.float16)
        outs.append(Y)
        descs.append(ops.FusedProjectionDesc(Y, to_dev(Wp), f16_dev(Sp), None, Np))
    ops.linear_int4_fused(f16_dev(Xb), descs, 4, 1, K)
    for Y, ref in zip(outs, refs):
        print(check_f16_tol(to_np(Y), ref))


@pytest.mark.parametrize("N,K", [(8194, 5120), (9000, 4096), (12290, 6144), (10000, 5120)])
def test_pair_plain_leftover_rows(N, K):
    """M = 1 plain launches on the row-pair kernel whose pairs do not divide
    over the waves (one leftover pair, 404, 904 of them): fp16 plain, fp32
    with bias, fp16 residual; every output against the oracle."""
    import torch
    ops = _ops()
    W, S = synth.packed_weights(N, N, K), synth.scales(N, N, K)
    Xb = synth.activations(N, 1, K)
    X = oracle.f16_to_f32(Xb)
    bias = kat.uniform_x(N + 1, 1, N, -1, 1)[0]
    dX, dW, dS = f16_dev(Xb), to_dev(W), f16_dev(S)
    ref = oracle.linear_int4(X, W, S, 1, N, K, nthreads=cpu_threads())
    Y = _empty((1, N), torch.float16)
    ops.linear_int4(Y, dX, dW, dS, None, 1, N, K)
    print(check_f16_tol(to_np(Y), ref))
    Yf = _empty((1, N), torch.float32)
    ops.linear_int4(Yf, dX, dW, dS, to_dev(bias), 1, N, K)
    reff = oracle.linear_int4(X, W, S, 1, N, K, bias=bias, nthreads=cpu_threads())
    yf = to_np(Yf)
    assert np.abs(yf - reff).max() <= 1e-4 * max(1.0, np.abs(reff).max()) and kat.rel_l2(yf, reff) <= 1e-4
    r0 = synth.activations(N + 2, 1, N)
    R = f16_dev(r0)
    ops.linear_int4_residual(R, dX, dW, dS, None, 1, N, K)
    print(check_f16_tol(to_np(R), oracle.f16_to_f32(r0).astype(np.float64) + ref))


def test_pair_plain_leftover_rows_la_in_proj():
    """The fused LA in_proj (10240 + 6144 + 48 + 48 rows, 8240 pairs over
    1024 waves: 48 leftover pairs) on the row-pair kernel, every output
    against the oracle."""
    import torch
    ops = _ops()
    K = 5120
    Xb = synth.activations(5, 1, K)
    X = oracle.f16_to_f32(Xb)
    descs, outs, refs = [], [], []
    for p, Np in enumerate((10240, 6144, 48, 48)):
        Wp, Sp = synth.packed_weights(50 + p, Np, K), synth.scales(50 + p, Np, K)
        refs.append(oracle.linear_int4(X, Wp, Sp, 1, Np, K, nthreads=cpu_threads()))
        Y = _empty((1, Np), torch.float16)
        outs.append(Y)
        descs.append(ops.FusedProjectionDesc(Y, to_dev(Wp), f16_dev(Sp), None, Np))
    ops.linear_int4_fused(f16_dev(Xb), descs, 4, 1, K)
    for Y, ref in zip(outs, refs):
        print(check_f16_tol(to_np(Y), ref))


@pytest.mark.parametrize("N,K", [(4096, 8192), (6144, 24576), (4100, 7168), (5120, 17408)])
def test_pair_kernel_long_k(N, K):
    """M = 1 beyond K = 6144: a row pair's 1 KB pieces split over four
    waves (parts of P / 4 pieces).  fp16 plain, fp32 with bias, fp16
    residual, and two descriptors in one launch."""
    import torch
    ops = _ops()
    print("case", N, K, flush=True)
    Xb = synth.activations(40 + K // 1024, 1, K)
    X = oracle.f16_to_f32(Xb)
    W, S = synth.packed_weights(41, N, K), synth.scales(41, N, K)
    dW, dS, dX = to_dev(W), f16_dev(S), f16_dev(Xb)
    ref = oracle.linear_int4(X, W, S, 1, N, K, nthreads=cpu_threads())
    Y = _empty((1, N), torch.float16)
    ops.linear_int4(Y, dX, dW, dS, None, 1, N, K)
    print(check_f16_tol(to_np(Y), ref))
    bias = np.linspace(-1, 1, N).astype(np.float32)
    Yf = _empty((1, N), torch.float32)
    ops.linear_int4(Yf, dX, dW, dS, to_dev(bias), 1, N, K)
    assert np.abs(to_np(Yf) - (ref + bias)).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    r0 = synth.activations(42, 1, N)
    R = f16_dev(r0)
    ops.linear_int4_residual(R, dX, dW, dS, None, 1, N, K)
    print(check_f16_tol(to_np(R), oracle.f16_to_f32(r0).astype(np.float64) + ref))
    # two descriptors (pair boundaries inside each)
    Ns = (N // 2 + 2, N // 2 - 2)
    descs, outs, refs = [], [], []
    for q, Nq in enumerate(Ns):
        Wq, Sq = synth.packed_weights(50 + q, Nq, K), synth.scales(50 + q, Nq, K)
        refs.append(oracle.linear_int4(X, Wq, Sq, 1, Nq, K, nthreads=cpu_threads()))
        Yq = _empty((1, Nq), torch.float16)
        outs.append(Yq)
        descs.append(ops.FusedProjectionDesc(Yq, to_dev(Wq), f16_dev(Sq), None, Nq))
    ops.linear_int4_fused(dX, descs, 2, 1, K)
    for Yq, refq in zip(outs, refs):
        print(check_f16_tol(to_np(Yq), refq))


def test_bias_is_added():
    import torch
    ops = _ops()
    M, N, K = 2, 300, 1024
    W, S = synth.packed_weights(5, N, K), synth.scales(5, N, K)
    Xb = synth.activations(5, M, K)
    bias = np.linspace(-2, 2, N).astype(np.float32)
    Y = _empty((M, N), torch.float32)
    ops.linear_int4(Y, f16_dev(Xb), to_dev(W), f16_dev(S), to_dev(bias), M, N, K)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, bias=bias)
    assert np.abs(to_np(Y) - ref).max() <= 1e-4


def test_cfg1_fused_gate_up_swiglu():
    import torch
    ops = _ops()
    M, N, K = 1, 17408, 5120
    # one interleaved allocation of 2N rows: W_up = W_gate + N*K/2
    Wall = synth.packed_weights(0, 2 * N, K)
    Sall = synth.scales(0, 2 * N, K)
    Xb = synth.activations(0, M, K)
    dW, dS = to_dev(Wall), f16_dev(Sall)
    Y = _empty((M, N), torch.float16)
    ops.mlp_gate_up_swiglu_int4(Y, f16_dev(Xb), dW[:N], dS[:N], dW[N:], dS[N:], M, N, K)
    ref = oracle.swiglu_int4(oracle.f16_to_f32(Xb), Wall[:N], Sall[:N], Wall[N:], Sall[N:],
                             M, N, K, nthreads=cpu_threads())
    print(check_f16_tol(to_np(Y), ref))


@pytest.mark.parametrize("N,K", [(17406, 5120), (16386, 5120), (8194, 4096), (16384, 6144), (12290, 6144)])
def test_pair_swiglu_leftover_split(N, K):
    """M = 1 gate/up SwiGLU on the row-pair kernel when the pairs do not
    divide over the waves: the leftover pairs' gate and up halves go to two
    waves of one block and meet in LDS (an odd leftover count, a single
    leftover pair, none); every output against the oracle."""
    import torch
    ops = _ops()
    M = 1
    Wall = synth.packed_weights(N, 2 * N, K)
    Sall = synth.scales(N, 2 * N, K)
    Xb = synth.activations(N, M, K)
    dW, dS = to_dev(Wall), f16_dev(Sall)
    Y = _empty((M, N), torch.float16)
    ops.mlp_gate_up_swiglu_int4(Y, f16_dev(Xb), dW[:N], dS[:N], dW[N:], dS[N:], M, N, K)
    ref = oracle.swiglu_int4(oracle.f16_to_f32(Xb), Wall[:N], Sall[:N], Wall[N:], Sall[N:],
                             M, N, K, nthreads=cpu_threads())
    print(check_f16_tol(to_np(Y), ref))


@pytest.mark.parametrize("M", [1, 8])
def test_cfg3_lm_head_argmax(M):
    import torch
    ops = _ops()
    N, K = 151936, 5120
    W, S = synth.packed_weights(0, N, K), synth.scales(0, N, K, 0.01)
    Xb = synth.activations(0, M, K)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
    dX, dW, dS = f16_dev(Xb), to_dev(W), f16_dev(S)
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    logits = _empty((M, N), torch.float32)
    ops.lm_head_argmax_int4(ids, logits, dX, dW, dS, M, N, K)
    got = to_np(ids)
    lg = to_np(logits)
    for m in range(M):
        margin = oracle.top2_margin(ref[m])
        print("row", m, "id", got[m], "margin", margin)
        assert got[m] == oracle.argmax(ref[m])
        assert got[m] == oracle.argmax(lg[m])
    assert np.abs(lg - ref).max() <= 1e-4 * max(1.0, np.abs(ref).max())
    assert kat.rel_l2(lg, ref) <= 1e-4
    # without storing logits, same ids; batched standalone argmax agrees
    ids2 = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    ops.lm_head_argmax_int4(ids2, None, dX, dW, dS, M, N, K)
    assert np.array_equal(to_np(ids2), got)
    out64 = torch.full((M,), -1, dtype=torch.int64, device="cuda")
    ops.argmax_rows(logits, out64, N, M)
    assert np.array_equal(to_np(out64), got.astype(np.int64))


def test_cfg4_prefill_m512_sampled_rows():
    print(_linear_case(512, 17408, 5120, sample_rows=[0, 1, 77, 255, 256, 300, 510, 511]))


def test_cfg4_prefill_m512_full_row_tile():
    """Config 4 on the prefill GEMM (fp16 output, B = fp16(q*s)): every
    output of the first 256-row block of M (one full row tile across all
    17408 columns, i.e. 128 column tiles) plus the first and last rows of
    the second, against the double-accumulate oracle."""
    print(_linear_case(512, 17408, 5120, sample_rows=list(range(256)) + [256, 383, 511]))


# --------------------------------------------------------- argmax edges ----

def test_argmax_edges():
    import torch
    ops = _ops()
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    cases = [
        np.array([3, 7, 7, 1], np.float32),
        np.array([nan, 5, 9], np.float32),
        np.array([1, nan, 9, nan], np.float32),
        np.array([-inf, -inf, -inf], np.float32),
        np.array([-inf, nan, nan], np.float32),
        np.array([nan, inf, 3], np.float32),
        np.array([2.0], np.float32),
    ]
    big = kat.uniform_x(9, 1, 4096 * 3 + 17, -5, 5)[0]
    big[4096 * 2 + 3] = 50.0
    big[4096 + 1] = 50.0
    cases.append(big)
    for x in cases:
        assert ops.argmax(to_dev(x), x.size) == oracle.argmax(x), x[:8]
    # batched rows, V not a multiple of the block span
    R, V = 5, 10007
    xs = kat.uniform_x(10, R, V, -1, 1)
    for r in range(R):
        xs[r, (r * 997) % V] = 3.0
    out = torch.full((R,), -1, dtype=torch.int64, device="cuda")
    scratch = torch.empty(ops.argmax_scratch_size(V, R), dtype=torch.uint8, device="cuda")
    ops.argmax_rows(to_dev(xs), out, V, R, scratch)
    assert list(to_np(out)) == [oracle.argmax(xs[r]) for r in range(R)]
    # empty vocab: token 0 (src/ops/sampling.cpp:17)
    assert ops.argmax(to_dev(np.zeros(4, np.float32)), 0) == 0


def test_lm_head_argmax_ties_lowest_index():
    import torch
    ops = _ops()
    # duplicate rows in W give bit-identical logits: the lower row index must win
    M, N, K = 1, 4096, 512
    W, S = synth.packed_weights(2, N, K), synth.scales(2, N, K)
    Xb = synth.activations(2, M, K)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K)
    b = int(np.argmax(ref[0]))
    for dst in (b + 1000) % N, (b + 3000) % N:
        W[dst] = W[b]
        S[dst] = S[b]
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    ops.lm_head_argmax_int4(ids, None, f16_dev(Xb), to_dev(W), f16_dev(S), M, N, K)
    assert int(to_np(ids)[0]) == min(b, (b + 1000) % N, (b + 3000) % N)


def test_noop_shapes_leave_output_untouched():
    import torch
    ops = _ops()
    Y = torch.full((4,), 7.0, dtype=torch.float16, device="cuda")
    X = torch.zeros(128, dtype=torch.float16, device="cuda")
    W = torch.zeros(64, dtype=torch.uint8, device="cuda")
    S = torch.zeros(1, dtype=torch.float16, device="cuda")
    ops.linear_int4(Y, X, W, S, None, 0, 4, 128)
    ops.linear_int4(Y, X, W, S, None, 1, 0, 128)
    torch.cuda.synchronize()
    assert (Y == 7.0).all()


# ------------------------------------------------ prefill GEMM (M > 8) ----

@pytest.mark.parametrize("M,N,K", [(9, 64, 128), (128, 272, 1024), (130, 300, 384), (512, 1000, 1024),
                                   (256, 4352, 2048), (33, 17, 3072), (1000, 64, 1024)])
def test_prefill_gemm_shapes(M, N, K):
    print(_linear_case(M, N, K, seed=M + N))


@pytest.mark.parametrize("M,N,K", [(128, 272, 1024), (130, 300, 384 * 8), (512, 4352, 5120)])
def test_prefill_gemm_f32_out_exact(M, N, K):
    """fp32-output GEMM (exact q, FP32 group scale), incl. a leftover tile."""
    print(_linear_case(M, N, K, seed=M + 3, out="f32"))


def test_prefill_gemm_f32_out_and_bias():
    import torch
    ops = _ops()
    M, N, K = 200, 520, 2048
    W, S = synth.packed_weights(8, N, K), synth.scales(8, N, K)
    Xb = synth.activations(8, M, K)
    bias = np.linspace(-1, 1, N).astype(np.float32)
    Y = _empty((M, N), torch.float32)
    ops.linear_int4(Y, f16_dev(Xb), to_dev(W), f16_dev(S), to_dev(bias), M, N, K)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, bias=bias, nthreads=cpu_threads())
    # fp32 output: exact q, FP32 group scale, the reference's fp32-out bound
    # (tests/test_ops_oracle.cpp:781)
    err = np.abs(to_np(Y) - ref).max()
    assert err <= 1e-4 * max(1.0, np.abs(ref).max()) and kat.rel_l2(to_np(Y), ref) <= 1e-4, err


@pytest.mark.parametrize("M,N,K", [(16, 256, 512), (40, 200, 1024), (512, 17408 // 8, 5120)])
def test_prefill_swiglu(M, N, K):
    import torch
    ops = _ops()
    Wg, Wu = synth.packed_weights(1, N, K), synth.packed_weights(1, N, K, synth.STREAM_W2)
    Sg, Su = synth.scales(1, N, K), synth.scales(1, N, K, stream=synth.STREAM_S2)
    Xb = synth.activations(1, M, K)
    Y = _empty((M, N), torch.float16)
    ops.mlp_gate_up_swiglu_int4(Y, f16_dev(Xb), to_dev(Wg), f16_dev(Sg), to_dev(Wu), f16_dev(Su),
                                M, N, K)
    rows = np.arange(0, M, max(1, M // 16))
    ref = oracle.swiglu_int4(oracle.f16_to_f32(Xb)[rows], Wg, Sg, Wu, Su, len(rows), N, K,
                             nthreads=cpu_threads())
    print(check_f16_tol(to_np(Y)[rows], ref))


@pytest.mark.parametrize("out", ["f16", "f32"])
@pytest.mark.parametrize("M,N,K", [(4, 33, 384), (8, 17, 640), (5, 31, 1152), (3, 9, 384)])
def test_small_batch_odd_groups_last_scale(M, N, K, out):
    """Small-batch shapes whose waves hold an odd number of 128-k groups:
    each row's last item pairs a real group with a padding group, and the
    scale array's last scale comes through the clamped 4-byte load (the
    dword read 2 bytes lower, its upper half used)."""
    print(_linear_case(M, N, K, seed=N, out=out))


@pytest.mark.parametrize("M,N,K", [(4, 33, 384), (8, 17, 640)])
def test_small_batch_swiglu_odd_groups(M, N, K):
    import torch
    ops = _ops()
    Wg, Wu = synth.packed_weights(2, N, K), synth.packed_weights(2, N, K, synth.STREAM_W2)
    Sg, Su = synth.scales(2, N, K), synth.scales(2, N, K, stream=synth.STREAM_S2)
    Xb = synth.activations(2, M, K)
    Y = _empty((M, N), torch.float16)
    ops.mlp_gate_up_swiglu_int4(Y, f16_dev(Xb), to_dev(Wg), f16_dev(Sg), to_dev(Wu), f16_dev(Su),
                                M, N, K)
    ref = oracle.swiglu_int4(oracle.f16_to_f32(Xb), Wg, Sg, Wu, Su, M, N, K, nthreads=cpu_threads())
    print(check_f16_tol(to_np(Y), ref))


def test_prefill_fused_descs_m64():
    import torch
    ops = _ops()
    M, K, Ns = 64, 2048, (384, 128, 64)
    Xb = synth.activations(4, M, K)
    X = oracle.f16_to_f32(Xb)
    descs, refs, outs = [], [], []
    for p, N in enumerate(Ns):
        W, S = synth.packed_weights(10 + p, N, K), synth.scales(10 + p, N, K)
        refs.append(oracle.linear_int4(X, W, S, M, N, K))
        Y = _empty((M, N), torch.float16)
        outs.append(Y)
        descs.append(ops.FusedProjectionDesc(Y, to_dev(W), f16_dev(S), None, N))
    ops.linear_int4_fused(f16_dev(Xb), descs, 3, M, K)
    for Y, ref in zip(outs, refs):
        check_f16_tol(to_np(Y), ref)


# Decode-shape plans of the small-batch planner and the GEMV planner: gate/up
# SwiGLU at M = 4 (256 blocks, four waves per tile) and M = 8 (one 80 KB X
# slice), fused QKV at M = 2 (GEMV, one block per CU) and M = 8 (one slice),
# the linear-attention in_proj at M = 4 / 8,
# and a 12-row chunk (two 80 KB slices, 8-wave blocks), all at K = 5120.
@pytest.mark.parametrize("M", [4, 8])
def test_planned_swiglu_decode_shape(M):
    import torch
    ops = _ops()
    N, K = 17408, 5120
    W = synth.packed_weights(50 + M, 2 * N, K)
    S = synth.scales(50 + M, 2 * N, K, 0.01)
    Xb = synth.activations(50 + M, M, K)
    dW, dS = to_dev(W), f16_dev(S)
    Y = _empty((M, N), torch.float16)
    ops.mlp_gate_up_swiglu_int4(Y, f16_dev(Xb), dW[:N], dS[:N], dW[N:], dS[N:], M, N, K)
    ref = oracle.swiglu_int4(oracle.f16_to_f32(Xb), W[:N], S[:N], W[N:], S[N:], M, N, K,
                             nthreads=cpu_threads())
    print(check_f16_tol(to_np(Y), ref))


# (the linear-attention in_proj's two 48-row descriptors get at least one
# range each from the balanced plan)
@pytest.mark.parametrize("M,Ns", [(2, (12288, 1024, 1024)), (8, (12288, 1024, 1024)),
                                  (4, (10240, 6144, 48, 48)), (8, (10240, 6144, 48, 48))])
def test_planned_fused_decode_shape(M, Ns):
    import torch
    ops = _ops()
    K = 5120
    Xb = synth.activations(60 + M, M, K)
    X = oracle.f16_to_f32(Xb)
    descs, outs, refs = [], [], []
    for p, Np in enumerate(Ns):
        W, S = synth.packed_weights(61 + p, Np, K), synth.scales(61 + p, Np, K)
        refs.append(oracle.linear_int4(X, W, S, M, Np, K, nthreads=cpu_threads()))
        Y = _empty((M, Np), torch.float16)
        outs.append(Y)
        descs.append(ops.FusedProjectionDesc(Y, to_dev(W), f16_dev(S), None, Np))
    ops.linear_int4_fused(f16_dev(Xb), descs, len(Ns), M, K)
    for Y, ref in zip(outs, refs):
        print(check_f16_tol(to_np(Y), ref))


def test_planned_chunk_rows_m12():
    print(_linear_case(12, 17408, 5120, seed=12, sigma=0.01))
