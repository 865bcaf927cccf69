"""GPU parity of the small-batch (2 <= M <= 8) decode path against the CPU
oracle: plain / fp32-out / bias, the split-K shapes (long K, short N) whose
k-slices are combined by the last block of each tile range, SwiGLU, fused
descriptors and the LM-head argmax.  Same bounds as the other parity tests:
fp16 outputs max abs <= 1e-2 and relative L2 <= 1e-3; fp32 outputs the
reference's 1e-4 bound (tests/test_ops_oracle.cpp:781); argmax ids exact."""
import numpy as np
import pytest

import oracle
from tests import kat
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


def _inputs(seed, M, N, K, sigma=0.02):
    W = synth.packed_weights(seed, N, K)
    S = synth.scales(seed, N, K, sigma)
    Xb = synth.activations(seed, M, K)
    return W, S, Xb


def _check_f32(y, ref):
    err = np.abs(y - ref).max()
    assert err <= 1e-4 * max(1.0, np.abs(ref).max()) and kat.rel_l2(y, ref) <= 1e-4, err
    return err


@pytest.mark.parametrize("M,N,K", [(2, 33, 128), (8, 17, 256), (3, 1000, 1536), (8, 4096, 5120),
                                   (6, 2000, 9984), (4, 5120, 17408), (7, 4100, 8192),
                                   (3, 5120, 6144), (4, 5120, 6144), (2, 2048, 4096), (4, 6144, 5120),
                                   (3, 48, 4096), (4, 2048, 5120), (4, 4096, 4096), (2, 12288, 5120),
                                   (2, 17410, 6144)])
def test_small_batch_shapes(M, N, K):
    import torch
    ops = _ops()
    print("case", M, N, K, flush=True)
    W, S, Xb = _inputs(M * 7 + N, M, N, K)
    dW, dS, dX = to_dev(W), f16_dev(S), f16_dev(Xb)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
    Y = _empty((M, N), torch.float16)
    ops.linear_int4(Y, dX, dW, dS, None, M, N, K)
    print(check_f16_tol(to_np(Y), ref))
    Yf = _empty((M, N), torch.float32)
    ops.linear_int4(Yf, dX, dW, dS, None, M, N, K)
    print(_check_f32(to_np(Yf), ref))


def test_split_k_repeatable_and_counters_reset():
    """Long-K shapes run as several k-slices per tile range; every call must
    give the same bits (slices are summed in slice order) and leave the
    arrival counters ready for the next call, also across shapes."""
    import torch
    ops = _ops()
    shapes = [(8, 1000, 17408), (2, 5120, 17408), (8, 1000, 17408), (5, 300, 25600)]
    first = {}
    for M, N, K in shapes:
        print("case", M, N, K, flush=True)
        W, S, Xb = _inputs(N + K, M, N, K)
        dW, dS, dX = to_dev(W), f16_dev(S), f16_dev(Xb)
        ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
        outs = []
        for _ in range(3):
            Y = _empty((M, N), torch.float32)
            ops.linear_int4(Y, dX, dW, dS, None, M, N, K)
            outs.append(to_np(Y))
        for y in outs[1:]:
            assert np.array_equal(y.view(np.uint32), outs[0].view(np.uint32))
        _check_f32(outs[0], ref)
        key = (M, N, K)
        if key in first:
            assert np.array_equal(first[key].view(np.uint32), outs[0].view(np.uint32))
        first[key] = outs[0]


def test_small_batch_bias_f32():
    import torch
    ops = _ops()
    M, N, K = 4, 777, 4096
    W, S, Xb = _inputs(12, M, N, K)
    bias = np.linspace(-3, 3, N).astype(np.float32)
    for K_ in (K, 17408):
        W, S, Xb = _inputs(12, M, N, K_)
        ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K_, bias=bias, nthreads=cpu_threads())
        Y = _empty((M, N), torch.float32)
        ops.linear_int4(Y, f16_dev(Xb), to_dev(W), f16_dev(S), to_dev(bias), M, N, K_)
        _check_f32(to_np(Y), ref)


@pytest.mark.parametrize("M,N,K", [(2, 17408, 5120), (3, 17408, 5120), (4, 17408, 5120), (8, 1000, 1024),
                                   (5, 640, 17408), (3, 16384, 4096), (3, 1024, 5120), (4, 1024, 6144)])
def test_small_batch_swiglu(M, N, K):
    import torch
    ops = _ops()
    print("case", M, N, K, flush=True)
    Wg, Wu = synth.packed_weights(3, N, K), synth.packed_weights(3, N, K, synth.STREAM_W2)
    Sg, Su = synth.scales(3, N, K), synth.scales(3, N, K, stream=synth.STREAM_S2)
    Xb = synth.activations(3, M, K)
    Y = _empty((M, N), torch.float16)
    ops.mlp_gate_up_swiglu_int4(Y, f16_dev(Xb), to_dev(Wg), f16_dev(Sg), to_dev(Wu), f16_dev(Su),
                                M, N, K)
    ref = oracle.swiglu_int4(oracle.f16_to_f32(Xb), Wg, Sg, Wu, Su, M, N, K, nthreads=cpu_threads())
    print(check_f16_tol(to_np(Y), ref))


@pytest.mark.parametrize("M", [2, 3, 8])
def test_small_batch_fused_descs(M):
    import torch
    ops = _ops()
    K, Ns = 2048, (384, 128, 64, 40)
    Xb = synth.activations(20 + M, M, K)
    X = oracle.f16_to_f32(Xb)
    descs, refs, outs = [], [], []
    for p, N in enumerate(Ns):
        W, S = synth.packed_weights(30 + p, N, K), synth.scales(30 + p, N, K)
        bias = np.linspace(-1, 1, N).astype(np.float32) if p == 1 else None
        refs.append(oracle.linear_int4(X, W, S, M, N, K, bias=bias))
        Y = _empty((M, N), torch.float16)
        outs.append(Y)
        descs.append(ops.FusedProjectionDesc(Y, to_dev(W), f16_dev(S),
                                             None if bias is None else to_dev(bias), N))
    ops.linear_int4_fused(f16_dev(Xb), descs, 4, M, K)
    for Y, ref in zip(outs, refs):
        print(check_f16_tol(to_np(Y), ref))


@pytest.mark.parametrize("M", [2, 4, 7])
def test_small_batch_lm_head_argmax(M):
    import torch
    ops = _ops()
    N, K = 50021, 5120
    W, S, Xb = _inputs(40 + M, M, N, K, 0.01)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    logits = _empty((M, N), torch.float32)
    ops.lm_head_argmax_int4(ids, logits, f16_dev(Xb), to_dev(W), f16_dev(S), M, N, K)
    got, lg = to_np(ids), to_np(logits)
    for m in range(M):
        print("row", m, "id", got[m], "margin", oracle.top2_margin(ref[m]))
        assert got[m] == oracle.argmax(ref[m]) == oracle.argmax(lg[m])
    _check_f32(lg, ref)


@pytest.mark.parametrize("M,N,K", [(3, 1001, 640), (8, 4099, 1152), (5, 33, 384), (2, 17, 128),
                                   (4, 3001, 17408), (8, 1000, 9216), (8, 2003, 17408)])
def test_small_batch_lm_head_odd_groups_ragged_rows(M, N, K):
    """LM head with odd group counts (a wave's last item has a padding
    group) and N not a multiple of 16 (the last tile's rows clamped), the
    winner planted in the last row: every logit and every id.  K = 17408 at
    M = 4 and K = 9216 at M = 8 stage X in two rounds; at M = 8, K = 17408
    the X slice exceeds LDS and the call takes the per-row path."""
    import torch
    ops = _ops()
    W, S, Xb = _inputs(60 + M, M, N, K, 0.01)
    # row N-1 = sign(X[0]) (quantized): the largest logit of row 0 at least
    Wq, Sq = oracle.quantize_int4(np.sign(oracle.f16_to_f32(Xb)[0])[None, :].astype(np.float32) * 0.3)
    W[N - 1], S[N - 1] = Wq[0], Sq[0]
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K)
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    logits = _empty((M, N), torch.float32)
    ops.lm_head_argmax_int4(ids, logits, f16_dev(Xb), to_dev(W), f16_dev(S), M, N, K)
    got, lg = to_np(ids), to_np(logits)
    _check_f32(lg, ref)
    for m in range(M):
        print("row", m, "id", got[m], "margin", oracle.top2_margin(ref[m]))
        assert got[m] == oracle.argmax(lg[m])
        if oracle.top2_margin(ref[m]) > 1e-3:
            assert got[m] == oracle.argmax(ref[m])
    assert got[0] == N - 1


@pytest.mark.parametrize("M,dc", [(8, 1.0), (4, -2.0), (8, 4.0), (1, 4.0), (1, -1.0)])
def test_small_batch_lm_head_dc_offset_activations(M, dc):
    """Activations with a large common offset (every x near dc): the FP32
    logits stay within the reference's 1e-4 bound and the ids match."""
    import torch
    ops = _ops()
    N, K = 4096, 5120
    W, S, _ = _inputs(90 + M, M, N, K, 0.01)
    rng = np.random.default_rng(90 + M)
    Xb = (dc + 0.05 * rng.standard_normal((M, K))).astype(np.float16).view(np.uint16)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    logits = _empty((M, N), torch.float32)
    ops.lm_head_argmax_int4(ids, logits, f16_dev(Xb), to_dev(W), f16_dev(S), M, N, K)
    got, lg = to_np(ids), to_np(logits)
    err = np.abs(lg - ref).max()
    print("max err", err, "bound", 1e-4 * max(1.0, np.abs(ref).max()), "rel_l2", kat.rel_l2(lg, ref))
    _check_f32(lg, ref)
    for m in range(M):
        assert got[m] == oracle.argmax(lg[m])
        if oracle.top2_margin(ref[m]) > 1e-3:
            assert got[m] == oracle.argmax(ref[m])


@pytest.mark.parametrize("M,N,K,dc", [(1, 4096, 5120, 4.0), (1, 4096, 17408, 2.0), (2, 4096, 5120, 4.0),
                                      (4, 2048, 6144, -3.0), (8, 2048, 5120, 4.0), (1, 48, 5120, 4.0)])
def test_linear_fp32_dc_offset_activations(M, N, K, dc):
    """fp32 outputs with activations near a common offset (the decode's
    folded bias terms grow with it) on every M = 1..8 route: within the
    reference's 1e-4 bound."""
    import torch
    ops = _ops()
    W, S, _ = _inputs(70 + M, M, N, K, 0.01)
    rng = np.random.default_rng(70 + M)
    Xb = (dc + 0.05 * rng.standard_normal((M, K))).astype(np.float16).view(np.uint16)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
    Y = _empty((M, N), torch.float32)
    ops.linear_int4(Y, f16_dev(Xb), to_dev(W), f16_dev(S), None, M, N, K)
    y = to_np(Y)
    print("max err", np.abs(y - ref).max(), "bound", 1e-4 * max(1.0, np.abs(ref).max()), "rel_l2", kat.rel_l2(y, ref))
    _check_f32(y, ref)


def test_small_batch_lm_head_ties_lowest_index():
    import torch
    ops = _ops()
    M, N, K = 3, 4096, 512
    W, S, Xb = _inputs(2, M, N, K)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K)
    want = []
    for m in range(M):
        b = int(np.argmax(ref[m]))
        dups = [(b + 1000 * (m + 1)) % N, (b + 2999) % N]
        for dst in dups:
            W[dst] = W[b]
            S[dst] = S[b]
        want.append(b)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K)
    ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    ops.lm_head_argmax_int4(ids, None, f16_dev(Xb), to_dev(W), f16_dev(S), M, N, K)
    got = to_np(ids)
    for m in range(M):
        assert got[m] == oracle.argmax(ref[m])


def test_lm_head_back_to_back_calls():
    """Consecutive LM-head calls with new inputs (GEMV and small-batch kernels,
    shared candidate scratch) each give the oracle's ids."""
    import torch
    ops = _ops()
    N, K = 20000, 2048
    W, S, _ = _inputs(77, 1, N, K, 0.01)
    dW, dS = to_dev(W), f16_dev(S)
    for M in (1, 4):
        for call in range(4):
            Xb = synth.activations(100 + 10 * M + call, M, K)
            ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
            ids = torch.full((M,), -1, dtype=torch.int32, device="cuda")
            ops.lm_head_argmax_int4(ids, None, f16_dev(Xb), dW, dS, M, N, K)
            got = to_np(ids)
            for m in range(M):
                assert got[m] == oracle.argmax(ref[m]), (M, call, m)


@pytest.mark.parametrize("M,N,K", [(9, 1000, 1024), (16, 4096, 5120), (17, 333, 2048), (33, 2000, 5120),
                                   (64, 5120, 17408), (48, 17408, 5120)])
def test_chunk_rows_m9_to_64(M, N, K):
    """Chunked-prefill row counts: 9..16 fill the small-batch kernel's 16-row
    MFMA tile (exact FP32 scaling: fp32 outputs within 1e-4), 17..64 run the
    MFMA GEMM (q*s rounded to fp16: fp32 outputs held to the fp16 bound).
    Plain fp16, fp32 with bias, residual."""
    import torch
    ops = _ops()
    print("case", M, N, K, flush=True)
    W, S, Xb = _inputs(M * 3 + N, M, N, K)
    dW, dS, dX = to_dev(W), f16_dev(S), f16_dev(Xb)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K, nthreads=cpu_threads())
    Y = _empty((M, N), torch.float16)
    ops.linear_int4(Y, dX, dW, dS, None, M, N, K)
    print(check_f16_tol(to_np(Y), ref))
    bias = np.linspace(-2, 2, N).astype(np.float32)
    Yf = _empty((M, N), torch.float32)
    ops.linear_int4(Yf, dX, dW, dS, to_dev(bias), M, N, K)
    if M <= 16:
        _check_f32(to_np(Yf), ref + bias)
    else:
        err = np.abs(to_np(Yf) - (ref + bias)).max()
        assert err <= 1e-2 and kat.rel_l2(to_np(Yf), ref + bias) <= 1e-3, err
    R = f16_dev(oracle.f32_to_f16(np.full((M, N), 0.5, np.float32)))
    ops.linear_int4_residual(R, dX, dW, dS, None, M, N, K)
    want = oracle.add_inplace_f16(oracle.f32_to_f16(np.full((M, N), 0.5, np.float32)), to_np(Y))
    assert np.array_equal(to_np(R), want)


@pytest.mark.parametrize("M", [12, 40])
def test_chunk_rows_swiglu_and_fused(M):
    import torch
    ops = _ops()
    K = 2048
    Xb = synth.activations(50 + M, M, K)
    X = oracle.f16_to_f32(Xb)
    N = 1500
    Wg, Wu = synth.packed_weights(5, N, K), synth.packed_weights(5, N, K, synth.STREAM_W2)
    Sg, Su = synth.scales(5, N, K), synth.scales(5, N, K, stream=synth.STREAM_S2)
    Y = _empty((M, N), torch.float16)
    ops.mlp_gate_up_swiglu_int4(Y, f16_dev(Xb), to_dev(Wg), f16_dev(Sg), to_dev(Wu), f16_dev(Su), M, N, K)
    print(check_f16_tol(to_np(Y), oracle.swiglu_int4(X, Wg, Sg, Wu, Su, M, N, K, nthreads=cpu_threads())))
    descs, refs, outs = [], [], []
    for p, n in enumerate((384, 128, 48)):
        W, S = synth.packed_weights(60 + p, n, K), synth.scales(60 + p, n, K)
        refs.append(oracle.linear_int4(X, W, S, M, n, K))
        Yd = _empty((M, n), torch.float16)
        outs.append(Yd)
        descs.append(ops.FusedProjectionDesc(Yd, to_dev(W), f16_dev(S), None, n))
    ops.linear_int4_fused(f16_dev(Xb), descs, 3, M, K)
    for Yd, ref in zip(outs, refs):
        print(check_f16_tol(to_np(Yd), ref))
