"""Pins the CPU oracle (oracle/int4_oracle.c) before anything is checked
against it.  Each check is independent of the oracle's own code: exhaustive
tables, numpy's IEEE conversions, a vectorised numpy formulation, closed
forms on the reference's integer-pattern fixtures, and invariants chosen so a
dropped term, a wrong sign, a swapped nibble or a transposed operand fails.
"""
import numpy as np
import pytest

import oracle
from tests import kat


# ---------------------------------------------------------------- fp16 ----

def test_half_to_float_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    ours = oracle.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.isnan(ours[nan]).all()


def test_float_to_half_matches_numpy_rne():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    # every half value, the midpoints between neighbours (ties) and +-1 ulp
    h = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    h = h[np.isfinite(h)]
    hs = np.sort(np.unique(h))
    mids = ((hs[:-1].astype(np.float64) + hs[1:]) / 2).astype(np.float32)
    extra = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)),
                            np.nextafter(mids, np.float32(-np.inf)), h,
                            np.array([65504, 65519.99, 65520, 65536, 1e-8, 2**-25,
                                      2**-24, 3 * 2**-26, np.inf, -np.inf], np.float32)])
    f = np.concatenate([f, extra.astype(np.float32)])
    ours = oracle.f32_to_f16(f)
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16).view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.isnan(ours[nan].view(np.float16)).all()


# ------------------------------------------------------------- nibbles ----

def test_nibble_decode_all_bytes():
    for b in range(256):
        lo, hi = b & 15, b >> 4
        assert oracle.nibble(b, False) == (lo - 16 if lo >= 8 else lo)
        assert oracle.nibble(b, True) == (hi - 16 if hi >= 8 else hi)
        # two's complement reading of the same bits via int8 arithmetic shift
        assert oracle.nibble(b, False) == int((np.int8(np.uint8(b << 4 & 0xFF).view(np.int8)) >> 4))
        assert oracle.nibble(b, True) == int(np.uint8(b).view(np.int8) >> 4)


def test_dequant_matches_numpy_and_is_exact():
    N, K = 24, 384
    W = kat.pattern_weights(N, K, 3, 7)
    S = kat.pattern_scales(N, K)
    d = oracle.dequant_int4(W, S, N, K)
    ref = kat.dense_dequant_np(W, oracle.f16_to_f32(S))
    # q * s is exact in fp32 (4-bit x 11-bit significands)
    assert np.array_equal(d.astype(np.float64), ref)


def test_dequant_index_mapping_closed_form():
    # element (n, k) comes from byte n*K/2 + k/2, low nibble for even k
    N, K = 3, 256
    W = np.zeros((N, K // 2), np.uint8)
    W[1, 5] = 0x9A      # k=10 -> 0xA = -6, k=11 -> 0x9 = -7
    W[2, 127] = 0x71    # k=254 -> 1, k=255 -> 7
    S = oracle.f32_to_f16(np.array([[1.0, 1.0]] * 3, np.float32))
    S[2, 1] = oracle.f32_to_f16(np.array([0.5], np.float32))[0]
    d = oracle.dequant_int4(W, S, N, K)
    expect = np.zeros((N, K), np.float32)
    expect[1, 10], expect[1, 11] = -6, -7
    expect[2, 254], expect[2, 255] = 0.5, 3.5
    assert np.array_equal(d, expect)


# ------------------------------------------------------------ quantise ----

def test_quantize_closed_forms():
    G = 128
    s = np.float32(0.25)
    j = (np.arange(G) % 15 - 7).astype(np.float32)         # integers -7..7, amax = 7
    w = np.stack([j * s, -j * s, np.zeros(G, np.float32)])
    W, S = oracle.quantize_int4(w, G)
    sf = oracle.f16_to_f32(S)
    assert sf[0, 0] == np.float32(0.25) and sf[1, 0] == np.float32(0.25)
    assert sf[2, 0] == oracle.f16_to_f32(oracle.f32_to_f16(np.array([1e-8], np.float32)))[0]
    q = kat.dense_dequant_np(W, np.ones_like(sf))
    assert np.array_equal(q[0], j) and np.array_equal(q[1], -j) and not q[2].any()
    # byte packing: low nibble = even k, two's complement
    assert W[0, 0] == ((int(j[0]) & 15) | ((int(j[1]) & 15) << 4))


def test_quantize_round_half_even_and_roundtrip_bound():
    G = 128
    x = np.zeros(G, np.float32)
    x[0] = 7.0           # amax 7 -> scale exactly 1.0
    x[1], x[2], x[3], x[4] = 2.5, 3.5, -2.5, -0.5
    W, S = oracle.quantize_int4(x[None, :], G)
    q = kat.dense_dequant_np(W, np.ones((1, 1)))[0]
    assert list(q[:5]) == [7, 2, 4, -2, 0]       # half to even, like torch.round
    rng = np.random.default_rng(7)
    w = rng.standard_normal((16, 1024)).astype(np.float32) * 0.02
    W, S = oracle.quantize_int4(w, G)
    s16 = oracle.f16_to_f32(S).astype(np.float64)
    err = np.abs(oracle.dequant_int4(W, S, 16, 1024) - w)
    # converter bound (convert.py:387): |err| <= s/2, plus the fp16 rounding of s times |q| <= 8
    s32 = np.abs(w.reshape(16, -1, G)).max(-1) / 7
    bound = s32 / 2 + 8 * np.abs(s16 - s32) + 1e-9
    assert (err.reshape(16, -1, G) <= bound[..., None]).all()
    assert (np.abs(kat.dense_dequant_np(W, np.ones_like(s16))) <= 8).all()


# -------------------------------------------------------------- linear ----

@pytest.mark.parametrize("M,N,K", [(1, 7, 128), (3, 33, 640), (2, 64, 5120)])
def test_linear_matches_numpy_dense(M, N, K):
    from xinfer_amd import synth
    W = synth.packed_weights(11, N, K)
    S = synth.scales(11, N, K)
    X = kat.uniform_x(11, M, K)
    bias = np.linspace(-1, 1, N).astype(np.float32)
    Y = oracle.linear_int4(X, W, S, M, N, K, bias=bias)
    D = kat.dense_dequant_np(W, oracle.f16_to_f32(S))
    ref = X.astype(np.float64) @ D.T + bias
    assert np.abs(Y - ref).max() <= 1e-6 * max(1.0, np.abs(ref).max())
    # the multithreaded build computes the identical loop
    assert np.array_equal(Y, oracle.linear_int4(X, W, S, M, N, K, bias=bias, nthreads=4))


def test_linear_reference_pattern_closed_form():
    # reference fixture (test_ops_oracle.cpp:304-315) with X = 1: every 64-byte
    # group of a row sees each nibble value 4 times in both halves, and
    # sum_{v=0..15} int4(v) = -8, so each group sums to 2 * 4 * -8 = -64.
    M, N, K = 1, 40, 5120
    W = kat.pattern_weights(N, K, 3, 7)
    S = kat.pattern_scales(N, K)
    X = np.ones((M, K), np.float32)
    Y = oracle.linear_int4(X, W, S, M, N, K)
    expect = -64.0 * oracle.f16_to_f32(S).astype(np.float64).sum(1)
    assert np.allclose(Y[0], expect, rtol=0, atol=1e-5)


def test_linear_unit_vectors_pin_indexing():
    # X = e_k picks column k: Y[n] = int4(nibble k of row n) * S[n][k/128]
    M, N, K = 1, 5, 384
    W = kat.pattern_weights(N, K, 3, 7)
    S = kat.pattern_scales(N, K)
    sf = oracle.f16_to_f32(S)
    for k in (0, 1, 2, 127, 128, 255, 383):
        X = np.zeros((M, K), np.float32)
        X[0, k] = 1.0
        Y = oracle.linear_int4(X, W, S, M, N, K)
        for n in range(N):
            i = n * (K // 2) + k // 2
            v = ((i + 3) & 15) if k % 2 == 0 else ((i + 7) & 15)
            v = v - 16 if v >= 8 else v
            assert Y[0, n] == np.float32(v * np.float64(sf[n, k // 128]))


def test_linear_invariants():
    from xinfer_amd import synth
    M, N, K = 2, 16, 1024
    W = synth.packed_weights(3, N, K)
    S = synth.scales(3, N, K)
    X1, X2 = kat.uniform_x(3, M, K), kat.uniform_x(4, M, K)
    Y1 = oracle.linear_int4(X1, W, S, M, N, K).astype(np.float64)
    Y2 = oracle.linear_int4(X2, W, S, M, N, K).astype(np.float64)
    Y12 = oracle.linear_int4(X1 + X2, W, S, M, N, K).astype(np.float64)
    assert np.abs(Y12 - (Y1 + Y2)).max() < 1e-5
    assert not oracle.linear_int4(X1, W, np.zeros_like(S), M, N, K).any()
    # q = c everywhere: Y = c * sum_g s_g * sum_{k in g} x_k
    Wc = np.full((N, K // 2), 0xDD, np.uint8)            # both nibbles = -3
    Yc = oracle.linear_int4(X1, Wc, S, M, N, K).astype(np.float64)
    gs = X1.astype(np.float64).reshape(M, -1, 128).sum(-1)   # [M, ng]
    assert np.abs(Yc - (-3.0) * gs @ oracle.f16_to_f32(S).astype(np.float64).T).max() < 1e-5


def test_swiglu_closed_form():
    from scipy.special import expit
    from xinfer_amd import synth
    M, N, K = 2, 24, 512
    Wg, Wu = kat.pattern_weights(N, K, 2, 5), kat.pattern_weights(N, K, 4, 9)
    Sg, Su = kat.pattern_scales(N, K), kat.pattern_scales(N, K, base=0.020, shift=3)
    X = kat.uniform_x(5, M, K)
    Y = oracle.swiglu_int4(X, Wg, Sg, Wu, Su, M, N, K)
    g = (X.astype(np.float64) @ kat.dense_dequant_np(Wg, oracle.f16_to_f32(Sg)).T)
    u = (X.astype(np.float64) @ kat.dense_dequant_np(Wu, oracle.f16_to_f32(Su)).T)
    ref = g * expit(g) * u
    assert np.abs(Y - ref).max() < 1e-5
    assert synth is not None


# -------------------------------------------------------------- argmax ----

def test_argmax_first_max_semantics():
    rng = np.random.default_rng(48)
    x = rng.uniform(-100, 100, 248320).astype(np.float32)
    x[123456] = 999.0                               # test_ops_oracle.cpp:921-923
    assert oracle.argmax(x) == 123456 == int(np.argmax(x))
    x[200000] = 999.0                               # tie: the lower index wins
    assert oracle.argmax(x) == 123456
    x[5] = 1000.0
    assert oracle.argmax(x) == 5
    assert oracle.argmax(np.full(10, -np.inf, np.float32)) == 0
    assert oracle.argmax(np.zeros(1, np.float32)) == 0
    y = np.array([np.nan, 5, 7], np.float32)        # nothing is > NaN
    assert oracle.argmax(y) == 0
    y = np.array([1, np.nan, 7, np.nan], np.float32)
    assert oracle.argmax(y) == 2
    assert oracle.top2_margin(np.array([1, 3, 2], np.float32)) == 1.0


def test_golden_fixtures_reproduce():
    import glob
    import os
    files = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))
    assert files, "tests/golden/*.npz missing (run tests/golden/make_golden.py)"
    for f in files:
        z = np.load(f, allow_pickle=False)
        kind = str(z["kind"])
        M, N, K = (int(v) for v in z["shape"])
        if kind == "linear":
            Y = oracle.linear_int4(z["X"], z["W"], z["S"], M, N, K)
            assert np.array_equal(Y, z["Y"]), f
        elif kind == "swiglu":
            Y = oracle.swiglu_int4(z["X"], z["W"], z["S"], z["W2"], z["S2"], M, N, K)
            assert np.array_equal(Y, z["Y"]), f
        elif kind == "argmax":
            assert oracle.argmax(z["X"]) == int(z["Y"]), f
        elif kind == "dequant":
            assert np.array_equal(oracle.dequant_int4(z["W"], z["S"], N, K), z["Y"]), f


# ------------------------------------------------------ RMSNorm, add ----

def test_rmsnorm_matches_float64_formulation():
    """The reference's own check (tests/test_ops_oracle.cpp:50-101): hidden 5120,
    4 tokens, x ~ U(-1, 1), w ~ U(0, 2), sum of squares in double.  The fp16
    oracle output must be that value rounded, give or take one fp16 ulp (the
    FP32 sum's rounding can move a result across a rounding boundary)."""
    rng = np.random.default_rng(42)
    T, H, eps = 4, 5120, 1e-6
    x = oracle.f32_to_f16(rng.uniform(-1, 1, (T, H)).astype(np.float32))
    w = (rng.uniform(-1, 1, H) + 1.0).astype(np.float32)
    got = oracle.f16_to_f32(oracle.rmsnorm_f16(x, w, eps)).astype(np.float64)
    xf = oracle.f16_to_f32(x).astype(np.float64)
    inv = 1.0 / np.sqrt((xf * xf).sum(1, keepdims=True) / H + eps)
    ref = xf * inv * w
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert (np.abs(got - ref) <= ulp).all()
    # a row scaled by 4 normalises to the same output (scale invariance,
    # exact: powers of two commute with every rounding step)
    got4 = oracle.rmsnorm_f16(oracle.f32_to_f16(oracle.f16_to_f32(x) * 4), w, 0.0)
    assert np.array_equal(got4, oracle.rmsnorm_f16(x, w, 0.0))


def test_rmsnorm_closed_forms():
    H = 256
    w = np.linspace(0.5, 1.5, H).astype(np.float32)
    # constant row c: out = c / sqrt(c^2 + eps) * w
    for c in (0.5, -2.0, 3.0):
        x = oracle.f32_to_f16(np.full((1, H), c, np.float32))
        got = oracle.f16_to_f32(oracle.rmsnorm_f16(x, w, 1e-6))[0]
        assert np.allclose(got, np.sign(c) * w, rtol=1e-3)
    # one-hot row e_j * a: out_j = sqrt(H) * w_j (eps = 0), zeros elsewhere
    x = np.zeros((1, H), np.float32)
    x[0, 17] = 2.0
    got = oracle.f16_to_f32(oracle.rmsnorm_f16(oracle.f32_to_f16(x), w, 0.0))[0]
    assert got[17] == oracle.f16_to_f32(oracle.f32_to_f16(np.array([16.0 * w[17]], np.float32)))[0]
    assert (got[np.arange(H) != 17] == 0).all()
    # zero row with eps > 0 stays zero, rows are independent
    x = np.zeros((3, H), np.float32)
    x[1] = 1.0
    got = oracle.f16_to_f32(oracle.rmsnorm_f16(oracle.f32_to_f16(x), w, 1e-6))
    assert (got[0] == 0).all() and (got[2] == 0).all() and np.allclose(got[1], w, rtol=1e-3)


def test_add_inplace_matches_numpy_half():
    rng = np.random.default_rng(5)
    a = rng.integers(0, 65536, 200_000, dtype=np.uint32).astype(np.uint16)
    b = rng.integers(0, 65536, 200_000, dtype=np.uint32).astype(np.uint16)
    with np.errstate(all="ignore"):
        ref = (a.view(np.float16).astype(np.float32) + b.view(np.float16).astype(np.float32)).astype(np.float16)
    got = oracle.add_inplace_f16(a, b)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin], ref.view(np.uint16)[fin])
    assert np.isnan(got.view(np.float16)[np.isnan(ref)]).all()
