"""Writes the golden fixtures in this folder (small .npz: inputs + expected).

Inputs are the reference's own integer-pattern known-answer cases
(tests/test_ops_oracle.cpp: linear f16 :707-775, fused :499-599, SwiGLU
:604-702, split-K small-N :389-466, argmax :911-947) at their original
shapes, with X drawn from the seeded SplitMix64 stream (the reference's
mt19937 + uniform_real_distribution mapping is implementation-defined).
Expected outputs come from the CPU oracle and are written only after an
independent float64 numpy evaluation agrees with them.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from tests import kat  # noqa: E402


def _check_linear(X, W, S, Y, bias=None):
    D = kat.dense_dequant_np(W, oracle.f16_to_f32(S))
    ref = X.astype(np.float64) @ D.T
    if bias is not None:
        ref = ref + bias
    assert np.abs(Y - ref).max() <= 1e-6 * max(1.0, np.abs(ref).max())


def linear_case(name, M, N, K, lo, hi, p=0, base=0.015, x_f16=False, seed=46):
    W = kat.pattern_weights(N, K, lo, hi, p)
    S = kat.pattern_scales(N, K, base=base, p=p)
    X = kat.uniform_x(seed, M, K)
    if x_f16:
        X = oracle.f16_to_f32(oracle.f32_to_f16(X))
    Y = oracle.linear_int4(X, W, S, M, N, K)
    _check_linear(X, W, S, Y)
    np.savez_compressed(os.path.join(HERE, name), kind="linear", shape=np.array([M, N, K]),
                        X=X, W=W, S=S, Y=Y, x_f16=x_f16)


def swiglu_case(name, M, N, K, x_f16=False, seed=47):
    from scipy.special import expit
    Wg, Wu = kat.pattern_weights(N, K, 2, 5), kat.pattern_weights(N, K, 4, 9)
    Sg, Su = kat.pattern_scales(N, K), kat.pattern_scales(N, K, base=0.020, shift=3)
    X = kat.uniform_x(seed, M, K)
    if x_f16:
        X = oracle.f16_to_f32(oracle.f32_to_f16(X))
    Y = oracle.swiglu_int4(X, Wg, Sg, Wu, Su, M, N, K)
    g = X.astype(np.float64) @ kat.dense_dequant_np(Wg, oracle.f16_to_f32(Sg)).T
    u = X.astype(np.float64) @ kat.dense_dequant_np(Wu, oracle.f16_to_f32(Su)).T
    assert np.abs(Y - g * expit(g) * u).max() < 1e-5
    np.savez_compressed(os.path.join(HERE, name), kind="swiglu", shape=np.array([M, N, K]),
                        X=X, W=Wg, S=Sg, W2=Wu, S2=Su, Y=Y, x_f16=x_f16)


def argmax_case(name):
    x = kat.uniform_x(48, 1, 8192, -100.0, 100.0)[0]
    x[1234] = 999.0
    x[5000] = 999.0          # tie: lower index wins
    x[77] = np.nan           # a NaN not at index 0 never wins
    y = oracle.argmax(x)
    assert y == 1234
    np.savez_compressed(os.path.join(HERE, name), kind="argmax", shape=np.array([1, 8192, 0]),
                        X=x, Y=np.int64(y))


def dequant_case(name, N=16, K=512):
    W = kat.pattern_weights(N, K, 3, 7)
    S = kat.pattern_scales(N, K)
    Y = oracle.dequant_int4(W, S, N, K)
    assert np.array_equal(Y.astype(np.float64), kat.dense_dequant_np(W, oracle.f16_to_f32(S)))
    np.savez_compressed(os.path.join(HERE, name), kind="dequant", shape=np.array([0, N, K]),
                        W=W, S=S, Y=Y)


if __name__ == "__main__":
    linear_case("linear_f16x_m1_n256_k512.npz", 1, 256, 512, 2, 5, x_f16=True)
    for p, n in enumerate((128, 64, 48, 48)):
        linear_case(f"fused_p{p}_m1_n{n}_k512.npz", 1, n, 512, 3, 7, p=p, seed=49)
    linear_case("splitk_m1_n48_k5120.npz", 1, 48, 5120, 5, 11, seed=50)
    swiglu_case("swiglu_m1_n256_k512.npz", 1, 256, 512)
    argmax_case("argmax_v8192.npz")
    dequant_case("dequant_n16_k512.npz")
    print("ok")
