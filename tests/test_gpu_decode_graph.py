"""A decode step's projection sequence captured in one HIP graph (the
reference captures its decode step as a SYCL graph,
src/targets/qwen3_8/decode_graph.cpp:93-175): input norm + fused QKV,
o_proj + residual, post-attention norm + gate/up SwiGLU, down + residual,
final norm + LM head argmax (forward.cpp:112-125, 229, 273-290, 293-308, 596).
Attention itself is out of scope: the q projection stands in for its output.

Every replay is checked bit for bit against the eager run of the same
sequence, with eager work and synchronisations between replays, at M = 1
(GEMV path, in-kernel norm) and M = 4 (small-batch path, norm kernel into a
library buffer)."""
import numpy as np
import pytest

import oracle
from tests.gpu_util import cpu_threads, f16_dev, to_dev, to_np
from xinfer_amd import synth

pytestmark = pytest.mark.gpu

H, QD, KVD, INTER, VOCAB = 1024, 1024, 256, 2816, 5000


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from xinfer_amd import _lib
    _lib.load_library()
    yield
    torch.cuda.synchronize()


class Layer:
    def __init__(self, seed):
        def w(i, n, k):
            return synth.packed_weights(seed * 10 + i, n, k), synth.scales(seed * 10 + i, n, k, 0.01)
        self.h = {}
        self.qkv = [w(0, QD, H), w(1, KVD, H), w(2, KVD, H)]
        self.o = w(3, H, QD)
        self.g, self.u = w(4, INTER, H), w(5, INTER, H)
        self.d = w(6, H, INTER)
        self.lm = w(7, VOCAB, H)
        rng = np.random.default_rng(seed)
        self.ln = [rng.uniform(0.5, 1.5, H).astype(np.float32) for _ in range(3)]

    def to_device(self):
        def dev(ws):
            return to_dev(ws[0]), f16_dev(ws[1])
        self.dqkv = [dev(x) for x in self.qkv]
        self.do, self.dg, self.du, self.dd, self.dlm = (dev(x) for x in (self.o, self.g, self.u, self.d, self.lm))
        self.dln = [to_dev(x) for x in self.ln]


def _buffers(M):
    import torch
    f16 = dict(dtype=torch.float16, device="cuda")
    return dict(q=torch.empty((M, QD), **f16), k=torch.empty((M, KVD), **f16), v=torch.empty((M, KVD), **f16),
                act=torch.empty((M, INTER), **f16), xn=torch.empty((M, H), **f16),
                ids=torch.empty((M,), dtype=torch.int32, device="cuda"),
                ws=torch.empty(M * H * 2, dtype=torch.uint8, device="cuda"),
                lm=torch.empty(max(8, ops_mod().lm_head_argmax_scratch_size(M, VOCAB, H)), dtype=torch.uint8,
                               device="cuda"))


def ops_mod():
    from xinfer_amd import ops
    return ops


def _step(ops, L, resid, b, M):
    """One decode step's projections; `resid` [M, H] is updated in place."""
    descs = [ops.FusedProjectionDesc(b[n], W, S, None, N)
             for n, (W, S), N in zip("qkv", L.dqkv, (QD, KVD, KVD))]
    ops.rmsnorm_linear_int4_fused(resid, L.dln[0], 1e-6, descs, 3, M, H, workspace=b["ws"])
    ops.linear_int4_residual(resid, b["q"], L.do[0], L.do[1], None, M, H, QD)
    ops.rmsnorm_mlp_gate_up_swiglu_int4(b["act"], resid, L.dln[1], 1e-6, L.dg[0], L.dg[1], L.du[0], L.du[1],
                                        M, INTER, H, workspace=b["ws"])
    ops.linear_int4_residual(resid, b["act"], L.dd[0], L.dd[1], None, M, H, INTER)
    ops.rmsnorm(b["xn"], resid, L.dln[2], M, H, 1e-6)
    ops.lm_head_argmax_int4(b["ids"], None, b["xn"], L.dlm[0], L.dlm[1], M, VOCAB, H, scratch=b["lm"])


def _oracle_step(L, x_bits, M):
    """The same sequence on the CPU oracle, fp16 roundings where the device
    stores fp16 (checks the eager run, which the replays must then match)."""
    t = cpu_threads()
    r = x_bits.copy()
    xn = oracle.f16_to_f32(oracle.rmsnorm_f16(r, L.ln[0], 1e-6))
    q = oracle.f32_to_f16(oracle.linear_int4(xn, *L.qkv[0], M, QD, H, nthreads=t).astype(np.float32))
    o = oracle.f32_to_f16(oracle.linear_int4(oracle.f16_to_f32(q), *L.o, M, H, QD, nthreads=t).astype(np.float32))
    r = oracle.add_inplace_f16(r, o)
    xn = oracle.f16_to_f32(oracle.rmsnorm_f16(r, L.ln[1], 1e-6))
    act = oracle.f32_to_f16(oracle.swiglu_int4(xn, *L.g, *L.u, M, INTER, H, nthreads=t).astype(np.float32))
    dn = oracle.f32_to_f16(oracle.linear_int4(oracle.f16_to_f32(act), *L.d, M, H, INTER, nthreads=t)
                           .astype(np.float32))
    r = oracle.add_inplace_f16(r, dn)
    xn = oracle.f16_to_f32(oracle.rmsnorm_f16(r, L.ln[2], 1e-6))
    logits = oracle.linear_int4(xn, *L.lm, M, VOCAB, H, nthreads=t)
    return r, logits


@pytest.mark.parametrize("M", [1, 4, 8])
def test_decode_step_graph_replays_match_eager(M):
    import torch
    from xinfer_amd import ops
    print("case M", M, flush=True)
    L = Layer(M)
    L.to_device()
    x0 = oracle.f32_to_f16(np.random.default_rng(M).normal(0, 1, (M, H)).astype(np.float32))
    b = _buffers(M)
    resid = f16_dev(x0)
    _step(ops, L, resid, b, M)  # eager
    torch.cuda.synchronize()
    want_r, want_ids = to_np(resid).copy(), to_np(b["ids"]).copy()

    # the eager run against the oracle: ids exact where the top-2 margin is
    # clear of the fp16 rounding of the intermediate activations
    ref_r, logits = _oracle_step(L, x0, M)
    err = np.abs(oracle.f16_to_f32(want_r) - oracle.f16_to_f32(ref_r)).max()
    assert err <= 5e-2, err
    for m in range(M):
        if oracle.top2_margin(logits[m]) > 1e-2:
            assert want_ids[m] == oracle.argmax(logits[m]), m

    start = f16_dev(x0)  # every replay starts from the step's input
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        resid.copy_(start)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            _step(ops, L, resid, b, M)
    torch.cuda.synchronize()
    other = _buffers(M)
    for rep in range(4):
        resid.copy_(start)
        b["ids"].fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(to_np(resid), want_r), rep
        assert np.array_equal(to_np(b["ids"]), want_ids), rep
        # eager work between replays (same shapes, other buffers, the current stream)
        r2 = f16_dev(x0[:1].repeat(M, 0))
        _step(ops, L, r2, other, M)
        torch.cuda.synchronize()
