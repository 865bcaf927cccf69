"""GPU tests of the .xinfer device path: the GPU CRC-64 against the oracle,
section uploads verified on the device, and an end-to-end load of an INT4
projection from a file (load_linear, weights.cpp:252-303) feeding the HIP
GEMV, checked against the CPU oracle."""
import json
import os

import numpy as np
import pytest

import oracle
from tests.gpu_util import check_f16_tol, f16_dev, to_np
from xinfer_amd import _lib, artifact, synth
from xinfer_amd.artifact import ArtifactError, ArtifactReader, ArtifactWriter, SectionType

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    _lib.load_library()
    yield
    torch.cuda.synchronize()


def test_crc64_device_sizes():
    import torch
    # tails 0..15, one unit, one block, partial front padding, > 1024 blocks (q > 1)
    sizes = [0, 1, 15, 16, 17, 511, 512, 513, 4095, (128 << 10) - 1, 128 << 10, (128 << 10) + 16,
             (1 << 20) + 5, (200 << 20) + 3]
    rng = np.random.default_rng(7)
    for n in sizes:
        print("size", n, flush=True)
        host = rng.integers(0, 256, max(n, 1), dtype=np.uint8)[:n]
        dev = torch.from_numpy(host.copy()).cuda() if n else torch.empty(16, dtype=torch.uint8, device="cuda")
        got = artifact.crc64_device(dev, n)
        want = oracle.crc64(host.tobytes()) if n < (8 << 20) else artifact.crc64(host.tobytes())
        assert got == want, n
    # the library CRC of the big buffer is itself pinned to the oracle on the CPU tests


def test_crc64_device_caller_scratch_and_stream():
    import ctypes
    import torch
    L = _lib.load_library()
    n = (3 << 20) + 9
    host = np.random.default_rng(8).integers(0, 256, n, dtype=np.uint8)
    d = torch.from_numpy(host).cuda()
    need = L.xinfer_crc64_device_scratch_bytes(n)
    scratch = torch.empty(need, dtype=torch.uint8, device="cuda")
    out = torch.zeros(1, dtype=torch.int64, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        rc = L.xinfer_crc64_device(ctypes.c_void_p(s.cuda_stream), ctypes.c_void_p(d.data_ptr()), n,
                                   ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(scratch.data_ptr()), need)
    assert rc == 0
    s.synchronize()
    assert (int(out.cpu().item()) & (2**64 - 1)) == oracle.crc64(host.tobytes())
    rc = L.xinfer_crc64_device(None, ctypes.c_void_p(d.data_ptr()), n, ctypes.c_void_p(out.data_ptr()),
                               ctypes.c_void_p(scratch.data_ptr()), need - 8)
    assert rc == _lib.XINFER_ERR_SCRATCH
    rc = L.xinfer_crc64_device(None, ctypes.c_void_p(d.data_ptr() + 1), n - 1,
                               ctypes.c_void_p(out.data_ptr()), None, 0)
    assert rc == _lib.XINFER_ERR_MISALIGNED


def test_upload_sections_verified(tmp_path):
    import torch
    big = np.random.default_rng(9).integers(0, 256, (70 << 20) + 13, dtype=np.uint8).tobytes()  # > 2 stages
    secs = [("big", SectionType.TensorWeights, big), ("small", SectionType.RawBlob, b"abc"),
            ("empty", SectionType.RawBlob, b"")]
    p = tmp_path / "a.xinfer"
    w = ArtifactWriter()
    for s in secs:
        w.add_section(*s)
    w.write_to_file(str(p))
    with ArtifactReader(str(p)) as r:
        for name, _, data in secs:
            dst = torch.empty(max(len(data), 1), dtype=torch.uint8, device="cuda")
            r.upload_section(name, dst)
            assert bytes(dst.cpu().numpy()[:len(data)].tobytes()) == data
        with pytest.raises(ArtifactError):  # destination too small
            r.upload_section("small", torch.empty(2, dtype=torch.uint8, device="cuda"))
    # corrupt one byte of the big section: the device CRC catches it
    b = bytearray(p.read_bytes())
    with ArtifactReader(str(p)) as r:
        off = r.get_section_info("big").offset
    b[off + (50 << 20)] ^= 0x10
    q = tmp_path / "bad.xinfer"
    q.write_bytes(bytes(b))
    with ArtifactReader(str(q)) as r:
        dst = torch.empty(len(big), dtype=torch.uint8, device="cuda")
        with pytest.raises(ArtifactError) as e:
            r.upload_section("big", dst)
        assert e.value.status == _lib.XINFER_ERR_CHECKSUM
        r.upload_section("big", dst, verify=False)  # unverified copy still lands


def test_load_linear_feeds_gemv(tmp_path):
    import torch
    from xinfer_amd import ops
    N, K, M = 1000, 5120, 1
    w = np.random.default_rng(11).normal(0, 0.02, size=(N, K)).astype(np.float32)
    W, S = oracle.quantize_int4(w)
    p = tmp_path / "m.xinfer"
    wr = ArtifactWriter()
    wr.set_metadata({"model_name": "t", "quant_scheme": "INT4-G128-SYM"})
    wr.add_section("layer.down_proj.weight", SectionType.TensorWeights, W.tobytes())
    wr.add_section("layer.down_proj.weight.scales", SectionType.TensorScales, S.tobytes())
    wr.write_to_file(str(p))
    with ArtifactReader(str(p)) as r:
        v = artifact.load_linear(r, "layer.down_proj.weight", N, K)
        with pytest.raises(ArtifactError):  # wrong shape: size check of weights.cpp:264-270
            artifact.load_linear(r, "layer.down_proj.weight", N + 1, K)
    assert v.is_valid()
    Xb = synth.activations(5, M, K)
    Y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    ops.linear_int4(Y, f16_dev(Xb), v.weights_int4, v.scales, None, M, N, K)
    ref = oracle.linear_int4(oracle.f16_to_f32(Xb), W, S, M, N, K)
    print(check_f16_tol(to_np(Y), ref))


def test_c_load_linear_on_golden_file():
    import ctypes
    import torch
    exp = json.load(open(os.path.join(GOLDEN, "artifact_ref_small.json")))
    lin = exp["linear"]
    L = _lib.load_library()
    path = os.path.join(GOLDEN, "artifact_ref_small.xinfer")
    h = ctypes.c_void_p()
    err = ctypes.create_string_buffer(512)
    assert L.xinfer_artifact_open(path.encode(), ctypes.byref(h), err, 512) == 0, err.value
    view = _lib.LinearWeightViewC()
    rc = L.xinfer_artifact_load_linear(h, lin["name"].encode(), lin["out_features"], lin["in_features"],
                                       lin["group_size"], None, ctypes.byref(view), err, 512)
    assert rc == 0, err.value
    try:
        with ArtifactReader(path) as r:
            W = np.frombuffer(r.read_section(lin["name"]), np.uint8)
            S = np.frombuffer(r.read_section(lin["name"] + ".scales"), np.uint8)
        hW = np.empty_like(W)
        hS = np.empty_like(S)
        torch.cuda.synchronize()
        hip = ctypes.CDLL("libamdhip64.so.7")  # copy back through the runtime torch loaded
        hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        assert hip.hipMemcpy(hW.ctypes.data, view.d_weights_int4, W.size, 2) == 0
        assert hip.hipMemcpy(hS.ctypes.data, view.d_scales, S.size, 2) == 0
        assert np.array_equal(hW, W) and np.array_equal(hS, S)
        assert (view.in_features, view.out_features, view.group_size) == (
            lin["in_features"], lin["out_features"], lin["group_size"])
        hip.hipFree.argtypes = [ctypes.c_void_p]
        hip.hipFree(view.d_weights_int4)
        hip.hipFree(view.d_scales)
    finally:
        L.xinfer_artifact_close(h)
