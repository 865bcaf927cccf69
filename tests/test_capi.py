"""CPU checks of the C-ABI library: it loads, exports every symbol the
header declares, and rejects bad arguments before touching a device."""
import ctypes
import glob
import os
import re

import pytest

from xinfer_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "xinfer_hip", "*.h")))


def header_functions():
    names = set()
    for h in HEADERS:
        txt = open(h).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        names |= set(re.findall(r"\b(xinfer_\w+)\s*\(", txt))
    return sorted(names)


@pytest.fixture(scope="module")
def L():
    return _lib.load_library()


def test_exports_match_header(L):
    declared = header_functions()
    assert declared == sorted(_lib.EXPORTS)
    for name in declared:
        assert hasattr(L, name), name


def test_symbols_visible_to_dlsym():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in header_functions():
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value


def test_version_and_status_strings(L):
    assert L.xinfer_version().decode().startswith("xinfer_hip")
    assert L.xinfer_status_string(0) == b"XINFER_OK"
    assert L.xinfer_status_string(-2) == b"XINFER_ERR_UNSUPPORTED"
    assert L.xinfer_status_string(-99) == b"XINFER_ERR_UNKNOWN"


def test_argument_checks_without_launch(L):
    fake = ctypes.c_void_p(0x10000)  # aligned, never dereferenced: every call fails validation
    odd = ctypes.c_void_p(0x10001)
    f = L.xinfer_linear_int4_f16
    # empty shapes are a no-op (src/ops/linear.cpp:176)
    assert f(None, None, None, None, None, None, 0, 16, 128, 128) == 0
    assert f(None, None, None, None, None, None, 1, -3, 128, 128) == 0
    # unsupported group size / K
    assert f(None, fake, fake, fake, fake, None, 1, 16, 128, 64) == _lib.XINFER_ERR_UNSUPPORTED
    assert f(None, fake, fake, fake, fake, None, 1, 16, 200, 128) == _lib.XINFER_ERR_UNSUPPORTED
    # null operand with a non-empty shape
    assert f(None, fake, None, fake, fake, None, 1, 16, 128, 128) == _lib.XINFER_ERR_INVALID_ARG
    # misaligned weights / activations
    assert f(None, fake, fake, odd, fake, None, 1, 16, 128, 128) == _lib.XINFER_ERR_MISALIGNED
    assert f(None, fake, odd, fake, fake, None, 1, 16, 128, 128) == _lib.XINFER_ERR_MISALIGNED
    # fused: descriptor count outside 1..4 (src/ops/linear.cpp:359)
    descs = (_lib.FusedDesc * 5)()
    assert L.xinfer_linear_int4_fused_f16(None, fake, descs, 0, 1, 128, 128) == _lib.XINFER_ERR_INVALID_ARG
    assert L.xinfer_linear_int4_fused_f16(None, fake, descs, 5, 1, 128, 128) == _lib.XINFER_ERR_INVALID_ARG
    assert L.xinfer_linear_int4_fused_f16(None, fake, None, 1, 1, 128, 128) == _lib.XINFER_ERR_INVALID_ARG
    # lm-head argmax handles M <= 8 only
    assert L.xinfer_lm_head_argmax_int4(None, fake, None, fake, fake, fake, 9, 16, 128, 128,
                                        None, 0) == _lib.XINFER_ERR_UNSUPPORTED
    # scratch too small
    assert L.xinfer_argmax_f32(None, fake, 100000, 1, fake, fake, 8) == _lib.XINFER_ERR_SCRATCH


def test_scratch_sizes(L):
    assert L.xinfer_argmax_scratch_bytes(0, 1) == 0
    assert L.xinfer_argmax_scratch_bytes(1, 1) == 0
    assert L.xinfer_argmax_scratch_bytes(4096, 1) == 8
    assert L.xinfer_argmax_scratch_bytes(4097, 3) == 3 * 2 * 8
    assert L.xinfer_lm_head_argmax_scratch_bytes(1, 151936, 5120) > 0
    assert L.xinfer_lm_head_argmax_scratch_bytes(9, 151936, 5120) == 0


def test_cxx_interface_compiles_links_and_validates(tmp_path):
    """The C++ mirrors (xinfer::ops, xinfer::artifact) build with g++ against
    the C-ABI; validation paths and the host-side reader behave (no GPU work
    is issued)."""
    import subprocess
    src = os.path.join(ROOT, "tests", "cabi_cxx_check.cpp")
    exe = str(tmp_path / "cabi_cxx_check")
    libdir = os.path.dirname(_lib.LIB_PATH)
    torch_lib = os.path.join(os.path.dirname(__import__("torch").__file__), "lib")
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), src, "-o", exe,
                    "-L", libdir, "-lxinfer_hip", f"-Wl,-rpath,{libdir}", f"-Wl,-rpath,{torch_lib}",
                    f"-Wl,-rpath-link,{torch_lib}", "-L", torch_lib],
                   check=True)
    golden = os.path.join(ROOT, "tests", "golden", "artifact_ref_small.xinfer")
    r = subprocess.run([exe, golden], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "OK", (r.stdout, r.stderr)
