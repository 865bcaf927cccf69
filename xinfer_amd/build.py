"""Build libxinfer_hip.so (gfx950) in-tree with hipcc (and bench.py's
measurement kernels, libxinfer_calib.so).

    python -m xinfer_amd.build          # build
    python -m xinfer_amd.build --asm    # also dump gfx950 ISA to _build/
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(OUT_DIR, "libxinfer_hip.so")
# measurement kernels of bench.py --calib-floor, a library of their own
CALIB_SRC = os.path.join(HERE, "calib", "read_calib.hip")
CALIB_LIB = os.path.join(OUT_DIR, "libxinfer_calib.so")
BUILD_DIR = os.path.join(ROOT, "_build")
ARCH = "gfx950"

SOURCES = ["gemv_int4.hip", "gemv_pair_int4.hip", "gemv_mb_int4.hip", "argmax.hip", "misc.hip", "gemm_int4.hip", "crc64.hip",
           "artifact.hip", "scratch.hip", "noalloc.hip", "gemm_ws_int4.hip"]

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32
# (packed fp16 ops are unaffected).
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    return os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(asm: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    r = subprocess.run([hipcc(), *HIPCC_FLAGS, "-shared", CALIB_SRC, "-o", CALIB_LIB + ".tmp"],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"calibration library failed:\n{r.stderr}")
    os.replace(CALIB_LIB + ".tmp", CALIB_LIB)
    if asm:
        for src in SOURCES:
            out = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".s")
            subprocess.run([hipcc(), *HIPCC_FLAGS, "--cuda-device-only", "-S",
                            os.path.join(CSRC, src), "-o", out], check=True)
    return LIB_PATH


if __name__ == "__main__":
    print(build(asm="--asm" in sys.argv))
