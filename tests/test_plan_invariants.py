"""Small-batch planner invariants over 60000 random shapes (host code only,
no GPU): built from tests/plan_invariants.hip with hipcc into a temporary
directory and run."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _hipcc():
    path = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    return path if os.path.exists(path) else shutil.which("hipcc")


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not available")
def test_small_batch_plan_invariants(tmp_path):
    exe = str(tmp_path / "plan_invariants")
    build = subprocess.run([_hipcc(), "-O1", "-std=c++17", "--offload-arch=gfx950",
                            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                            os.path.join(HERE, "plan_invariants.hip"), "-o", exe],
                           capture_output=True, text=True, timeout=600)
    assert build.returncode == 0, build.stderr[-2000:]
    run = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    print(run.stdout)
    assert run.returncode == 0, run.stdout[-2000:]


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not available")
def test_pair_split(tmp_path):
    """The row-pair kernels' pair ranges (host-computed split, multiply-shift
    division on the device) against exact 64-bit division."""
    exe = str(tmp_path / "pair_split_check")
    build = subprocess.run([_hipcc(), "-O1", "-std=c++17", "--offload-arch=gfx950",
                            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                            os.path.join(HERE, "pair_split_check.hip"), "-o", exe],
                           capture_output=True, text=True, timeout=900)
    assert build.returncode == 0, build.stderr[-2000:]
    run = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    print(run.stdout)
    assert run.returncode == 0, run.stdout[-2000:]
