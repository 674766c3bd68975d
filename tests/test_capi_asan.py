"""Host AddressSanitizer run over the C-ABI validation paths: the library's
host code is rebuilt with -fsanitize=address on the host pass only (device
code is unchanged) and a small driver exercises every rejection path."""
import os
import shutil
import subprocess
import tempfile

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "ernie-evolve-results_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_capi_validation_under_asan():
    tmp = tempfile.mkdtemp(prefix="moe_asan_")
    try:
        exe = os.path.join(tmp, "capi_validation")
        from moe_route.build import SOURCES
        srcs = [os.path.join(CSRC, f) for f in SOURCES]
        cmd = [HIPCC, "-O1", "-g", "-std=c++17", "--offload-arch=gfx950",
               "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-I", os.path.join(REPO, "include"), "-I", CSRC, "-x", "hip"] + srcs + \
              ["-x", "none", os.path.join(REPO, "tests", "asan", "capi_validation.cpp"),
               "-fsanitize=address", "-o", exe]
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, res.stdout + res.stderr
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0")
        run = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=120)
        assert run.returncode == 0, run.stdout + run.stderr
        assert "OK (0 failures)" in run.stdout
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
