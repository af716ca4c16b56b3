"""The host-side native code under the compiler's sanitizers (CPU only): the
host gather's thread pool under ThreadSanitizer, the gather and the planner
under AddressSanitizer + UndefinedBehaviorSanitizer.  The harnesses in
tests/native/ are built with g++ from the library's own sources."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "meshy_amd", "csrc")
ROCM_INCLUDE = "/opt/rocm/include"

pytestmark = pytest.mark.skipif(shutil.which("g++") is None or not os.path.isdir(ROCM_INCLUDE),
                                reason="needs g++ and the ROCm headers")


def _build_and_run(tmp_path, name, source, harness, sanitize):
    exe = str(tmp_path / name)
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-pthread", f"-I{ROCM_INCLUDE}", "-D__HIP_PLATFORM_AMD__",
           *sanitize, os.path.join(CSRC, source), os.path.join(ROOT, "tests", "native", harness), "-o", exe]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-2000:]
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1", ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    run = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert run.returncode == 0, (run.stdout + run.stderr)[-4000:]
    assert "ERROR" not in run.stderr and "runtime error" not in run.stderr, run.stderr[-4000:]
    return run.stdout


def test_gather_pool_has_no_data_race(tmp_path):
    out = _build_and_run(tmp_path, "gather_tsan", "hostio.cpp", "gather_harness.cpp", ["-fsanitize=thread"])
    assert "0 bad gathers" in out


@pytest.mark.parametrize("source,harness,expect", [
    ("hostio.cpp", "gather_harness.cpp", "0 bad gathers"),
    ("plan.cpp", "plan_harness.cpp", "built"),
])
def test_address_and_undefined_behaviour(tmp_path, source, harness, expect):
    out = _build_and_run(tmp_path, source.split(".")[0] + "_asan", source, harness,
                         ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"])
    assert expect in out
