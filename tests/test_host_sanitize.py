"""The engine's host layer (csrc/host/*.cpp: CSR/BSR builders, generators,
binary I/O, partitions, metrics, host references) built with g++ under
AddressSanitizer (leak checking on) and UndefinedBehaviorSanitizer, running
tests/host_sanitize.cpp.  CPU only; no device code is compiled."""
import glob
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_host_layer_under_sanitizers(tmp_path):
    srcs = sorted(glob.glob(os.path.join(ROOT, "sparse-matrix-multiplication_amd", "csrc", "host",
                                         "*.cpp")))
    exe = str(tmp_path / "host_sanitize")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-omit-frame-pointer", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I" + os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "host_sanitize.cpp"),
           *srcs, "-L/opt/rocm/lib", "-Wl,-rpath,/opt/rocm/lib", "-lamdhip64", "-lpthread",
           "-o", exe]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    run = subprocess.run([exe], capture_output=True, text=True, cwd=str(tmp_path), env=env,
                         timeout=300)
    assert run.returncode == 0, (run.stdout + run.stderr)[-4000:]
    assert "all checks passed" in run.stdout
