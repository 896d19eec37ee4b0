"""The host side of the staged boundary copies (camel_amd/csrc/hip/host_copy.h),
on the CPU: chunk plans at the staging slots' edges and the parallel copy from
unaligned sources (the reference's tensor payload is 8-byte aligned only,
modules/tensor/runtime.cpp:482-485), built with g++ as is and under
ThreadSanitizer.  The device side of the same copies is tested by
tests/test_gpu_kernels.py."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "host_copy", "host_copy_test.cpp")
INC = os.path.join(ROOT, "camel_amd", "csrc", "hip")
OUT = os.path.join(ROOT, "_build", "host_copy")


@pytest.mark.parametrize("sanitize", [False, True], ids=["plain", "tsan"])
def test_staged_copy_host_side(sanitize):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    os.makedirs(OUT, exist_ok=True)
    exe = os.path.join(OUT, "host_copy_test" + ("_tsan" if sanitize else ""))
    flags = ["-fsanitize=thread", "-g"] if sanitize else []
    b = subprocess.run(["g++", "-std=c++17", "-O2", "-pthread", *flags, f"-I{INC}", SRC, "-o", exe],
                       capture_output=True, text=True, timeout=300)
    assert b.returncode == 0, b.stdout + b.stderr
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1 exitcode=66")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    assert "failures=0" in r.stdout
