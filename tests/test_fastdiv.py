"""The decode kernel divides by run-time constants (heads per entry, query
heads per kv head, ring slots) with bmo::FastDiv from kernels.hpp.  This
compiles that header on the host with g++ and checks the multiply-and-shift
quotient against integer division (tests/fastdiv_check.cpp)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.mark.skipif(shutil.which("g++") is None or not os.path.isdir("/opt/rocm/include"),
                    reason="needs g++ and the ROCm headers")
def test_fastdiv_matches_integer_division(tmp_path):
    exe = tmp_path / "fastdiv_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + os.path.join(ROOT, "bmo_jetson_amd", "csrc"),
                    os.path.join(HERE, "fastdiv_check.cpp"), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0 and res.stdout.startswith("ok "), res.stdout + res.stderr
