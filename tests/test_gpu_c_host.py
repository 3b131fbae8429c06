"""The library from a C++ host: tests/c_host_check.cpp (built by
tests/Makefile, which __graft_entry__.build() runs) drives a two-layer ring
and a per-session handle through include/bmo_attn.h alone -- 75 token steps
at consecutive positions over a 48-slot ring: 25 eager, 20 replayed from the
handle's captured step, 7 queued one layer at a time and 23 replayed from a
step captured layer by layer, without and with RoPE -- and checks every
output against the CPU oracle at |gpu - ref| <= 2e-3 + 1e-3 |ref| and the
ring's blocks bit for bit."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "build", "c_host_check")


def test_c_host_session_steps():
    assert os.path.exists(EXE), "tests/build/c_host_check is not built (run __graft_entry__.build())"
    res = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.count("ok theta") == 2, res.stdout
