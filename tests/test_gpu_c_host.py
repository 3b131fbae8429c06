"""The library from a C++ host, through include/bmo_attn.h alone (programs
built by tests/Makefile, which __graft_entry__.build() runs):

  * tests/c_host_check.cpp drives a two-layer ring and a per-session handle
    -- 75 token steps at consecutive positions over a 48-slot ring: 25
    eager, 20 replayed from the handle's captured step, 7 queued one layer
    at a time and 23 replayed from a step captured layer by layer, without
    and with RoPE;
  * tests/c_host_kernels.cpp calls the node-level entry points as the
    reference's C++ engine calls its kernels: bmo_launch_decode_attention
    with the position as n_past and through pos_dev, bmo_kv_ring_prefill on
    two sessions (one-kernel and staged paths, a chunk that wraps the ring)
    and bmo_launch_gemv_q4_0_q8_1 at a shape of each of its kernels;

and both check every output against the CPU oracle (attention at
|gpu - ref| <= 2e-3 + 1e-3 |ref|, the GEMV within its rounding-error scale)
and the rings' blocks and the Q8_1 scratch bit for bit."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BUILD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "build")
EXE = os.path.join(BUILD, "c_host_check")
EXE_KERNELS = os.path.join(BUILD, "c_host_kernels")


def test_c_host_session_steps():
    assert os.path.exists(EXE), "tests/build/c_host_check is not built (run __graft_entry__.build())"
    res = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.count("ok theta") == 2, res.stdout


def test_c_host_node_prefill_gemv():
    assert os.path.exists(EXE_KERNELS), "tests/build/c_host_kernels is not built (run __graft_entry__.build())"
    res = subprocess.run([EXE_KERNELS], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.count("ok ") == 5, res.stdout
