"""The diagnostic prefill library (libbmo_attn_phases.so, built from the same
sources with BMO_PREFILL_PHASES=1) through `bench.py --prefill-phases`, in a
subprocess: every wave of the cfg5 call leaves its phase stamps, in order,
and the summary has the shape the profile reads (two rounds of 256
workgroups; 12 barrier periods with the ring's history full, 4 without)."""
import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_prefill_phases_summary():
    lib = os.path.join(ROOT, "bmo_jetson_amd", "libbmo_attn_phases.so")
    assert os.path.exists(lib), "libbmo_attn_phases.so is not built (run __graft_entry__.build())"
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--prefill-phases"],
                         capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert res.returncode == 0, res.stderr[-2000:]
    ph = json.loads(res.stdout.strip().splitlines()[-1])["prefill_phases"]
    for name, periods in (("full", 12), ("empty", 4)):
        c = ph[name]
        assert c["periods"] == periods
        assert c["round1"]["workgroups"] == 256 and c["round2"]["workgroups"] == 256
        assert c["round1"]["start_us"] < 5.0 < c["round2"]["start_us"]
        for r in ("round1", "round2"):
            for k in ("query_rows_converted_us", "chunk_quantized_us", "loop_us", "epilogue_us"):
                assert 0.0 < c[r][k] < c["kernel_span_us"], (name, r, k, c[r][k])
        assert 0.0 < c["period_us"] and c["kernel_span_us"] <= 1.5 * c["call_us"]
        assert len(c["multiply_total_us_by_wave_age"]) == 4
