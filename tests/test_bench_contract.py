"""The bench's output contract: one JSON line with the metric, its value and
unit, the step timing, the roofline entry of the dominant kernel and the
workload config; more than one GPU is refused with a message."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]


@pytest.mark.gpu
def test_bench_json_line(gpu, monkeypatch, capsys):
    sys.path.insert(0, ROOT)
    import bench
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        metric = json.load(f)["metric"]
    monkeypatch.setattr(sys, "argv", ["bench.py", "--no-cpu", "--no-b1", "--steps", "3",
                                      "--warmup", "1"])
    bench.main()
    lines = [l for l in capsys.readouterr().out.splitlines() if l.startswith("{")]
    assert len(lines) == 1
    r = json.loads(lines[0])
    assert r["metric"] == metric and r["unit"] == "GB/s" and r["higher_is_better"] is True
    assert r["n_gpus"] == 1 and r["steps"] == 3 and r["warmup"] == 1
    assert r["value"] > 0 and r["ms_per_step"] > 0 and r["vs_baseline"] is None
    assert r["dtype"] == "f32" and r["data"] == "synthetic" and r["scaling"] == "weak"
    assert r["config"]["workload"].startswith("cfg3")
    rf = r["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    assert rf["traffic"] is None or rf["traffic"] > 0
    # value is the whole step's bytes over its time; achieved is one launch's
    assert abs(r["value"] - r["config"]["bytes_per_step"] / (r["ms_per_step"] * 1e-3) / 1e9) \
        < 1e-3 * r["value"] + 0.01
    # BASELINE config 4 leg: fused append + decode over 256 sessions
    c4 = r["cfg4"]
    assert c4["config"]["workload"].startswith("cfg4") and c4["config"]["sessions"] == 256
    assert c4["value"] > 0 and c4["roofline"]["kernel"].endswith("true>")
    assert abs(c4["value"] - c4["config"]["bytes_per_step"] / (c4["ms_per_step"] * 1e-3) / 1e9) \
        < 1e-3 * c4["value"] + 0.01
