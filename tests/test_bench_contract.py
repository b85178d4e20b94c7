"""The bench line's contract on the CPU: one GPU only, and the roofline's
traffic figure is the committed rocprofv3 summary's, rebuilt from its counter
values and calibration factors."""

import json
import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 2
    assert "one GPU" in res.stderr


@pytest.mark.skipif(torch.cuda.is_available(), reason="would run the bench on the GPU")
def test_no_gpu_is_an_error():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--no-suite"],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 1
    assert "needs a GPU" in res.stderr


def test_roofline_traffic_is_the_profiled_summary():
    d = json.loads((ROOT / "profiles" / "attn_fwd_c2.json").read_text())
    want = (d["fetch_size_kib_per_dispatch"] * d["fetch_calibration_factor"] +
            d["write_size_kib_per_dispatch"] * d["write_calibration_factor"]) * 1024
    assert bench.profiled_traffic("c2") == d["traffic_bytes_per_launch"] == int(want)
    # the traffic is at least the launch's algorithmic bytes (Q, K, V read once, O written)
    assert d["traffic_bytes_per_launch"] >= d["algorithmic_bytes_per_launch"]
    for cmd in d["commands"]:
        assert cmd.startswith("rocprofv3 --pmc ") and "python3 bench.py" in cmd
    assert bench.profiled_traffic("c5") is None
