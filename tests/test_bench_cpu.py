"""bench.py's contract pieces that need no GPU: the one-GPU refusal and the reading of the
committed rocprofv3 summaries."""

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr and proc.stdout == ""


def test_profiles_parse():
    # every committed traffic summary yields its traffic, and per-kernel L2 hit rates in [0, 1]
    names = [f for f in os.listdir(os.path.join(ROOT, "profiles")) if f.endswith("_traffic.txt")]
    assert names
    for f in names:
        prof = bench._profile(f[:-len("_traffic.txt")])
        assert prof["traffic"] > 0, f
        for k, v in prof.get("l2_hit_rate", {}).items():
            assert 0.0 <= v <= 1.0, (f, k)
    assert bench._profile("no_such_profile") == {}
    json.dumps(prof)
