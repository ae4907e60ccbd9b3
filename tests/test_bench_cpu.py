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


def test_probe_group_indices():
    # --probe-group / --probe-range / --probe-sorted: every index inside its workgroup's XCD
    # eighth and inside one range per group; sorted groups laid out lane-major
    import torch

    hi, n, group, span = 1 << 20, 4 * 4096, 2048, 1 << 14
    for sort in (False, True):
        idx = bench._probe_indices(n, hi, True, "cpu", torch, 4096, group, span, sort)
        idx = idx.to(torch.int64)
        assert idx.numel() == n and int(idx.min()) >= 0 and int(idx.max()) < hi
        w = hi // 8
        blk = torch.arange(n) // 4096
        assert torch.equal(idx // w, blk % 8)                     # the XCD's eighth
        g = idx.view(-1, group)
        assert torch.equal(g.min(1)[0] // span, g.max(1)[0] // span)  # one range per group
        if sort:
            # thread t takes positions 16t..16t+15; instruction k of a wave gathers sorted
            # indices 64k .. 64k + 63 of that wave's 1024, one per lane, in lane order
            wave = idx.view(-1, 64, 16).transpose(1, 2).reshape(-1, 1024)
            assert bool((wave[:, 1:] >= wave[:, :-1]).all())
    plain = bench._probe_indices(n, hi, True, "cpu", torch, 4096)
    assert torch.equal(plain.to(torch.int64) // (hi // 8), torch.arange(n) // 4096 % 8)


def test_cpu_baselines_block():
    # cpu_baseline is the reference's own CPU path (torch.sparse.mm on torch's host threads);
    # the C oracle port and scipy are reported beside it under their own keys
    import torch

    ptr = torch.tensor([0, 2, 3, 5], dtype=torch.int64)
    idx = torch.tensor([0, 2, 1, 0, 2], dtype=torch.int64)
    data = torch.tensor([1.0, 2.0, 3.0, 4.0, 5.0])
    x = torch.tensor([1.0, -1.0, 0.5])
    w = {"cpu": lambda s: {"value": 1.0, "unit": "GB/s", "cores": 1, "kind": "port"},
         "cpu_lib": bench._cpu_lib("csr", (ptr, idx, data), x, (3, 3), 10**12, 10**12, torch)}
    # byte and flop counts large enough that the rounded rates of this tiny matrix stay > 0
    base, port, ref = bench._cpu_baselines(w, 0.01, torch)
    assert base["kind"] == "reference" and "torch.sparse.mm" in base["path"], base
    assert base["cores"] == torch.get_num_threads() and base["value"] > 0
    assert "host" in base and port["kind"] == "port"
    assert ref["scipy"]["cores"] == 1 and ref["scipy"]["value"] > 0
    # a workload without a library path reports the port as its baseline
    only_port = bench._cpu_baselines({"cpu": w["cpu"]}, 0.01, torch)
    assert only_port[0]["kind"] == "port" and only_port[1] is None and only_port[2] is None
