"""One prepared object used from two streams without synchronising between the calls.

The prepared objects keep their partial-sum workspaces across calls (no per-call allocation,
unlike the reference's spmm_csr.py:979-983); a call from another stream than the previous one
is ordered after the work queued on that stream (_plan.StreamOrder).  Every layout with a
workspace is driven from two same-priority streams in alternation - the row-block SpMV with
split rows, the XCS + panel hybrid, the staged-x layout (its staged values are a workspace
too), and SpMM with split rows - and each result must match the
fp64 oracle.
"""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _spmv_layouts, synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu


def _matrix(lengths, n_cols, seed, dtype=torch.float32):
    keys = synthetic._distinct_sorted_columns(torch.as_tensor(lengths, dtype=torch.int64),
                                              n_cols, seed, 1)
    ip, cols = synthetic._csr_from_keys(keys, len(lengths), n_cols)
    vals = synthetic.uniform_values(seed, 2, cols.numel(), dtype, "cpu")
    return vals, cols.to(torch.int32), ip


def _alternate(dev, call, inputs, rounds=4):
    """Run call(input) on two streams in turn, rounds times each, without synchronising;
    returns the outputs of the last round, one per stream."""
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    torch.cuda.synchronize()
    outs = [None, None]
    for _ in range(rounds):
        for k, s in enumerate(streams):
            with torch.cuda.stream(s):
                outs[k] = call(inputs[k])
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("layout", ["rowblock", "xcs-hybrid", "xstage"])
def test_spmv_two_streams(dev, layout, monkeypatch):
    monkeypatch.setattr(_spmv_layouts, "FORCE", layout)
    rng = np.random.default_rng(7)
    n_cols = 2_000_000
    lengths = rng.zipf(1.7, 40000).clip(max=60000)  # long rows split into chunks / panels
    vals, cols, ip = _matrix(lengths, n_cols, 7)
    p = fs.prepare_spmv_csr(vals.to(dev), cols.to(dev), ip.to(dev), (len(lengths), n_cols))
    xs = [synthetic.uniform_values(7, 10 + k, n_cols, torch.float32, "cpu") for k in range(2)]
    xd = [x.to(dev) for x in xs]
    print(f"two-stream SpMV {layout}", flush=True)
    ys = _alternate(dev, lambda x: fs.flagsparse_spmv_csr(x=x, prepared=p), xd)
    assert p._kernel(False).kind == layout
    for x, y in zip(xs, ys):
        ref = oracle.spmv_csr(ip, cols, vals, x)
        assert oracle.rel_l2(y, ref) <= oracle.REL_L2_BOUND["float32"]


def test_spmm_two_streams(dev):
    lengths = [3000] * 64 + [17] * 2000 + [9000] * 8  # rows cut into parts (workspace)
    n_cols = 50000
    vals, cols, ip = _matrix(lengths, n_cols, 8)
    p = fs.prepare_spmm_csr_opt(vals.to(dev), cols.to(dev), ip.to(dev), (len(lengths), n_cols))
    Bs = [synthetic.dense_uniform(n_cols, 32, dtype=torch.float32, seed=20 + k, device="cpu")
          for k in range(2)]
    Bd = [B.to(dev) for B in Bs]
    print("two-stream SpMM", flush=True)
    Cs = _alternate(dev, lambda B: fs.flagsparse_spmm_csr_opt(B=B, prepared=p), Bd)
    for B, C in zip(Bs, Cs):
        ref = oracle.spmm_csr(ip, cols, vals, B)
        assert oracle.rel_l2(C, ref) <= oracle.REL_L2_BOUND["float32"]
