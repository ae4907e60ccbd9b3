"""Prepared calls captured in a HIP graph (torch.cuda.CUDAGraph) and replayed.

A serving loop that calls SpMV or SpMM on a prepared matrix many times can capture the call
once and replay it, which takes the host launch work out of every step.  Each layout with a
workspace is captured after a warm-up on a side stream, then replayed several times with new
x / B values written in between by ordinary eager work, and every replay must equal the eager
call on the same input bit for bit (the same kernels, the same fixed summation order) and
match the fp64 oracle.  No path records a memset into the graph: y and C are cleared, where a
launch needs it, by a fill kernel.
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


def _capture(dev, call):
    """Warm up on a side stream, then capture call() into a graph."""
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for _ in range(2):
            call()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    torch.cuda.synchronize()
    return g


def _replay_and_check(dev, g, src, out, inputs, eager, ref_fn, dtype):
    for k, host_in in enumerate(inputs):
        src.copy_(host_in.to(dev))          # eager work between replays
        expect = eager(src)                  # an eager call of the same object, another output
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        print(f"  replay {k}", flush=True)
        assert torch.equal(out, expect), f"replay {k} differs from the eager call"
        assert oracle.rel_l2(out, ref_fn(host_in)) <= oracle.REL_L2_BOUND[dtype]


@pytest.mark.parametrize("layout,dtype", [("rowblock", torch.float32),
                                          ("rowblock", torch.float64),
                                          ("xcs-l2", torch.float32),
                                          ("xcs-hybrid", torch.float32),
                                          ("xcs-hybrid", torch.float64),
                                          ("xstage", torch.float32),
                                          ("xstage", torch.float64)])
@pytest.mark.parametrize("use_opt", [False, True])
def test_spmv_csr_graph_replay(dev, monkeypatch, layout, dtype, use_opt):
    monkeypatch.setattr(_spmv_layouts, "FORCE", layout)
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANEL_ROW_MIN", 32)
    rng = np.random.default_rng(11)
    n_cols = 300_000
    lengths = rng.zipf(1.7, 30000).clip(max=40000)  # split rows / panel rows have workspaces
    vals, cols, ip = _matrix(lengths, n_cols, 11, dtype)
    p = fs.prepare_spmv_csr(vals.to(dev), cols.to(dev), ip.to(dev), (len(lengths), n_cols))
    x = torch.empty(n_cols, dtype=dtype, device=dev)
    y = torch.empty(len(lengths), dtype=dtype, device=dev)
    x.copy_(synthetic.uniform_values(11, 9, n_cols, dtype, "cpu").to(dev))
    print(f"graph SpMV {layout} {dtype} use_opt={use_opt}", flush=True)
    g = _capture(dev, lambda: fs.flagsparse_spmv_csr(x=x, prepared=p, out=y, use_opt=use_opt))
    assert p._kernel(use_opt).kind == {"xcs-l2": "xcs"}.get(layout, layout)  # XCS alone
    inputs = [synthetic.uniform_values(11, 20 + k, n_cols, dtype, "cpu") for k in range(4)]
    _replay_and_check(dev, g, x, y, inputs,
                      lambda xx: fs.flagsparse_spmv_csr(x=xx, prepared=p, use_opt=use_opt),
                      lambda xh: oracle.spmv_csr(ip, cols, vals, xh), str(dtype)[6:])


def test_spmv_coo_graph_replay(dev):
    n, draws = 50_000, 600_000
    rng = np.random.default_rng(12)
    r = rng.integers(0, n, draws)
    c = rng.integers(0, n, draws)
    key = np.unique(r.astype(np.int64) * n + c)
    rows = torch.from_numpy(key // n).to(torch.int32)
    cols = torch.from_numpy(key % n).to(torch.int32)
    vals = synthetic.uniform_values(12, 2, rows.numel(), torch.float32, "cpu")
    p = fs.prepare_spmv_coo(vals.to(dev), rows.to(dev), cols.to(dev), (n, n))
    x = torch.empty(n, dtype=torch.float32, device=dev)
    x.copy_(synthetic.uniform_values(12, 9, n, torch.float32, "cpu").to(dev))
    y = torch.empty(n, dtype=torch.float32, device=dev)
    print("graph COO SpMV", flush=True)
    g = _capture(dev, lambda: fs.flagsparse_spmv_coo(x=x, prepared=p, out=y))
    inputs = [synthetic.uniform_values(12, 20 + k, n, torch.float32, "cpu") for k in range(3)]
    ip = torch.zeros(n + 1, dtype=torch.int64)
    ip[1:] = torch.cumsum(torch.bincount(rows.to(torch.int64), minlength=n), 0)
    _replay_and_check(dev, g, x, y, inputs,
                      lambda xx: fs.flagsparse_spmv_coo(x=xx, prepared=p),
                      lambda xh: oracle.spmv_csr(ip, cols, vals, xh), "float32")


@pytest.mark.parametrize("dtype,N", [(torch.float32, 32), (torch.float64, 16)])
def test_spmm_csr_opt_graph_replay(dev, dtype, N):
    lengths = [3000] * 32 + [17] * 2000 + [9000] * 4  # rows cut into parts (workspace)
    n_cols = 40000
    vals, cols, ip = _matrix(lengths, n_cols, 13, dtype)
    p = fs.prepare_spmm_csr_opt(vals.to(dev), cols.to(dev), ip.to(dev), (len(lengths), n_cols))
    B = torch.empty((n_cols, N), dtype=dtype, device=dev)
    B.copy_(synthetic.dense_uniform(n_cols, N, dtype=dtype, seed=30, device="cpu").to(dev))
    C = torch.empty((len(lengths), N), dtype=dtype, device=dev)
    print(f"graph SpMM {dtype} N={N}", flush=True)
    g = _capture(dev, lambda: fs.flagsparse_spmm_csr_opt(B=B, prepared=p, out=C))
    inputs = [synthetic.dense_uniform(n_cols, N, dtype=dtype, seed=40 + k, device="cpu")
              for k in range(3)]
    _replay_and_check(dev, g, B, C, inputs,
                      lambda BB: fs.flagsparse_spmm_csr_opt(B=BB, prepared=p),
                      lambda Bh: oracle.spmm_csr(ip, cols, vals, Bh), str(dtype)[6:])
