"""COO SpMV on the GPU against the fp64 CPU oracle (spmv_coo.py routes of the reference).

Both routes are checked, as the reference's COO test does (tests/test_spmv_coo.py:190-201):
row runs (sort_by_row=True, deterministic) and atomics (sort_by_row=False).  Bars: relative L2
error <= 1e-5 / 1e-12 against the fp64 oracle and the allclose ratio of
tests/test_spmv_coo.py:323-326.
"""

import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu


def _check(y, ref64):
    name = "float64" if y.dtype == torch.float64 else "float32"
    err = oracle.rel_l2(y, ref64)
    assert err <= oracle.REL_L2_BOUND[name], f"rel_l2 {err:.3e}"
    atol, rtol = oracle.REF_SCRIPT_TOL[name]
    assert oracle.allclose_ratio(y, ref64, atol, rtol) <= 1.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_cfg4_like_sorted(dev, dtype):
    # cfg4's generator at 1/16 of the rows and draws
    data, row, col, x, shape = synthetic.coo_uniform(1 << 17, 40 << 16, dtype=dtype)
    print(f"cfg4-like nnz={data.numel()} {dtype}", flush=True)
    ref = oracle.spmv_coo(row, col, data, x, shape[0])
    p = fs.prepare_spmv_coo(data.to(dev), row.to(dev), col.to(dev), shape)
    assert p.use_seg_kernel and p.n_segs == int(torch.unique(row).numel())
    xd = x.to(dev)
    y = fs.flagsparse_spmv_coo(x=xd, prepared=p)
    _check(y, ref)
    assert torch.equal(y, fs.flagsparse_spmv_coo(x=xd, prepared=p))  # deterministic


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("sort_by_row", [True, False])
def test_unsorted_duplicates_empty_rows(dev, dtype, sort_by_row):
    n_rows, n_cols, nnz = 30000, 20000, 200000
    row = synthetic.randint(2, 1, nnz, n_rows - 5000, "cpu")  # the last 5000 rows are empty
    col = synthetic.randint(2, 2, nnz, n_cols, "cpu")
    row[:1000] = row[1000:2000]
    col[:1000] = col[1000:2000]
    data = synthetic.uniform_values(2, 3, nnz, dtype, "cpu")
    x = synthetic.uniform_values(2, 4, n_cols, dtype, "cpu")
    ref = oracle.spmv_coo(row, col, data, x, n_rows)
    y = fs.flagsparse_spmv_coo(data.to(dev), row.to(torch.int32).to(dev), col.to(dev), x.to(dev),
                               (n_rows, n_cols), sort_by_row=sort_by_row)
    _check(y, ref)
    assert torch.count_nonzero(y[n_rows - 5000:]) == 0


def test_long_runs_split(dev):
    # one row with 60000 entries (split across workgroups) among short runs
    n_cols = 100000
    keys = synthetic._distinct_sorted_columns(torch.tensor([3, 60000, 0, 5, 2]), n_cols, 4, 1)
    row = keys // n_cols
    col = keys % n_cols
    data = synthetic.uniform_values(4, 2, row.numel(), torch.float32, "cpu")
    x = synthetic.uniform_values(4, 3, n_cols, torch.float32, "cpu")
    ref = oracle.spmv_coo(row, col, data, x, 5)
    for sort_by_row in (True, False):
        y = fs.flagsparse_spmv_coo(data.to(dev), row.to(dev), col.to(dev), x.to(dev), (5, n_cols),
                                   sort_by_row=sort_by_row)
        _check(y, ref)


def test_api_knobs_out_and_errors(dev):
    data, row, col, x, shape = synthetic.coo_uniform(4096, 40000)
    d, r, c, xd = data.to(dev), row.to(dev), col.to(dev), x.to(dev)
    ref = oracle.spmv_coo(row, col, data, x, shape[0])
    out = torch.empty(shape[0], device=dev)
    y, ms = fs.flagsparse_spmv_coo(d, r, c, xd, shape, out=out, return_time=True)
    assert y is out and ms >= 0.0
    _check(y, ref)
    for bs in (1, 64, 256, 1000):
        _check(fs.flagsparse_spmv_coo(d, r, c, xd, shape, sort_by_row=False, block_size=bs), ref)
    with pytest.raises(ValueError):
        fs.flagsparse_spmv_coo(d, r, c, xd, shape, num_warps=3)
    with pytest.raises(ValueError):
        fs.flagsparse_spmv_coo(d, r, c, xd, shape, block_inner=100)
    with pytest.raises(TypeError):
        fs.prepare_spmv_coo(d.half(), r, c, shape)
    with pytest.raises(IndexError):
        fs.prepare_spmv_coo(d, r + shape[0], c, shape)
    with pytest.raises(IndexError):
        fs.prepare_spmv_coo(d, r, c - 5000, shape)
    with pytest.raises(ValueError):
        fs.prepare_spmv_coo(d, r[:-1], c, shape)
    p = fs.prepare_spmv_coo(d, r, c, shape)
    with pytest.raises(TypeError):
        fs.flagsparse_spmv_coo(prepared=p)
    with pytest.raises(ValueError):
        fs.flagsparse_spmv_coo(x=xd, prepared=p, shape=(3, 3))
    with pytest.raises(TypeError):
        fs.flagsparse_spmv_coo(x=xd.double(), prepared=p)
    # empty matrix
    e = fs.flagsparse_spmv_coo(torch.empty(0, device=dev), torch.empty(0, dtype=torch.int32,
                               device=dev), torch.empty(0, dtype=torch.int32, device=dev),
                               torch.ones(4, device=dev), (6, 4))
    assert e.shape == (6,) and torch.count_nonzero(e) == 0
