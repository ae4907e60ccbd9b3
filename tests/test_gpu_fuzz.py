"""Seeded fuzz on the GPU: random shapes and row-length mixes (power law, uniform, mostly
empty, one huge row among empty ones).  SpMV is forced through the row-block, XCS and XCS +
panel layouts, CSR and COO, both accumulation modes; the same matrices then go through CSR SpMM
(base and opt, row- and column-major B), COO SpMM and SDDMM with a dense width drawn per case;
and all of them once more with +inf, -inf and NaN in a few columns of x and B, where the NaN and
infinity pattern must be the oracle's.  All against the fp64 oracle.

Bars as in test_gpu_spmv_csr.py: relative L2 error <= 1e-5 / 1e-12, the reference scripts'
allclose ratio, and for the default float32 SpMV path at most 1 ulp from float32(fp64 oracle).
"""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _spmv_layouts, synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu

# (row-length mix, number of columns) per seed
CASES = (("zipf", 70001), ("uniform", 1 << 20), ("sparse", 1000), ("one_huge", 3_000_000),
         ("zipf_heavy", 1 << 20), ("uniform", 7), ("zipf", 3_000_000), ("sparse", 70001),
         ("one_huge", 70001), ("zipf_heavy", 5000), ("uniform", 70001), ("zipf", 1000))


def _lengths(rng, kind, n_rows, n_cols):
    if kind == "zipf":
        lengths = rng.zipf(1.7, n_rows)
    elif kind == "zipf_heavy":
        lengths = rng.zipf(1.3, n_rows)
    elif kind == "uniform":
        lengths = rng.integers(0, 40, n_rows)
    elif kind == "sparse":  # nine rows in ten empty
        lengths = (rng.random(n_rows) < 0.1) * rng.integers(1, 6, n_rows)
    else:  # one_huge: a single long row among empty ones
        lengths = np.zeros(n_rows, dtype=np.int64)
        lengths[int(rng.integers(0, n_rows))] = int(rng.integers(1, 150000))
    # distinct columns per row: at most half the columns of a wide matrix (drawing nearly all
    # of them takes long), all of them for a narrow one
    cap = n_cols if n_cols <= 64 else n_cols // 2
    lengths = np.minimum(lengths, min(cap, 150000)).astype(np.int64)
    total = int(lengths.sum())
    if total > 2_000_000:  # a few seconds of oracle and setup per case
        lengths = (lengths * (2_000_000 / total)).astype(np.int64)
    return lengths


def _matrix(seed):
    rng = np.random.default_rng(1000 + seed)
    kind, n_cols = CASES[seed]
    n_rows = int(rng.integers(1, 30000))
    dtype = (torch.float32, torch.float64)[seed % 2]
    lengths = _lengths(rng, kind, n_rows, n_cols)
    keys = synthetic._distinct_sorted_columns(torch.as_tensor(lengths), n_cols, seed, 1)
    ptr, cols = synthetic._csr_from_keys(keys, n_rows, n_cols)
    vals = synthetic.uniform_values(seed, 2, cols.numel(), dtype, "cpu")
    x = synthetic.uniform_values(seed, 3, n_cols, dtype, "cpu")
    return kind, rng, vals, cols, ptr, x, (n_rows, n_cols)


def _check(y, ref64, exact_fp32):
    name = "float64" if y.dtype == torch.float64 else "float32"
    err = oracle.rel_l2(y, ref64)
    assert err <= oracle.REL_L2_BOUND[name], f"rel_l2 {err:.3e}"
    atol, rtol = oracle.REF_SCRIPT_TOL[name]
    assert oracle.allclose_ratio(y, ref64, atol, rtol) <= 1.0
    if exact_fp32:
        def ordered(v):
            i = np.ascontiguousarray(v, dtype=np.float32).view(np.int32).astype(np.int64)
            return np.where(i < 0, -(i & 0x7FFFFFFF), i)
        u = np.abs(ordered(y.cpu().numpy()) - ordered(ref64.astype(np.float32)))
        assert u.size == 0 or u.max() <= 1, u.max()


def _force(monkeypatch, layout):
    """Force a layout; "-sorted" takes the XCS items with sorted gathers (format 1) wherever
    the panels allow it, else row-order items (format 0)."""
    mode = layout.replace("-sorted", "")
    monkeypatch.setattr(_spmv_layouts, "FORCE", mode)
    monkeypatch.setattr(_spmv_layouts, "SORTED_ITEMS", layout.endswith("-sorted"))
    monkeypatch.setattr(_spmv_layouts, "SORTED_MIN_RUN", 0.0)
    return mode


LAYOUTS = ["rowblock", "xcs-l2", "xcs-l2-sorted", "xcs-hybrid", "xcs-hybrid-sorted", "xstage"]


@pytest.mark.parametrize("seed", range(len(CASES)))
@pytest.mark.parametrize("layout", LAYOUTS)
def test_fuzz_spmv(dev, monkeypatch, seed, layout):
    kind, rng, vals, cols, ptr, x, shape = _matrix(seed)
    layout = _force(monkeypatch, layout)
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANEL_ROW_MIN", int(rng.integers(2, 64)))
    print(f"fuzz seed={seed} {kind} {layout} shape={shape} nnz={vals.numel()} {vals.dtype}",
          flush=True)
    ref = oracle.spmv_csr(ptr, cols, vals, x)
    d, c, p, xd = vals.to(dev), cols.to(torch.int32).to(dev), ptr.to(dev), x.to(dev)
    prepared = fs.prepare_spmv_csr(d, c, p, shape)
    lay = prepared._kernel(False)
    built = lay.kind
    xcs = getattr(lay, "short", lay)
    print(f"  layout built: {built} item format {getattr(xcs, 'item_format', '-')}", flush=True)
    # the forced layout is the one tested (the hybrid needs a row of FORCE_PANEL_ROW_MIN entries)
    has_long = bool(((ptr[1:] - ptr[:-1]) >= _spmv_layouts.FORCE_PANEL_ROW_MIN).any())
    expect = {"rowblock": "rowblock", "xcs-l2": "xcs", "xstage": "xstage",
              "xcs-hybrid": "xcs-hybrid" if has_long else "xcs"}[layout]
    assert built == expect
    for use_opt in (False, True):
        y = fs.flagsparse_spmv_csr(x=xd, prepared=prepared, use_opt=use_opt)
        _check(y, ref, exact_fp32=(vals.dtype == torch.float32 and not use_opt))
        # a second call reuses the layout's workspaces: the same result, bit for bit
        assert torch.equal(y, fs.flagsparse_spmv_csr(x=xd, prepared=prepared, use_opt=use_opt))
    rows = torch.repeat_interleave(torch.arange(shape[0]), ptr[1:] - ptr[:-1])
    y = fs.flagsparse_spmv_coo(d, rows.to(dev), c, xd, shape)
    _check(y, oracle.spmv_coo(rows, cols, vals, x, shape[0]), exact_fp32=False)


def _check_dense(out, ref64):
    name = "float64" if out.dtype == torch.float64 else "float32"
    if ref64.size == 0:
        return
    err = oracle.rel_l2(out, ref64)
    assert err <= oracle.REL_L2_BOUND[name], f"rel_l2 {err:.3e}"
    atol, rtol = oracle.REF_SCRIPT_TOL[name]
    assert oracle.allclose_ratio(out, ref64, atol, rtol) <= 1.0


@pytest.mark.parametrize("seed", range(len(CASES)))
def test_fuzz_spmm_sddmm(dev, seed):
    # the same matrices with a dense operand of random width: CSR SpMM (base and opt), COO SpMM,
    # a column-major B, and SDDMM with K = N
    kind, rng, vals, cols, ptr, x, shape = _matrix(seed)
    n_rows, n_cols = shape
    N = int(rng.choice([1, 2, 3, 5, 16, 17, 64, 100]))
    N = max(1, min(N, 20_000_000 // max(n_rows, n_cols)))  # B and C within 20M values
    dtype = vals.dtype
    print(f"fuzz spmm seed={seed} {kind} shape={shape} nnz={vals.numel()} N={N} {dtype}",
          flush=True)
    B = synthetic.uniform_values(seed, 4, n_cols * N, dtype, "cpu").reshape(n_cols, N)
    ref = oracle.spmm_csr(ptr, cols, vals, B)
    d, c, p, Bd = vals.to(dev), cols.to(torch.int32).to(dev), ptr.to(dev), B.to(dev)
    _check_dense(fs.flagsparse_spmm_csr(d, c, p, Bd, shape), ref)
    _check_dense(fs.flagsparse_spmm_csr_opt(d, c, p, Bd, shape), ref)
    _check_dense(fs.flagsparse_spmm_csr(d, c, p, Bd.t().contiguous().t(), shape), ref)
    rows = torch.repeat_interleave(torch.arange(n_rows), ptr[1:] - ptr[:-1])
    _check_dense(fs.flagsparse_spmm_coo(d, rows.to(dev), c, Bd, shape),
                 oracle.spmm_coo(rows, cols, vals, B, n_rows))
    xs = synthetic.uniform_values(seed, 5, n_rows * N, dtype, "cpu").reshape(n_rows, N)
    out = fs.flagsparse_sddmm_csr(data=d, indices=c, indptr=p, x=xs.to(dev), y=Bd, shape=shape,
                                  alpha=0.5, beta=2.0)
    _check_dense(out, oracle.sddmm_csr(ptr, cols, xs, B, vals, alpha=0.5, beta=2.0))


def _check_nonfinite(out, ref64):
    """NaN and signed infinities exactly where the oracle has them (for a sum that does not
    depend on the summation order), the finite values within the usual bars."""
    out = out.cpu().numpy() if torch.is_tensor(out) else out
    assert np.array_equal(np.isnan(out), np.isnan(ref64))
    inf = np.isinf(ref64)
    assert np.array_equal(np.isinf(out), inf)
    assert np.array_equal(np.sign(out[inf]), np.sign(ref64[inf]))
    fin = np.isfinite(ref64)
    if fin.any():
        _check_dense(torch.as_tensor(out[fin]), ref64[fin])


@pytest.mark.parametrize("seed", range(len(CASES)))
def test_fuzz_nonfinite(dev, monkeypatch, seed):
    # x (and B, and SDDMM's y) with +inf, -inf and NaN in a few random columns: every path
    # gives the oracle's NaN / inf pattern - padding and masked lanes must add exactly 0
    kind, rng, vals, cols, ptr, x, shape = _matrix(seed)
    n_rows, n_cols = shape
    bad_cols = rng.choice(n_cols, size=min(n_cols, 3), replace=False)
    x = x.clone()
    for c, v in zip(bad_cols, (float("inf"), float("-inf"), float("nan"))):
        x[int(c)] = v
    print(f"fuzz non-finite seed={seed} {kind} shape={shape} nnz={vals.numel()}", flush=True)
    ref = oracle.spmv_csr(ptr, cols, vals, x)
    d, c, p, xd = vals.to(dev), cols.to(torch.int32).to(dev), ptr.to(dev), x.to(dev)
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANEL_ROW_MIN", int(rng.integers(2, 64)))
    for layout in LAYOUTS:
        _force(monkeypatch, layout)
        prepared = fs.prepare_spmv_csr(d, c, p, shape)
        for use_opt in (False, True):
            _check_nonfinite(fs.flagsparse_spmv_csr(x=xd, prepared=prepared, use_opt=use_opt),
                             ref)
    rows = torch.repeat_interleave(torch.arange(n_rows), ptr[1:] - ptr[:-1])
    for sort_by_row in (True, False):
        _check_nonfinite(fs.flagsparse_spmv_coo(d, rows.to(dev), c, xd, shape,
                                                sort_by_row=sort_by_row), ref)
    N = 5
    B = synthetic.uniform_values(seed, 4, n_cols * N, vals.dtype, "cpu").reshape(n_cols, N)
    B[torch.as_tensor(bad_cols)] = x[torch.as_tensor(bad_cols)].unsqueeze(1)
    ref_c = oracle.spmm_csr(ptr, cols, vals, B)
    Bd = B.to(dev)
    _check_nonfinite(fs.flagsparse_spmm_csr(d, c, p, Bd, shape), ref_c)
    _check_nonfinite(fs.flagsparse_spmm_csr_opt(d, c, p, Bd, shape), ref_c)
    _check_nonfinite(fs.flagsparse_spmm_coo(d, rows.to(dev), c, Bd, shape), ref_c)
    xs = synthetic.uniform_values(seed, 5, n_rows * N, vals.dtype, "cpu").reshape(n_rows, N)
    out = fs.flagsparse_sddmm_csr(data=d, indices=c, indptr=p, x=xs.to(dev), y=Bd, shape=shape)
    _check_nonfinite(out, oracle.sddmm_csr(ptr, cols, xs, B))
