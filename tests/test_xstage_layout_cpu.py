"""The staged-x SpMV layout (flagsparse_amd/_spmv_layouts.py, XstageLayout), built on the CPU and
checked without a GPU: the structure the kernels rely on (every short entry staged exactly once
and placed exactly once in its window, windows of consecutive rows within their caps, segment
tables that tile each window, LDS positions in (row, panel) order, staging ranges of whole
groups of 8 inside their panel, one job per panel at least), and a step-by-step emulation of
spmv_panel_kernel's staging and stage_combine_kernel's sums (with the panel part's long rows
through the panel emulation) against the fp64 oracle."""

import numpy as np
import pytest
import torch

from flagsparse_amd import _abi, _spmv_layouts
from flagsparse_amd._spmv_layouts import XstageLayout, panel_row_min
from oracle import oracle
from test_xcs_layout_cpu import _case, _check_panels, _emulate_panels, _long_part


def _stage(layout, x):
    """spmv_panel_kernel's staging: job j stages entries [stage_jobs[j], stage_jobs[j+1]) of
    its panel, xs[e] = x[(panel << col_bits) + scol[e]]."""
    cb = layout.col_bits
    scol = layout.scol.numpy().view(np.uint16).astype(np.int64)
    sj = layout.stage_jobs.numpy().astype(np.int64)
    jp = layout.job_panel.numpy().astype(np.int64)
    xs = np.zeros(layout.xs.numel(), dtype=np.float64)
    for j in range(layout.n_jobs):
        e = np.arange(sj[j], sj[j + 1])
        col = (jp[j] << cb) + scol[e]
        xs[e] = x[np.minimum(col, x.size - 1)]
    return xs


def _windows(layout):
    """Per window: (row0, rows, entries, first, [(panel, staged start, staged end)])."""
    w = layout.windows.numpy().astype(np.int64)
    seg = layout.seg.numpy().astype(np.int64)
    out = []
    for k in range(layout.n_windows):
        segs = [(p, seg[k, p], seg[k + 1, p]) for p in range(layout.n_panels)
                if seg[k + 1, p] > seg[k, p]]
        out.append((*w[k].tolist(), segs))
    return out


def _emulate(layout, x, y, row_map=None, acc=np.float64):
    """stage_combine_kernel's windows: entry f of window k (its segments in panel order) adds
    vals[first + f] * xs[segment position] at LDS position dest[first + f]; row r of the window
    gets its row_count[r] positions summed in order (count 0xFFFF: left alone)."""
    xs = _stage(layout, x).astype(acc)
    vals = layout.vals.numpy().astype(acc)
    dest = layout.dest.numpy().astype(np.int64)
    rc = layout.row_count.numpy().view(np.uint16).astype(np.int64)
    for row0, nr, L, first, segs in _windows(layout):
        s = np.full(_abi.caps()["stage_window"], np.nan)
        f = 0
        for _, g0, g1 in segs:
            for g in range(g0, g1):
                s[dest[first + f]] = acc(vals[first + f] * xs[g])
                f += 1
        assert f == L
        pos = 0
        for i in range(nr):
            c = rc[row0 + i]
            if c == 0xFFFF:
                continue
            acc_v = acc(0)
            for u in range(c):
                acc_v = acc(acc_v + s[pos + u])
            out = row0 + i if row_map is None else row_map[row0 + i]
            y[out] = acc_v
            pos += c
        assert pos == L
    return y


def _check(layout, vals, cols, ip, long_mask):
    caps = _abi.caps()
    cb, P = layout.col_bits, layout.n_panels
    rp = ip.numpy().astype(np.int64)
    n_rows = rp.size - 1
    lengths = np.diff(rp)
    short = ~long_mask
    # windows: consecutive rows from 0 to n_rows, within both caps
    w = layout.windows.numpy().astype(np.int64)
    assert w[0, 0] == 0 and w[-1, 0] + w[-1, 1] == n_rows
    assert np.all(w[1:, 0] == w[:-1, 0] + w[:-1, 1])
    assert np.all(w[:, 1] <= caps["stage_window_rows"]) and np.all(w[:, 2] <= caps["stage_window"])
    assert np.all(w[1:, 3] == w[:-1, 3] + w[:-1, 2]) and w[0, 3] == 0
    rc = layout.row_count.numpy().view(np.uint16).astype(np.int64)
    assert np.all(rc[long_mask] == 0xFFFF)
    assert np.array_equal(rc[short], lengths[short])
    # staging ranges: whole groups of 8, inside the job's panel, covering the staged entries
    sj = layout.stage_jobs.numpy().astype(np.int64)
    jp = layout.job_panel.numpy().astype(np.int64)
    assert sj[0] == 0 and sj[-1] == layout.n_staged and np.all(sj % 8 == 0)
    assert np.all(np.diff(sj) >= 0) and np.all(np.diff(jp) >= 0)
    assert np.array_equal(np.unique(jp), np.arange(P))  # every panel has a job
    seg = layout.seg.numpy().astype(np.int64)
    for p in range(P):
        js = np.nonzero(jp == p)[0]
        lo, hi = sj[js[0]], sj[js[-1] + 1]
        assert lo <= seg[:, p].min() and seg[:, p].max() <= hi and hi - seg[-1, p] < 8
        assert np.all(np.diff(seg[:, p]) >= 0)
    # every short entry once, its LDS position its rank in (row, panel) order
    scol = layout.scol.numpy().view(np.uint16).astype(np.int64)
    v = layout.vals.numpy()
    dest = layout.dest.numpy().astype(np.int64)
    got = []
    for row0, nr, L, first, segs in _windows(layout):
        counts = np.where(rc[row0:row0 + nr] == 0xFFFF, 0, rc[row0:row0 + nr])
        row_of_pos = np.repeat(np.arange(row0, row0 + nr), counts)
        panel_at = np.full(L, -1)
        f = 0
        for p, g0, g1 in segs:
            for g in range(g0, g1):
                d = dest[first + f]
                assert 0 <= d < L and panel_at[d] == -1
                panel_at[d] = p
                got.append((int(row_of_pos[d]), int((p << cb) + scol[g]), float(v[first + f])))
                f += 1
        # inside each row, positions in panel order
        for r in range(nr):
            a = counts[:r].sum()
            assert np.all(np.diff(panel_at[a:a + counts[r]]) >= 0)
    want = [(r, int(cols[i]), float(vals[i])) for r in range(n_rows) if short[r]
            for i in range(rp[r], rp[r + 1])]
    assert sorted(got) == sorted(want)
    if layout.long is not None:
        _check_panels(layout.long, *_long_part(vals, cols, ip, torch.as_tensor(long_mask)))


def _run(layout, x, n_rows, row_map=None, n_out=None):
    y = np.full(n_rows if n_out is None else n_out, np.nan)
    y = _emulate(layout, x, y, row_map)
    if layout.long is not None:
        y = _emulate_panels(layout.long, x, y, row_map=row_map)
    return y


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_xstage_power_law_with_long_rows(seed):
    rng = np.random.default_rng(seed)
    n_cols = 300000  # 10 panels of 2^15 columns
    lengths = rng.zipf(1.6, 5000).clip(max=40000)
    lengths[rng.integers(0, 5000, 300)] = 0
    vals, cols, ip, x = _case(lengths, n_cols, seed)
    long_mask = lengths >= panel_row_min(n_cols, 4)
    assert 0 < long_mask.sum() < 5000
    lay = XstageLayout(vals, cols, ip, n_cols, torch.as_tensor(long_mask))
    assert lay.long is not None and lay.n_panels == 10
    # rows longer than a quarter window are in the panel part too
    assert lay.long.n_rows == int((long_mask | (lengths > 1024)).sum())
    _check(lay, vals.numpy(), cols.numpy(), ip, long_mask | (lengths > 1024))
    y = _run(lay, x.numpy(), lengths.size)
    np.testing.assert_allclose(y, oracle.spmv_csr(ip, cols, vals, x), rtol=1e-12, atol=1e-12)
    # through a row map (COO row runs): layout row r is output row map[r]
    rmap = np.arange(lengths.size) * 2
    y2 = _run(lay, x.numpy(), lengths.size, row_map=rmap, n_out=2 * lengths.size)
    np.testing.assert_array_equal(y2[rmap], y)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_xstage_short_rows_only(dtype):
    rng = np.random.default_rng(7)
    lengths = rng.integers(0, 40, 9000)
    n_cols = 70000
    vals, cols, ip, x = _case(lengths, n_cols, 3, dtype=dtype)
    long_mask = np.zeros(lengths.size, dtype=bool)
    lay = XstageLayout(vals, cols, ip, n_cols, torch.as_tensor(long_mask))
    assert lay.long is None
    assert lay.col_bits == (15 if dtype == torch.float32 else 14)
    _check(lay, vals.numpy(), cols.numpy(), ip, long_mask)
    y = _run(lay, x.numpy(), lengths.size)
    np.testing.assert_allclose(y, oracle.spmv_csr(ip, cols, vals, x), rtol=1e-12, atol=1e-12)
    assert np.all(y[lengths == 0] == 0.0)


def test_xstage_window_row_cap_and_small_x():
    # mostly empty rows: windows are cut by their row cap; x of one panel
    lengths = np.zeros(7000, dtype=np.int64)
    lengths[::97] = 3
    vals, cols, ip, x = _case(lengths, 5000, 5)
    lay = XstageLayout(vals, cols, ip, 5000, torch.zeros(7000, dtype=torch.bool))
    assert lay.n_panels == 1 and lay.n_windows >= 4
    _check(lay, vals.numpy(), cols.numpy(), ip, np.zeros(7000, dtype=bool))
    y = _run(lay, x.numpy(), 7000)
    np.testing.assert_allclose(y, oracle.spmv_csr(ip, cols, vals, x), rtol=1e-12, atol=1e-12)


def test_xstage_too_many_panels():
    vals, cols, ip, x = _case([2] * 10, 1 << 26, 1)  # 2048 panels of 2^15 columns
    with pytest.raises(ValueError):
        XstageLayout(vals, cols, ip, 1 << 26, torch.zeros(10, dtype=torch.bool))


def test_xstage_is_the_default_for_spread_columns(monkeypatch):
    vals, cols, ip, _ = _case([12] * 20000, 4 << 20, 2)
    assert _spmv_layouts.build_layout(vals, cols, ip, 4 << 20).kind == "xstage"
    monkeypatch.setattr(_spmv_layouts, "STAGED", False)
    assert _spmv_layouts.build_layout(vals, cols, ip, 4 << 20).kind == "xcs"
    monkeypatch.setattr(_spmv_layouts, "STAGED", True)
    monkeypatch.setattr(_spmv_layouts, "FORCE", "xcs")  # the XCS layouts stay reachable
    assert _spmv_layouts.build_layout(vals, cols, ip, 4 << 20).kind == "xcs"
