"""The staged-x SpMV layout (flagsparse_amd/_spmv_layouts.py, XstageLayout), built on the CPU and
checked without a GPU: the structure the kernels rely on (every short entry staged exactly once
and placed exactly once in its window, windows of consecutive rows within their caps, staged
chunks inside one panel whose segment marks, first segments and offsets send every entry to
its window position, LDS positions in (row, panel) order, one job per panel at least), and a
step-by-step emulation of spmv_panel_kernel's staging and stage_combine_kernel's sums (with
the panel part's long rows through the panel emulation) against the fp64 oracle."""

import numpy as np
import pytest
import torch

from flagsparse_amd import _abi, _spmv_layouts
from flagsparse_amd._spmv_layouts import XstageLayout, panel_row_min
from oracle import oracle
from test_xcs_layout_cpu import _case, _check_panels, _emulate_panels, _long_part


def _stage(layout, x):
    """spmv_panel_kernel's staging: job j stages chunks [stage_jobs[j], stage_jobs[j+1]) of its
    panel; entry e of a chunk (below the chunk's count in use) has segment s = the chunk's first
    segment plus the segment marks after the chunk's first entry up to e, and stores
    x[(panel << col_bits) + its column] at xs[e + seg_delta[s]].  Returns xs and, per window
    position, the staged entry stored there."""
    chunk = _abi.caps()["stage_chunk"]
    cb = layout.col_bits
    sc = layout.scol.numpy().view(np.uint16).astype(np.int64)
    col, mark = sc & 0x7FFF, (sc >> 15) & 1
    info = layout.stage_info.numpy().astype(np.int64)
    delta = layout.seg_delta.numpy().astype(np.int64)
    sj = layout.stage_jobs.numpy().astype(np.int64)
    jp = layout.job_panel.numpy().astype(np.int64)
    xs = np.full(layout.xs.numel(), np.nan)
    src = np.full(layout.xs.numel(), -1)
    for j in range(layout.n_jobs):
        for c in range(sj[j], sj[j + 1]):
            e0 = c * chunk
            seg = info[c, 0]
            for q in range(info[c, 1]):
                e = e0 + q
                if q > 0 and mark[e]:
                    seg += 1
                out = e + delta[seg]
                assert 0 <= out < layout.xs.numel() - 8 and src[out] == -1
                src[out] = e
                xs[out] = x[min((jp[j] << cb) + col[e], x.size - 1)]
    return xs, src


def _row_spans(layout, row0, nr):
    """The window's rows' positions [start, end) from row_end (a row starts where the one
    before ends, the first at 0) and which of them the window leaves alone (bit 15)."""
    re = layout.row_end.numpy().view(np.uint16).astype(np.int64)[row0:row0 + nr]
    end = re & 0x7FFF
    start = np.concatenate([[0], end[:-1]])
    return start, end, (re & 0x8000) != 0


def _emulate(layout, x, y, row_map=None, acc=np.float64):
    """stage_combine_kernel's windows: entry i of the window adds vals[i] * xs[i] at LDS
    position dest[i]; row r of the window gets its positions [row_end[r-1], row_end[r]) summed
    in order (bit 15: left alone)."""
    xs, _ = _stage(layout, x)
    xs = xs.astype(acc)
    vals = layout.vals.numpy().astype(acc)
    dest = layout.dest.numpy().astype(np.int64)
    for row0, nr, L, first in layout.windows.numpy().astype(np.int64):
        s = np.full(layout.window_cap, np.nan)
        for i in range(first, first + L):
            s[dest[i]] = acc(vals[i] * xs[i])
        start, end, skip = _row_spans(layout, row0, nr)
        for i in range(nr):
            if skip[i]:
                continue
            acc_v = acc(0)
            for u in range(start[i], end[i]):
                acc_v = acc(acc_v + s[u])
            out = row0 + i if row_map is None else row_map[row0 + i]
            y[out] = acc_v
        assert end[-1] == L
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
    assert np.all(w[:, 1] <= layout.window_cap // 2) and np.all(w[:, 2] <= layout.window_cap)
    # window starts: packed at multiples of 8 entries
    assert np.all(w[1:, 3] == w[:-1, 3] + (w[:-1, 2] + 7) // 8 * 8) and w[0, 3] == 0
    assert layout.vals.numel() == layout.n_positions + 8 == layout.xs.numel()
    assert layout.n_positions == w[-1, 3] + (w[-1, 2] + 7) // 8 * 8
    # row ends: the rows' lengths (none for the long rows, marked), and the row-start bits
    # exactly where a row with entries starts
    heads = layout.heads.numpy()
    hb = layout.window_cap // 8
    counts_all = np.zeros(n_rows, dtype=np.int64)
    for k, (row0, nr, L, first) in enumerate(w):
        start, end, skip = _row_spans(layout, row0, nr)
        assert np.array_equal(skip, long_mask[row0:row0 + nr]) and end[-1] == L
        counts_all[row0:row0 + nr] = end - start
        bits = np.unpackbits(heads[k * hb:(k + 1) * hb], bitorder="little")
        want_bits = np.zeros(layout.window_cap, dtype=np.uint8)
        want_bits[start[end > start]] = 1
        assert np.array_equal(bits, want_bits)
    assert np.all(counts_all[long_mask] == 0)
    assert np.array_equal(counts_all[short], lengths[short])
    # staged chunks: each job's inside its panel, every panel with a job, chunks covering
    # the staged entries; every window position written by exactly one staged entry
    chunk = caps["stage_chunk"]
    sj = layout.stage_jobs.numpy().astype(np.int64)
    jp = layout.job_panel.numpy().astype(np.int64)
    assert sj[0] == 0 and sj[-1] * chunk == layout.n_staged
    assert np.all(np.diff(sj) >= 0) and np.all(np.diff(jp) >= 0)
    assert np.array_equal(np.unique(jp), np.arange(P))  # every panel has a job
    x_probe = np.arange(layout.n_cols, dtype=np.float64)  # x[c] = c names the column
    xs, src = _stage(layout, x_probe)
    written = np.zeros(src.size, dtype=bool)
    for row0, nr, L, first in w:
        written[first:first + L] = True
    assert np.all(src[written] >= 0) and np.all(src[~written] == -1)
    assert int(written.sum()) == layout.n_entries
    # every short entry once, its LDS position its rank in (row, panel) order
    v = layout.vals.numpy()
    dest = layout.dest.numpy().astype(np.int64)
    got = []
    for row0, nr, L, first in layout.windows.numpy().astype(np.int64):
        counts = counts_all[row0:row0 + nr]
        row_of_pos = np.repeat(np.arange(row0, row0 + nr), counts)
        panel_at = np.full(L, -1)
        for i in range(first, first + L):
            d = dest[i]
            assert 0 <= d < L and panel_at[d] == -1
            col = int(xs[i])
            panel_at[d] = col >> cb
            got.append((int(row_of_pos[d]), col, float(v[i])))
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


@pytest.fixture(params=[None, 8192], ids=["auto-window", "window8192"])
def window(request, monkeypatch):
    """Each test with the window size the layout picks, and with the largest (1024-thread
    combine workgroups)."""
    monkeypatch.setattr(_spmv_layouts, "FORCE_STAGE_WINDOW", request.param)
    return request.param


@pytest.mark.parametrize("seed,unsorted", [(0, False), (1, False), (2, False), (0, True)])
def test_xstage_power_law_with_long_rows(seed, unsorted, window):
    # unsorted: each row's columns in falling order (the (row, panel) ranks then need a sort)
    rng = np.random.default_rng(seed)
    n_cols = 300000  # 10 panels of 2^15 columns
    lengths = rng.zipf(1.6, 5000).clip(max=40000)
    lengths[rng.integers(0, 5000, 300)] = 0
    vals, cols, ip, x = _case(lengths, n_cols, seed, unsorted=unsorted)
    long_mask = lengths >= panel_row_min(n_cols, 4)
    assert 0 < long_mask.sum() < 5000
    lay = XstageLayout(vals, cols, ip, n_cols, torch.as_tensor(long_mask))
    assert lay.long is not None and lay.n_panels == 10
    # rows longer than an eighth of the largest window are in the panel part too
    assert lay.long.n_rows == int((long_mask | (lengths > 1024)).sum())
    _check(lay, vals.numpy(), cols.numpy(), ip, long_mask | (lengths > 1024))
    y = _run(lay, x.numpy(), lengths.size)
    np.testing.assert_allclose(y, oracle.spmv_csr(ip, cols, vals, x), rtol=1e-12, atol=1e-12)
    # through a row map (COO row runs): layout row r is output row map[r]
    rmap = np.arange(lengths.size) * 2
    y2 = _run(lay, x.numpy(), lengths.size, row_map=rmap, n_out=2 * lengths.size)
    np.testing.assert_array_equal(y2[rmap], y)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_xstage_short_rows_only(dtype, window):
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


def test_xstage_window_row_cap_and_small_x(window):
    # mostly empty rows: windows are cut by their row cap; x of one panel
    lengths = np.zeros(17000, dtype=np.int64)
    lengths[::97] = 3
    vals, cols, ip, x = _case(lengths, 5000, 5)
    lay = XstageLayout(vals, cols, ip, 5000, torch.zeros(17000, dtype=torch.bool))
    assert lay.n_panels == 1 and lay.n_windows >= 4
    assert int(lay.windows[:, 1].max()) == lay.window_cap // 2  # windows cut by rows
    _check(lay, vals.numpy(), cols.numpy(), ip, np.zeros(17000, dtype=bool))
    y = _run(lay, x.numpy(), 17000)
    np.testing.assert_allclose(y, oracle.spmv_csr(ip, cols, vals, x), rtol=1e-12, atol=1e-12)


def test_xstage_chunks_of_many_segments(window):
    # sparse rows: windows cut by their row cap, each panel's entries spread over ~150 windows
    # in segments of one or two entries, so that chunks close at the kernel's 64 segments and
    # end in padding
    n = 600000
    lengths = np.zeros(n, dtype=np.int64)
    lengths[::40] = 1
    lengths[5::200] = 3
    vals, cols, ip, x = _case(lengths, 1 << 21, 1)
    lay = XstageLayout(vals, cols, ip, 1 << 21, torch.zeros(n, dtype=torch.bool))
    assert lay.n_panels == 64
    info = lay.stage_info.numpy().astype(np.int64)
    segs_in_chunk = np.diff(np.append(info[:, 0], lay.n_segments))
    # a chunk's segments: those starting in it, plus the one its first entry continues
    sc = lay.scol.numpy().view(np.uint16).astype(np.int64)[:lay.n_staged].reshape(-1, 512)
    pieces = (sc[:, 1:] >> 15).sum(1) + 1
    assert pieces.max() == 64 and (info[:, 1] < 512).sum() > lay.n_panels
    assert np.all(segs_in_chunk <= pieces)
    _check(lay, vals.numpy(), cols.numpy(), ip, np.zeros(n, dtype=bool))
    y = _run(lay, x.numpy(), n)
    np.testing.assert_allclose(y, oracle.spmv_csr(ip, cols, vals, x), rtol=1e-12, atol=1e-12)


def test_xstage_is_the_default_for_spread_columns(monkeypatch):
    vals, cols, ip, _ = _case([12] * 20000, 4 << 20, 2)
    assert _spmv_layouts.build_layout(vals, cols, ip, 4 << 20).kind == "xstage"
    monkeypatch.setattr(_spmv_layouts, "STAGED", False)
    assert _spmv_layouts.build_layout(vals, cols, ip, 4 << 20).kind == "xcs"
    monkeypatch.setattr(_spmv_layouts, "STAGED", True)
    monkeypatch.setattr(_spmv_layouts, "FORCE", "xcs")  # the XCS layouts stay reachable
    assert _spmv_layouts.build_layout(vals, cols, ip, 4 << 20).kind == "xcs"
