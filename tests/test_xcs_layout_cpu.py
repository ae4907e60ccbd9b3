"""The XCD column-split and panel SpMV layouts (flagsparse_amd/_spmv_layouts.py), built on the
CPU and checked without a GPU: structural invariants the kernels rely on (every entry exactly
once, item capacity and alignment, in-bounds packed indices, panel-to-XCD slot order; for
panels, chunk-aligned panel runs padded with zero entries of their last row, jobs inside one
panel, chunk slot offsets), and step-by-step emulations of spmv_xcs_kernel's and
spmv_panel_kernel's semantics over the layouts (one partial slot per run, each row's slots
added in order through the combine's row table, rows without entries written as 0) - for the hybrid, the XCS part and then
the panel part - against the fp64 oracle."""

import numpy as np
import pytest
import torch

from flagsparse_amd import _abi, synthetic
from flagsparse_amd import _spmv_layouts
from flagsparse_amd._spmv_layouts import (PanelLayout, XcsHybridLayout, XcsLayout,
                                          panel_row_min, prefers_xcs, sample_indices)
from oracle import oracle


@pytest.fixture(autouse=True, params=[0, 1], ids=["rows", "sorted"])
def item_format(request, monkeypatch):
    """Every test runs with both XCS item formats: 0 (entries in row order, rows packed in
    the index words) and 1 (gathers in column order; wherever the panels allow it)."""
    monkeypatch.setattr(_spmv_layouts, "SORTED_ITEMS", request.param == 1)
    monkeypatch.setattr(_spmv_layouts, "SORTED_MIN_RUN", 0.0)  # whatever the row lengths
    return request.param


def _sorted_item(layout, e0, ln):
    """Decode a format-1 item: (memory positions of its values in row order, column in the
    panel and run-start flag of each row-order position).  Values: position 8t + e at quad
    (e/4) * P/8 + t; gather words in column order at the same quads, entry (t/64)*512 + 64k +
    t%64 as element k of thread t.  Checks that the words name every row-order position once,
    in non-decreasing column order."""
    sb = _abi.caps()["xcs_sorted_col_bits"]
    P = -(-ln // 512) * 512
    thr = P // 8
    o = np.arange(ln)
    vpos = e0 + 4 * ((o % 8) // 4 * thr + o // 8) + o % 4
    t_g = (o // 512) * 64 + o % 64
    k = (o % 512) // 64
    gpos = e0 + 4 * (k // 4 * thr + t_g) + k % 4
    w = layout.pidx.numpy().view(np.uint32)[gpos].astype(np.int64)
    pos = w >> (sb + 1)
    colg = w & ((1 << sb) - 1)
    assert sorted(pos.tolist()) == list(range(ln))  # a permutation of the positions
    assert np.all(np.diff(colg) >= 0)               # gathers in column order
    col = np.empty(ln, dtype=np.int64)
    col[pos] = colg
    flag = np.empty(ln, dtype=bool)
    flag[pos] = ((w >> sb) & 1) == 1
    assert ln == 0 or flag[0]
    return vpos, col, flag


def _window_row_starts(layout, row0, nr):
    """First LDS position of each row of a window: the exclusive sum of the window's row counts
    (row_count, one byte per row; ROW_SKIP counts as none), as the combine scans them."""
    cnt = layout.row_count.numpy().astype(np.int64)[row0:row0 + nr]
    cnt = np.where(cnt == _spmv_layouts.ROW_SKIP, 0, cnt)
    return np.concatenate([[0], np.cumsum(cnt)])


def _combine_slot_rows(layout):
    """The row of every stored slot according to the combine tables (-1: padding or unused):
    slot s of window w is at position dest[s], inside row r's row_count[r] positions."""
    windows = layout.windows.numpy().reshape(-1, 8).astype(np.int64)
    dest = layout.dest.numpy().astype(np.int64)
    rows = np.full(layout.n_partials, -1, dtype=np.int64)
    for row0, nr, base, ln, total, _, _, _ in windows:
        sl = np.arange(base, base + ln)
        if nr < 0:
            rows[sl] = row0
            continue
        d = dest[sl]
        ok = d >= 0
        starts = _window_row_starts(layout, row0, nr)[:-1]
        rows[sl[ok]] = row0 + np.searchsorted(starts, d[ok], side="right") - 1
    return rows


def _item_positions(e0, ln):
    """Memory positions of an item's entries in logical (row) order: thread-major storage with
    Q = ceil(ln/4) quads, qp = ceil(Q/256) quads per thread, nt = ceil(Q/qp) threads, logical
    quad qp*t + u at memory quad t + nt*u."""
    q = (ln + 3) // 4
    qp = max(1, (q + 255) // 256)
    nt = (q + qp - 1) // qp
    o = np.arange(ln)
    lq = o // 4
    return e0 + 4 * (lq // qp + nt * (lq % qp)) + o % 4


def _emulate(layout, x, acc=np.float64, y=None, row_map=None):
    """numpy restatement of spmv_xcs_kernel + xcs_window_combine_kernel over the layout: every
    item sums each row run it holds (in row order) and stores the sums through its runs
    (item_runs: {first slot, first sum, sums, stored length}, zeros after the sums); each combine
    window then places its stored slots at their dest positions (-1: padding) and row r gets
    the sum of its row_count[r] positions (from the sum of the window's counts before it) in
    order - its sums in item order -, 0 without any, at y[row_map[r]] when a row map is given.
    A big window (rows -1) is one row given the sum of all its slots."""
    caps = _spmv_layouts._abi.caps()
    items = layout.items.numpy().reshape(-1, 12).astype(np.int64)
    item_runs = layout.item_runs.numpy().astype(np.int64)
    vals = layout.vals.numpy().astype(acc)
    pidx = layout.pidx.numpy().view(np.uint32)
    cbits = layout.col_bits
    out = (lambda r: r) if row_map is None else (lambda r: int(row_map[r]))  # noqa: E731
    y = np.full(layout.n_rows, np.nan) if y is None else y
    n_store = layout.n_partials
    partials = np.full(n_store, np.nan)
    slot_row = np.full(n_store, -1, dtype=np.int64)  # -2: padding
    slot_item = np.full(n_store, -1, dtype=np.int64)
    comb_rows = _combine_slot_rows(layout) if layout.item_format == 1 else None
    for e0, ln, k, run0, r0, R, cbase, n_ir, _, _, tile, _ in items:
        if tile < 0:
            continue
        assert 0 <= n_ir <= caps["xcs_item_runs"]
        if layout.item_format == 1:
            assert ln <= caps["xcs_sorted_item"]
            pos, colp, flag = _sorted_item(layout, e0, ln)
            col = cbase + colp
            run_of = np.cumsum(flag) - 1  # run index of every row-order position
        else:
            pos = _item_positions(e0, ln)
            p = pidx[pos]
            lrow = (p >> cbits).astype(np.int64)
            col = cbase + (p & ((1 << cbits) - 1)).astype(np.int64)
            assert np.all(np.diff(lrow) >= 0) and np.all(lrow < R)
            run_of = np.unique(lrow, return_inverse=True)[1].ravel()
        prod = vals[pos] * x[col].astype(acc)
        sums = []
        for r in range(int(run_of.max()) + 1 if ln else 0):  # runs in row order
            s = acc(0)
            for v in prod[run_of == r]:
                s = acc(s + v)
            sums.append(s)
        if layout.item_format == 1:  # a run's row: where the combine tables place its sum
            rows = [None] * len(sums)
            for first, s0, cnt, stored in item_runs[run0:run0 + n_ir]:
                for j in range(cnt):
                    rows[s0 + j] = int(comb_rows[first + j])
            assert all(r is not None and r >= 0 for r in rows)
            assert all(a < b for a, b in zip(rows, rows[1:]))  # one sum per row, in row order
        else:
            rows = [r0 + int(r) for r in np.unique(lrow)]
        nxt = 0
        for first, s0, cnt, stored in item_runs[run0:run0 + n_ir]:
            assert s0 == nxt and stored >= cnt  # the runs take the sums in order
            for j in range(stored):
                assert slot_row[first + j] == -1  # one writer per slot
                if j < cnt:
                    partials[first + j] = sums[s0 + j]
                    slot_row[first + j] = rows[s0 + j]
                    slot_item[first + j] = run0  # increases with the item number
                else:
                    partials[first + j] = 0.0
                    slot_row[first + j] = -2
            nxt = s0 + cnt
        assert nxt == len(sums)
    # the combine windows: consecutive rows and consecutive stored ranges, each starting on
    # a line (WINDOW_ALIGN slots), every slot once; the slots between windows are never written
    # and their dest is -1
    windows = layout.windows.numpy().reshape(-1, 8).astype(np.int64)
    dest = layout.dest.numpy().astype(np.int64)
    row_count = layout.row_count.numpy().astype(np.int64)
    line = _spmv_layouts.WINDOW_ALIGN
    next_row, next_slot = 0, 0
    for row0, nr, base, ln, total, _, _, _ in windows:
        assert row0 == next_row and base == -(-next_slot // line) * line
        gap = np.arange(next_slot, base)
        assert np.all(slot_row[gap] == -1) and np.all(dest[gap] == -1)
        sl = np.arange(base, base + ln)
        next_slot = base + ln
        real = sl[slot_row[sl] >= 0] if ln else sl
        assert real.size == total
        if nr < 0:  # one row with more sums than a window holds, or than a count byte
            assert total > min(layout.window_slots, _spmv_layouts.ROW_COUNT_MAX) and ln == total
            assert row_count[row0] == 0
            assert np.all(slot_row[sl] == row0)
            s = acc(0)
            for v in partials[sl]:
                s = acc(s + v)
            y[out(row0)] = s
            next_row = row0 + 1
            continue
        assert total <= layout.window_slots <= caps["xcs_window_slots"]
        assert 1 <= nr <= caps["xcs_window_rows"]
        assert np.all(dest[sl][slot_row[sl] == -2] == -1)  # padding dropped
        d = dest[real]
        assert sorted(d.tolist()) == list(range(total))  # a permutation of the positions
        lds = np.full(total, np.nan)
        lds[d] = partials[real]
        lds_slot = np.full(total, -1, dtype=np.int64)
        lds_slot[d] = real
        starts = _window_row_starts(layout, row0, nr)
        assert starts[-1] == total and row_count[row0:row0 + nr].max() <= 255
        for i in range(nr):
            a, b = starts[i], starts[i + 1]
            if row_count[row0 + i] == _spmv_layouts.ROW_SKIP:  # written by the panel rows
                assert a == b
                continue
            mine = lds_slot[a:b]
            # the row's own sums, all of them, in item order
            assert np.all(slot_row[mine] == row0 + i)
            assert np.all(np.diff(slot_item[mine]) > 0)
            assert mine.size == int(np.sum(slot_row[sl] == row0 + i))
            s = acc(0)
            for v in lds[a:b]:
                s = acc(s + v)
            y[out(row0 + i)] = s
        next_row = row0 + nr
    tail = -(-next_slot // line) * line
    assert next_row == layout.n_rows and tail == n_store or n_store == 1
    assert np.all(dest[next_slot:] == -1) and np.all(slot_row[next_slot:] == -1)
    return y


def _check_structure(layout, data, cols, rowptr):
    caps = _abi.caps()
    items = layout.items.numpy().reshape(-1, 12).astype(np.int64)
    real = items[items[:, 10] >= 0]
    cap = caps["xcs_sorted_item"] if layout.item_format == 1 else caps["xcs_item"]
    assert np.all(real[:, 0] % 4 == 0) and np.all(real[:, 1] <= cap)
    assert np.all(real[:, 5] <= layout.rows_cap)
    # slot x*q + j runs on XCD x: every real item of XCD x's range gathers from a panel
    # p with p % 8 == x, and the panels come one after the other
    q = layout.max_items_per_panel
    cbl = list(layout.panel_base.numpy())
    for x in range(8):
        seq = [it for it in items[x * q:(x + 1) * q] if it[10] >= 0]
        panels = [max(i for i, b in enumerate(cbl) if b == it[6]) for it in seq]
        home = (lambda p: p % 8 == x) if layout.n_panels >= 8 else \
            (lambda p: p == x % layout.n_panels)  # a panel shared by 8 / P XCDs
        assert all(home(p) or cbl.count(cbl[p]) > 1 for p in panels)
        assert panels == sorted(panels) or any(cbl.count(b) > 1 for b in cbl)
    # every original entry appears exactly once (multiset of (row, col, value))
    pidx = layout.pidx.numpy().view(np.uint32)
    vals = layout.vals.numpy()
    cb = layout.panel_base.numpy()
    got = []
    if layout.item_format == 1:
        assert np.all(real[:, 0] % 512 == 0) and np.all(real[:, 1] <= caps["xcs_sorted_item"])
        comb_rows = _combine_slot_rows(layout)
        item_runs = layout.item_runs.numpy().astype(np.int64)
    for e0, ln, k, S, r0, R, cbase, moff, plo, phi, tile, _ in real:
        panel = max(i for i, b in enumerate(cb) if b == cbase)
        if layout.item_format == 1:
            pos, colp, flag = _sorted_item(layout, e0, ln)
            c = cbase + colp
            run_of = np.cumsum(flag) - 1
            run_row = np.full(int(run_of.max()) + 1 if ln else 0, -1, dtype=np.int64)
            for first, s0, cnt, stored in item_runs[S:S + moff]:
                run_row[s0:s0 + cnt] = comb_rows[first:first + cnt]
            assert np.all(run_row >= r0) and np.all(run_row < r0 + R)
            rows_e = run_row[run_of]
        else:
            pos = _item_positions(e0, ln)
            p = pidx[pos]
            lr = (p >> layout.col_bits).astype(np.int64)
            assert np.all(lr < R)
            c = cbase + (p & ((1 << layout.col_bits) - 1)).astype(np.int64)
            rows_e = r0 + lr
        assert pos.size == 0 or pos.max() < layout.n_entries
        hi = cb[panel + 1] if panel + 1 < len(cb) else layout.n_cols
        assert np.all((c >= cbase) & (c < hi))
        got += list(zip(rows_e.tolist(), c.tolist(), vals[pos].tolist()))
    rp = rowptr.numpy()
    want = [(r, int(cols[i]), float(data[i])) for r in range(rp.size - 1)
            for i in range(rp[r], rp[r + 1])]
    assert sorted(got) == sorted(want)


def _emulate_panels(layout, x, y, row_map=None, acc=np.float64):
    """numpy restatement of spmv_panel_kernel + the combine over a PanelLayout: each chunk's
    runs (a chunk start or an entry marked as a run start opens one) go to consecutive slots
    from chunk_info[c, 0], its entries from chunk_info[c, 1] on (padding) adding 0; row i of the
    layout then gets its slots' sum in slot order."""
    chunk = _abi.caps()["panel_chunk"]
    cb = layout.col_bits
    vals, pidx, start = _panel_logical(layout)
    vals = vals.astype(acc)
    jobs = layout.jobs.numpy()
    jp = layout.job_panel.numpy()
    info = layout.chunk_info.numpy()
    cslot = info[:, 0]
    partials = np.full(max(layout.n_partials, 1), np.nan)
    for j in range(layout.n_jobs):
        base = int(jp[j]) << cb
        for c in range(jobs[j], jobs[j + 1]):
            sl = int(cslot[c])
            e = np.arange(c * chunk, (c + 1) * chunk)
            cols = base + (pidx[e] & ((1 << cb) - 1))
            in_use = np.arange(chunk) < info[c, 1]
            with np.errstate(invalid="ignore"):
                prod = np.where(in_use, vals[e] * x[np.minimum(cols, x.size - 1)].astype(acc),
                                acc(0))
            assert np.all(cols[in_use] < x.size)
            s = acc(0)
            for q in range(chunk):
                if q > 0 and start[e[q]]:
                    partials[sl] = s
                    sl += 1
                    s = acc(0)
                s = acc(s + prod[q])
            partials[sl] = s
            assert c + 1 == len(cslot) or sl + 1 == cslot[c + 1]
    out = layout.rows.numpy() if row_map is None else row_map[layout.rows.numpy()]
    rp = layout.row_ptr.numpy()
    slots = layout.slots.numpy()
    for i in range(layout.n_rows):
        s = acc(0)
        for k in range(rp[i], rp[i + 1]):
            s = acc(s + partials[slots[k]])
        y[out[i]] = s
    return y


def _panel_logical(layout):
    """(vals, pidx = row << col_bits | column in the panel, run-start flags) of a PanelLayout
    in logical order.  Values: inside a chunk of 512, lane L's quad h (logical quad 2L + h) is
    read from quad 64h + L.  The 16-bit entries hold no row: an entry's row is that of its
    slot (chunk_info[c, 0] of its chunk + the run starts before it in the chunk), read back through
    the combine tables (row_ptr, slots) - so the check below also checks that the run starts
    and the slot tables agree."""
    n = layout.n_entries
    if n == 0:
        return layout.vals.numpy()[:0], np.zeros(0, np.int64), np.zeros(0, bool)
    p = np.arange(n)
    lq = (p % 512) // 4
    mem = (p // 512) * 512 + ((lq % 2) * 64 + lq // 2) * 4 + p % 4
    pc = layout.pcol.numpy().view(np.uint16)[:n].astype(np.int64)
    start = (pc & 0x8000) != 0
    col = pc & 0x7FFF
    assert np.all(col < (1 << layout.col_bits))
    assert np.all(start[::512])  # every chunk opens a run
    run_in_chunk = np.cumsum(start.reshape(-1, 512), axis=1).reshape(-1) - 1
    slot = layout.chunk_info.numpy()[:, 0].astype(np.int64)[p // 512] + run_in_chunk
    rp, slots = layout.row_ptr.numpy(), layout.slots.numpy()
    slot_row = np.full(layout.n_partials, -1, dtype=np.int64)
    for i in range(layout.n_rows):
        slot_row[slots[rp[i]:rp[i + 1]]] = i
    assert np.all(slot_row >= 0)
    row = slot_row[slot]
    return layout.vals.numpy()[:n][mem], (row << layout.col_bits) | col, start


def _check_panels(layout, data, cols, rowptr):
    """Panel runs chunk-aligned and padded with zero entries of their last row; jobs of one
    panel covering every chunk once; every entry exactly once; the x panel fits the LDS copy."""
    caps = _abi.caps()
    chunk = caps["panel_chunk"]
    cb = layout.col_bits
    assert (1 << cb) * layout.vals.element_size() <= caps["panel_bytes"]
    assert layout.n_entries % chunk == 0
    jobs, jp = layout.jobs.numpy().astype(np.int64), layout.job_panel.numpy()
    assert jobs[0] == 0 and jobs[-1] == layout.n_entries // chunk
    assert np.all(np.diff(jobs) >= 1)
    assert np.all(np.diff(jobs) <= _spmv_layouts.PANEL_JOB_CHUNKS)
    assert np.all(np.diff(jp) >= 0)
    vals, pidx, start = _panel_logical(layout)
    e = np.arange(layout.n_entries)
    rows_all = pidx >> cb
    # a run starts exactly where the row changes or a chunk opens; no chunk holds more runs
    # than the kernel stages
    assert np.array_equal(start, (e % chunk == 0) | np.r_[True, rows_all[1:] != rows_all[:-1]])
    if layout.n_entries:
        assert start.reshape(-1, chunk).sum(1).max() <= caps["panel_chunk_runs"]
    assert np.array_equal(np.sort(_spmv_layouts.panel_storage_positions(
        layout.n_entries, chunk, "cpu").numpy()), np.arange(layout.n_entries))  # a permutation
    # entries in use: each chunk's first chunk_info[c, 1]; the rest (its tail) padding of
    # value 0 in the row of the last run
    info = layout.chunk_info.numpy().astype(np.int64)
    assert np.all((info[:, 1] >= 1) & (info[:, 1] <= chunk))
    in_use = (e % chunk) < np.repeat(info[:, 1], chunk)
    assert np.all(vals[~in_use] == 0)
    got = []
    for j in range(layout.n_jobs):
        e = np.arange(jobs[j] * chunk, jobs[j + 1] * chunk)
        rows = pidx[e] >> cb
        assert np.all(np.diff(rows) >= 0)  # a job lies in one panel, whose rows ascend
        cols_e = (int(jp[j]) << cb) + (pidx[e] & ((1 << cb) - 1))
        u = in_use[e]
        got += list(zip(rows[u].tolist(), cols_e[u].tolist(), vals[e][u].tolist()))
    rp = rowptr.numpy()
    want = [(r, int(cols[i]), float(data[i])) for r in range(rp.size - 1)
            for i in range(rp[r], rp[r + 1])]
    assert sorted(got) == sorted(want)  # every entry once, explicit zeros included


def _case(lengths, n_cols, seed, dtype=torch.float32, unsorted=False):
    lengths = torch.as_tensor(lengths, dtype=torch.int64)
    keys = synthetic._distinct_sorted_columns(lengths, n_cols, seed, 1)
    ip, cols = synthetic._csr_from_keys(keys, lengths.numel(), n_cols)
    if unsorted:  # reverse each row's columns
        for r in range(lengths.numel()):
            a, b = int(ip[r]), int(ip[r + 1])
            cols[a:b] = cols[a:b].flip(0)
    vals = synthetic.uniform_values(seed, 2, cols.numel(), dtype, "cpu")
    x = synthetic.uniform_values(seed, 3, n_cols, dtype, "cpu")
    return vals, cols.to(torch.int32), ip, x


@pytest.mark.parametrize("seed,per_xcd", [(0, 1), (1, 1), (0, 2), (1, 4), (2, None)])
def test_xcs_random_short_rows(seed, per_xcd):
    rng = np.random.default_rng(seed)
    lengths = rng.zipf(2.0, 6000).clip(max=300)
    lengths[rng.integers(0, 6000, 400)] = 0
    vals, cols, ip, x = _case(lengths, 50000, seed)
    lay = XcsLayout(vals, cols, ip, 50000, panels_per_xcd=per_xcd)
    assert lay.n_panels == (8 * per_xcd if per_xcd else 4)  # small x: 4 shared panels
    _check_structure(lay, vals, cols, ip)
    assert lay.n_split_rows > 0
    y = _emulate(lay, x.numpy())
    ref = oracle.spmv_csr(ip, cols, vals, x)
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)


def test_xcs_long_rows_and_empty_tiles():
    # long rows beyond a tile (8 * item cap), item splits, a run of empty rows wider than a tile
    lengths = [3, 0, 40000, 1, 1, 2] + [0] * 9000 + [17000, 5, 0, 2048 * 3, 7]
    vals, cols, ip, x = _case(lengths, 300000, 4, unsorted=True)
    lay = XcsLayout(vals, cols, ip, 300000, panels_per_xcd=2)
    _check_structure(lay, vals, cols, ip)
    y = _emulate(lay, x.numpy())
    ref = oracle.spmv_csr(ip, cols, vals, x)
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)


def test_xcs_skewed_columns_and_empty_matrix():
    # every entry in a narrow column range: most panels empty
    n_cols = 200000
    lengths = torch.full((3000,), 4, dtype=torch.int64)
    keys = synthetic._distinct_sorted_columns(lengths, 64, 9, 1)
    ip, cols = synthetic._csr_from_keys(keys, 3000, 64)
    cols = (cols + 1000).to(torch.int32)
    vals = synthetic.uniform_values(9, 2, cols.numel(), torch.float64, "cpu")
    x = synthetic.uniform_values(9, 3, n_cols, torch.float64, "cpu")
    lay = XcsLayout(vals, cols, ip, n_cols)
    _check_structure(lay, vals, cols, ip)
    np.testing.assert_allclose(_emulate(lay, x.numpy()), oracle.spmv_csr(ip, cols, vals, x),
                               rtol=1e-12, atol=1e-12)
    # no entries at all: every row written as 0 by its tile's dummy item
    ip0 = torch.zeros(5001, dtype=torch.int64)
    lay = XcsLayout(torch.empty(0), torch.empty(0, dtype=torch.int32), ip0, 100)
    assert np.all(_emulate(lay, np.ones(100)) == 0.0)


@pytest.mark.parametrize("win_slots,win_rows", [(8, 2048), (64, 16), (4096, 3)])
def test_xcs_combine_windows(win_slots, win_rows, monkeypatch):
    # small combine windows: rows with more slots than a window holds become one-row windows
    # (summed whole), tiles cut into several windows, windows of a few rows
    monkeypatch.setattr(_spmv_layouts, "WINDOW_SLOTS", win_slots)
    monkeypatch.setattr(_spmv_layouts, "WINDOW_ROWS", win_rows)
    # tiny windows make an item reach more of them than the kernel's run table holds; the
    # emulation checks the layout logic, so the cap is lifted here
    real = _abi.caps()
    monkeypatch.setattr(_spmv_layouts._abi, "caps", lambda: dict(real, xcs_item_runs=1 << 20))
    lengths = [3, 0, 40000, 1, 1, 2] + [0] * 900 + [17000, 5, 0, 2048 * 3, 7] + [9] * 3000
    vals, cols, ip, x = _case(lengths, 300000, 5, unsorted=True)
    lay = XcsLayout(vals, cols, ip, 300000, panels_per_xcd=2)
    _check_structure(lay, vals, cols, ip)
    w = lay.windows.numpy().reshape(-1, 8)
    assert (w[:, 1] < 0).any() == (win_slots == 8)  # one-row windows only when rows exceed 8
    assert lay.n_windows > lay.n_tiles
    y = _emulate(lay, x.numpy())
    np.testing.assert_allclose(y, oracle.spmv_csr(ip, cols, vals, x), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("count_max", [3, 8])
def test_xcs_rows_over_the_count_byte(count_max, monkeypatch):
    # the combine reads one byte of sum count per row: a row with more sums than
    # ROW_COUNT_MAX (lowered here) is a window of its own, summed whole; the other rows keep
    # their counts and windows
    monkeypatch.setattr(_spmv_layouts, "ROW_COUNT_MAX", count_max)
    lengths = [3, 0, 400, 1, 1, 2] + [0] * 90 + [170, 5, 0, 61, 7] + [1] * 3000 + [2] * 300
    vals, cols, ip, x = _case(lengths, 300000, 6, unsorted=True)
    lay = XcsLayout(vals, cols, ip, 300000, panels_per_xcd=2)
    _check_structure(lay, vals, cols, ip)
    w = lay.windows.numpy().reshape(-1, 8)
    assert (w[:, 1] < 0).sum() > 0
    assert lay.row_count.numpy().max() <= count_max
    y = _emulate(lay, x.numpy())
    np.testing.assert_allclose(y, oracle.spmv_csr(ip, cols, vals, x), rtol=1e-12, atol=1e-12)


def test_xcs_item_run_cap(monkeypatch, item_format):
    # an item stores its sums through at most the kernel's number of runs (one per combine
    # window its rows reach); a layout that needs more is refused, and build_layout then takes
    # the row-order items (shorter tiles, fewer windows per item) or, when those do not fit
    # either, row blocks
    real = _abi.caps()
    rng = np.random.default_rng(3)
    lengths = rng.zipf(2.0, 20000).clip(max=200)
    vals, cols, ip, x = _case(lengths, 60000, 3)
    lay = XcsLayout(vals, cols, ip, 60000, panels_per_xcd=1)
    assert lay.item_format == item_format
    most = int(lay.item_n_runs.max())
    assert 2 <= most <= real["xcs_item_runs"]
    fmt0 = XcsLayout(vals, cols, ip, 60000, panels_per_xcd=1, item_format=0)
    most0 = int(fmt0.item_n_runs.max())
    monkeypatch.setattr(_spmv_layouts._abi, "caps", lambda: dict(real, xcs_item_runs=most - 1))
    with pytest.raises(ValueError):
        XcsLayout(vals, cols, ip, 60000, panels_per_xcd=1)
    monkeypatch.setattr(_spmv_layouts, "FORCE", "xcs-l2")
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANELS_PER_XCD", 1)
    got = _spmv_layouts.build_layout(vals, cols, ip, 60000)
    if item_format == 1 and most0 < most:
        assert got.kind == "xcs" and got.item_format == 0
        np.testing.assert_allclose(_emulate(got, x.numpy()), oracle.spmv_csr(ip, cols, vals, x),
                                   rtol=1e-12, atol=1e-12)
    else:
        assert got.kind == "rowblock"
    monkeypatch.setattr(_spmv_layouts._abi, "caps",
                        lambda: dict(real, xcs_item_runs=min(most, most0) - 1))
    assert _spmv_layouts.build_layout(vals, cols, ip, 60000).kind == "rowblock"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_panel_layout(dtype, monkeypatch):
    # long rows over 200k columns (15 or 14 bits per panel), jobs cut at PANEL_JOB_CHUNKS
    monkeypatch.setattr(_spmv_layouts, "PANEL_JOB_CHUNKS", 3)
    lengths = [9000, 20000, 5000, 0, 12000, 30000, 7]
    vals, cols, ip, x = _case(lengths, 200000, 6, dtype)
    rows = torch.arange(len(lengths)) * 3 + 1  # output rows of the layout's rows
    lay = PanelLayout(vals, cols, ip, 200000, rows)
    assert lay.n_jobs > lay.n_panels
    _check_panels(lay, vals, cols, ip)
    y = np.full(3 * len(lengths) + 1, np.nan)
    _emulate_panels(lay, x.numpy(), y)
    np.testing.assert_allclose(y[rows.numpy()], oracle.spmv_csr(ip, cols, vals, x),
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seed", [0, 1])
def test_xcs_hybrid(seed):
    rng = np.random.default_rng(seed)
    n_cols = 300000
    lengths = rng.zipf(1.6, 5000).clip(max=40000)
    lengths[rng.integers(0, 5000, 300)] = 0
    vals, cols, ip, x = _case(lengths, n_cols, seed)
    long_mask = torch.as_tensor(lengths >= panel_row_min(n_cols, 4))
    assert 0 < int(long_mask.sum()) < 5000
    h = XcsHybridLayout(vals, cols, ip, n_cols, long_mask)
    assert h.short.nnz + h.long.nnz == vals.numel()
    _check_panels(h.long, *_long_part(vals, cols, ip, long_mask))
    y = _emulate(h.short, x.numpy())
    assert np.all(np.isnan(y[long_mask.numpy()]))  # long rows: left to the panel rows
    assert np.all(h.short.row_count.numpy()[long_mask.numpy()] == _spmv_layouts.ROW_SKIP)
    y = _emulate_panels(h.long, x.numpy(), y)
    np.testing.assert_allclose(y, oracle.spmv_csr(ip, cols, vals, x), rtol=1e-12, atol=1e-12)
    # through a row map (COO row runs): layout row r is output row map[r]
    rmap = np.arange(5000) * 2
    y2 = _emulate(h.short, x.numpy(), y=np.full(10000, np.nan), row_map=rmap)
    y2 = _emulate_panels(h.long, x.numpy(), y2, row_map=rmap)
    np.testing.assert_array_equal(y2[rmap], y)


def _long_part(vals, cols, ip, long_mask):
    """The compacted CSR of the long rows (the panel part's input)."""
    lengths = ip[1:] - ip[:-1]
    entry_long = torch.repeat_interleave(long_mask, lengths)
    lp = torch.zeros(int(long_mask.sum()) + 1, dtype=torch.int64)
    lp[1:] = torch.cumsum(lengths[long_mask], 0)
    return vals[entry_long], cols[entry_long], lp


@pytest.mark.parametrize("n,off", [(10494, 5), (777, 3), (4096, 17), (129, 2)])
def test_band_launch_order(n, off):
    # a permutation; launch slot i lands on the XCD its block was given (i mod 8) except in the
    # tail where the XCDs' lists have unequal lengths; a block and its +-off neighbours in
    # the same chain segment share an XCD
    order = _spmv_layouts.band_launch_order(n, off, "cpu").numpy()
    assert sorted(order.tolist()) == list(range(n))
    c, k = order % off, order // off
    xcd = (c + off * (k // _spmv_layouts.BAND_SEGMENT)) % 8
    assert np.mean(xcd == np.arange(n) % 8) > 0.97
    b = np.arange(n - off)
    same = (b // off // _spmv_layouts.BAND_SEGMENT) == ((b + off) // off // _spmv_layouts.BAND_SEGMENT)
    xb = ((b % off) + off * (b // off // _spmv_layouts.BAND_SEGMENT)) % 8
    xb2 = (((b + off) % off) + off * ((b + off) // off // _spmv_layouts.BAND_SEGMENT)) % 8
    assert np.all(xb[same] == xb2[same])


def test_band_offset_detection():
    d, i, p, _, shape = synthetic.csr_poisson2d(2048)
    assert _spmv_layouts.band_block_offset(i, p, 10494) == 5  # far diagonals 2048 rows away
    _, cols, ip, _ = _case([12] * 20000, 4 << 20, 2)
    assert _spmv_layouts.band_block_offset(cols, ip, 200) is None  # uniform random columns


def test_layout_choice():
    # uniform random columns over a large x -> XCS; a banded matrix -> row blocks
    vals, cols, ip, _ = _case([12] * 20000, 4 << 20, 2)
    assert prefers_xcs(cols, ip, 4 << 20, 4)
    d, i, p, _, shape = synthetic.csr_poisson2d(1024)
    assert not prefers_xcs(i, p, shape[1], 8)
    assert not prefers_xcs(cols, ip, 1 << 20, 4)  # x of 4 MiB fits one L2


def test_sorted_item_choice(monkeypatch):
    # sorted-gather items by default for rows that put several entries into each panel
    # (cfg4's kind), row-order items for rows of about one entry per panel (cfg3's short rows)
    monkeypatch.setattr(_spmv_layouts, "SORTED_ITEMS", True)
    monkeypatch.setattr(_spmv_layouts, "SORTED_MIN_RUN", 3.0)
    est = _spmv_layouts._entries_per_panel_run
    assert est(torch.full((1000,), 21), 4) > 5.0
    assert est(torch.ones(1000, dtype=torch.int64), 16) == 1.0
    assert est(torch.zeros(10, dtype=torch.int64), 16) == 0.0
    vals, cols, ip, x = _case([21] * 3000, 60000, 4)
    assert XcsLayout(vals, cols, ip, 60000).item_format == 1
    vals, cols, ip, x = _case([2] * 3000, 60000, 4)
    assert XcsLayout(vals, cols, ip, 60000, panels_per_xcd=2).item_format == 0
    # mostly one entry per row and panel reached (cfg3's short rows): row-order items
    assert est(torch.tensor([1] * 100 + [2] * 20 + [50] * 2), 16) < 3.0


def test_sample_indices_stay_in_bounds():
    # float32 spacing is 2 above 2^24: an evenly spaced sample must still end at n - 1
    for n in (1, 5, 1 << 20, (1 << 24) + 2, 25165824, 100663296, (1 << 31) - 1):
        idx = sample_indices(n, 1 << 20, "cpu")
        assert idx.numel() == min(n, 1 << 20)
        assert int(idx.min()) == 0 and int(idx.max()) == n - 1
        assert bool((idx[1:] >= idx[:-1]).all())


def test_panel_partials_beyond_store_range(monkeypatch):
    # the panel kernel stores its partial sums through a buffer of < 2^31 bytes; a layout
    # needing more is refused at build time (build_layout then takes row blocks)
    lengths = [9000, 20000, 5000]
    vals, cols, ip, x = _case(lengths, 200000, 6)
    rows = torch.arange(len(lengths))
    lay = PanelLayout(vals, cols, ip, 200000, rows)
    monkeypatch.setattr(_spmv_layouts, "_INDEX_LIMIT_INT32", 8 * lay.n_partials - 1)
    with pytest.raises(ValueError):
        PanelLayout(vals, cols, ip, 200000, rows)


def test_panel_chunk_plan_known_answers():
    # chunk of 8 entries, at most 2 runs: the third run opens a new chunk (the rest of the
    # first is padding); a run longer than a chunk continues across chunks and counts in each;
    # every panel ends on a chunk boundary; an empty panel takes no room
    plan = _spmv_layouts.plan_panel_chunks
    pos, end = plan(torch.tensor([0, 3]), torch.tensor([3, 3, 3]), 8, 2)
    assert pos.tolist() == [0, 3, 8] and end.tolist() == [16]
    pos, end = plan(torch.tensor([0, 1, 1, 3]), torch.tensor([20, 5, 2]), 8, 2)
    assert pos.tolist() == [0, 24, 29] and end.tolist() == [24, 24, 32]
    # run 0 ends the chunk exactly, so run 1 opens a fresh one
    pos, end = plan(torch.tensor([0, 2]), torch.tensor([8, 1]), 8, 1)
    assert pos.tolist() == [0, 8] and end.tolist() == [16]


@pytest.mark.parametrize("seed", range(4))
def test_panel_chunk_plan_properties(seed):
    # random runs: runs in order, contiguous, never overlapping; each chunk within the entry
    # and run caps; a chunk is cut short only when it holds the run cap (greedy)
    rng = np.random.default_rng(seed)
    chunk, cap = 16, 3
    n_panels = 5
    counts = rng.integers(0, 30, n_panels)
    counts[2] = 0
    lens = rng.integers(1, 40, int(counts.sum()))
    short = rng.random(lens.size) < 0.5
    lens[short] = rng.integers(1, 3, int(short.sum()))
    pr = np.r_[0, np.cumsum(counts)]
    pos, end = _spmv_layouts.plan_panel_chunks(torch.as_tensor(pr), torch.as_tensor(lens),
                                                chunk, cap)
    pos, end = pos.numpy(), end.numpy()
    start = 0
    for p in range(n_panels):
        assert start % chunk == 0 and end[p] % chunk == 0
        owner = np.full(end[p] - start, -1)
        for r in range(pr[p], pr[p + 1]):
            a = pos[r] - start
            assert np.all(owner[a:a + lens[r]] == -1)
            owner[a:a + lens[r]] = r
        if pr[p + 1] > pr[p]:
            assert pos[pr[p]] == start
            assert np.all(np.diff(pos[pr[p]:pr[p + 1]]) >= lens[pr[p]:pr[p + 1] - 1])
        for c in range(0, owner.size, chunk):
            seg = owner[c:c + chunk]
            runs = np.unique(seg[seg >= 0])
            assert 1 <= runs.size <= cap
            if (seg < 0).any() and c + chunk < owner.size:
                assert runs.size == cap  # closed early only at the run cap
        start = end[p]


@pytest.mark.parametrize("seed", range(6))
def test_panel_chunk_plan_prefix_matches_host(seed):
    # the prefix-sum plan (the device path's fast route, device-agnostic torch) either equals
    # the host greedy planner or declines, and it declines exactly when the host plan closes a
    # chunk early at the run cap
    rng = np.random.default_rng(100 + seed)
    chunk = int(rng.choice([8, 16, 512]))
    for trial in range(40):
        n_panels = int(rng.integers(1, 9))
        counts = rng.integers(0, 60, n_panels)
        lens = rng.integers(1, 3 * chunk, int(counts.sum()))
        short = rng.random(lens.size) < rng.random()
        lens[short] = rng.integers(1, 4, int(short.sum()))
        cap = int(rng.integers(2, 70))
        pr = torch.as_tensor(np.r_[0, np.cumsum(counts)])
        rl = torch.as_tensor(lens)
        host_pos, host_end = _spmv_layouts.plan_panel_chunks(pr, rl, chunk, cap)
        got = _spmv_layouts.plan_panel_chunks_prefix(pr, rl, chunk, cap)
        packed = np.r_[0, np.cumsum(lens)][:-1] if lens.size else np.zeros(0, dtype=np.int64)
        # host plan with no early close: every panel's runs back to back
        starts = np.repeat(np.r_[0, host_end.numpy()[:-1]], counts)
        firsts = np.repeat(np.r_[0, np.cumsum(lens)][pr.numpy()[:-1]], counts)
        no_early = np.array_equal(host_pos.numpy(), starts + packed - firsts)
        if got is None:
            assert not no_early
        else:
            assert no_early
            assert torch.equal(got[0], host_pos) and torch.equal(got[1], host_end)


def test_panel_layout_short_runs():
    # rows with one or two entries in each of many panels: chunks close at the run cap, and
    # the sums still match the oracle
    rng = np.random.default_rng(5)
    lengths = rng.integers(2, 120, 600)
    vals, cols, ip, x = _case(lengths, 200000, 8)
    rows = torch.arange(len(lengths))
    lay = PanelLayout(vals, cols, ip, 200000, rows)
    _check_panels(lay, vals, cols, ip)
    y = _emulate_panels(lay, x.numpy(), np.full(len(lengths), np.nan))
    np.testing.assert_allclose(y, oracle.spmv_csr(ip, cols, vals, x), rtol=1e-12, atol=1e-12)


def _without_panel_bases(vals, cols, ip, cb):
    """The matrix without its entries in each panel's first column (multiples of 2^cb)."""
    keep = (cols.to(torch.int64) & ((1 << cb) - 1)) != 0
    row = torch.repeat_interleave(torch.arange(ip.numel() - 1), ip[1:] - ip[:-1])[keep]
    ip2 = torch.zeros_like(ip)
    ip2[1:] = torch.cumsum(torch.bincount(row, minlength=ip.numel() - 1), 0)
    return vals[keep], cols[keep], ip2


@pytest.mark.parametrize("bad", [float("inf"), float("nan")])
def test_panel_padding_adds_zero_for_nonfinite_x(bad):
    # padding entries point at their panel's first column with value 0; with x infinite or NaN
    # there (and no entry of the matrix in that column) they must still add exactly 0
    rng = np.random.default_rng(6)
    lengths = rng.integers(2, 120, 600)
    vals, cols, ip, x = _case(lengths, 200000, 10)
    cb = _spmv_layouts._panel_col_bits(200000, 4)
    vals, cols, ip = _without_panel_bases(vals, cols, ip, cb)
    lay = PanelLayout(vals, cols, ip, 200000, torch.arange(len(lengths)))
    _check_panels(lay, vals, cols, ip)
    assert int(lay.chunk_info[:, 1].min()) < _abi.caps()["panel_chunk"]  # there is padding
    x = x.clone()
    x[::1 << cb] = bad
    y = _emulate_panels(lay, x.numpy(), np.full(len(lengths), np.nan))
    ref = oracle.spmv_csr(ip, cols, vals, x)
    assert np.all(np.isfinite(ref))
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)


def test_hybrid_falls_back_to_xcs(monkeypatch):
    # a panel part that does not fit its packing (PanelLayout raises ValueError, as for too
    # many partial sums) leaves the matrix to the XCS layout alone, not to row blocks
    rng = np.random.default_rng(9)
    lengths = np.concatenate([rng.zipf(2.0, 3000).clip(max=50), [30000] * 4])
    vals, cols, ip, x = _case(lengths, 300000, 9)
    monkeypatch.setattr(_spmv_layouts, "FORCE", "xcs-hybrid")
    assert _spmv_layouts.build_layout(vals, cols, ip, 300000).kind == "xcs-hybrid"

    def refuse(*args, **kwargs):
        raise ValueError("does not fit")

    monkeypatch.setattr(_spmv_layouts.PanelLayout, "__init__", refuse)
    lay = _spmv_layouts.build_layout(vals, cols, ip, 300000)
    assert lay.kind == "xcs"
    np.testing.assert_allclose(_emulate(lay, x.numpy()), oracle.spmv_csr(ip, cols, vals, x),
                               rtol=1e-12, atol=1e-12)
