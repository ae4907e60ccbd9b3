"""SpMV through the layouts for columns spread over a large x on the GPU, forced for every matrix
here: the XCD column-split layout (spmv_xcs_kernel) alone and as the hybrid with the long rows
in the panel layout, and the staged-x layout (spmv_panel_kernel staging x for the short rows,
stage_combine_kernel) - against the fp64 CPU oracle; the automatic choice is checked to pick
the staged-x layout for random-column matrices and to keep row blocks for banded ones.

Bars as for the row-block kernel: relative L2 error <= 1e-5 / 1e-12, the reference scripts'
allclose ratio, and for the default float32 path at most 1 ulp from float32(fp64 oracle).
"""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _spmv_layouts, synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(params=[("xcs-l2", 0), ("xcs-l2", 1), ("xcs-hybrid", 0), ("xcs-hybrid", 1),
                        ("xstage", 0), ("xstage", 8192)],
                ids=["xcs-rows", "xcs-sorted", "hybrid-rows", "hybrid-sorted", "xstage",
                     "xstage-8192"])
def force_xcs(request, monkeypatch):
    # the hybrid with rows of >= 32 entries in the panel part, so that these small matrices
    # have long rows in every case that checks the layout kind; the XCS items in row order
    # (format 0) or with sorted gathers (format 1) wherever the panels allow it
    mode, fmt = request.param
    monkeypatch.setattr(_spmv_layouts, "FORCE", mode)
    monkeypatch.setattr(_spmv_layouts, "SORTED_ITEMS", fmt == 1)
    monkeypatch.setattr(_spmv_layouts, "SORTED_MIN_RUN", 0.0)
    if mode in ("xcs-hybrid", "xstage"):
        monkeypatch.setattr(_spmv_layouts, "FORCE_PANEL_ROW_MIN", 32)
    if mode == "xstage":  # the staged-x windows: the size the layout picks, or the largest
        monkeypatch.setattr(_spmv_layouts, "FORCE_STAGE_WINDOW", fmt or None)
    return mode


def _kind(mode):
    return {"xcs-l2": "xcs"}.get(mode, mode)


def _ulp(a, b):
    def ordered(v):
        i = np.ascontiguousarray(v, dtype=np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(ordered(a) - ordered(b))


def _check(y, ref64, exact_fp32=False):
    name = "float64" if y.dtype == torch.float64 else "float32"
    err = oracle.rel_l2(y, ref64)
    assert err <= oracle.REL_L2_BOUND[name], f"rel_l2 {err:.3e}"
    atol, rtol = oracle.REF_SCRIPT_TOL[name]
    assert oracle.allclose_ratio(y, ref64, atol, rtol) <= 1.0
    if exact_fp32:
        u = _ulp(y.cpu().numpy(), ref64.astype(np.float32))
        assert u.size == 0 or u.max() <= 1, u.max()


def _csr_from_lengths(lengths, n_cols, seed, dtype):
    keys = synthetic._distinct_sorted_columns(torch.as_tensor(lengths, dtype=torch.int64),
                                              n_cols, seed, 1)
    ip, cols = synthetic._csr_from_keys(keys, len(lengths), n_cols)
    vals = synthetic.uniform_values(seed, 2, cols.numel(), dtype, "cpu")
    x = synthetic.uniform_values(seed, 3, n_cols, dtype, "cpu")
    return vals, cols, ip, x, (len(lengths), n_cols)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("use_opt", [False, True])
def test_powerlaw(dev, force_xcs, dtype, use_opt):
    data, idx, ptr, x, shape = synthetic.csr_powerlaw(1 << 17, cap=60000, dtype=dtype)
    print(f"xcs powerlaw {force_xcs} {dtype} use_opt={use_opt}", flush=True)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(dev), ptr.to(dev), shape)
    assert p._kernel(use_opt).kind == _kind(force_xcs)
    y = fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p, use_opt=use_opt)
    _check(y, oracle.spmv_csr(ptr, idx, data, x),
           exact_fp32=(dtype == torch.float32 and not use_opt))
    assert torch.equal(y, fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p, use_opt=use_opt))


@pytest.mark.parametrize("lengths", [
    [3, 0, 40000, 1, 1, 2] + [0] * 9000 + [17000, 5, 0, 6144, 7],
    [1] * 20000 + [0] * 5000 + [2] * 7000,
    [0] * 100 + [200000] + [0] * 100,
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_edges(dev, force_xcs, lengths, dtype):
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, 1 << 20, 13, dtype)
    for use_opt in (False, True):
        y = fs.flagsparse_spmv_csr(data.to(dev), idx.to(torch.int32).to(dev), ptr.to(dev),
                                   x.to(dev), shape, use_opt=use_opt)
        _check(y, oracle.spmv_csr(ptr, idx, data, x),
               exact_fp32=(dtype == torch.float32 and not use_opt))


HYBRID_EDGES = [
    ([40] * 3000, 1 << 20),                              # every row long: empty XCS part
    ([40, 0, 3, 100, 1] * 600, 5000),                    # x of one small panel (13 bits)
    ([33] * 1000 + [31] * 1000 + [32] * 1000, 70001),    # rows at the threshold; ragged panels
    ([5000] + [0] * 3000 + [2] * 3000 + [7000], 300000),  # two long rows, short rows between
]


@pytest.mark.parametrize("lengths,n_cols", HYBRID_EDGES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("mode", ["xcs-hybrid", "xstage"])
def test_hybrid_edges(dev, monkeypatch, lengths, n_cols, dtype, mode):
    monkeypatch.setattr(_spmv_layouts, "FORCE", mode)
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANEL_ROW_MIN", 32)
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, n_cols, 21, dtype)
    print(f"hybrid edges {mode} rows={len(lengths)} n_cols={n_cols} {dtype}", flush=True)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(torch.int32).to(dev), ptr.to(dev), shape)
    assert p._kernel(False).kind == mode
    ref = oracle.spmv_csr(ptr, idx, data, x)
    for use_opt in (False, True):
        y = fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p, use_opt=use_opt)
        _check(y, ref, exact_fp32=(dtype == torch.float32 and not use_opt))
    # a second call on the same layout reuses its partial buffers: same result, bit for bit
    assert torch.equal(y, fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p, use_opt=True))


def test_hybrid_marks_every_panel_array(dev, monkeypatch):
    # A hybrid built on one stream and called from another: the caller's stream must be
    # ordered after the build stream, and every array the panel kernel and its combine read
    # must be marked as used on it, so that the allocator does not hand their memory out while
    # the panel kernel may still read it.
    monkeypatch.setattr(_spmv_layouts, "FORCE", "xcs-hybrid")
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANEL_ROW_MIN", 32)
    lengths, n_cols = HYBRID_EDGES[3]
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, n_cols, 23, torch.float32)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(torch.int32).to(dev), ptr.to(dev), shape)
    layout = p._kernel(False)
    assert layout.kind == "xcs-hybrid"
    seen = []
    real = _spmv_layouts.StreamOrder.stream

    def spy(self, device, tensors=()):
        seen.append((self, tuple(tensors)))
        return real(self, device, tensors)

    monkeypatch.setattr(_spmv_layouts.StreamOrder, "stream", spy)
    side = torch.cuda.Stream(device=dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        y = fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p)
    torch.cuda.synchronize()
    panel = layout.long
    wanted = (panel.partials, panel.vals, panel.pcol, panel.jobs, panel.job_panel,
              panel.chunk_info, panel.rows, panel.row_ptr, panel.slots)
    got = [ts for order, ts in seen if order is panel._order]
    assert got, "the panel part's stream order was not consulted"
    for t in wanted:
        assert any(any(u is t for u in ts) for ts in got), "a panel array was not marked"
    _check(y, oracle.spmv_csr(ptr, idx, data, x), exact_fp32=True)


def test_xstage_marks_every_array(dev, monkeypatch):
    # As above for the staged-x layout: one stream order for both launches, and every array
    # they read or write (the staged part's and the panel part's) marked on the caller's stream.
    monkeypatch.setattr(_spmv_layouts, "FORCE", "xstage")
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANEL_ROW_MIN", 32)
    lengths, n_cols = HYBRID_EDGES[3]
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, n_cols, 23, torch.float32)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(torch.int32).to(dev), ptr.to(dev), shape)
    layout = p._kernel(False)
    assert layout.kind == "xstage" and layout.long is not None
    seen = []
    real = _spmv_layouts.StreamOrder.stream

    def spy(self, device, tensors=()):
        seen.append((self, tuple(tensors)))
        return real(self, device, tensors)

    monkeypatch.setattr(_spmv_layouts.StreamOrder, "stream", spy)
    side = torch.cuda.Stream(device=dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        y = fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p)
    torch.cuda.synchronize()
    lg = layout.long
    wanted = (layout.scol, layout.stage_info, layout.seg_delta, layout.xs, layout.vals,
              layout.dest, layout.row_end, layout.heads, layout.windows, layout.jobs,
              layout.job_panel, layout.stage_jobs, lg.partials, lg.vals, lg.pcol, lg.chunk_info, lg.rows,
              lg.row_ptr, lg.slots)
    got = [ts for order, ts in seen if order is layout._order]
    assert got, "the layout's stream order was not consulted"
    for t in wanted:
        assert any(any(u is t for u in ts) for ts in got), "an array was not marked"
    _check(y, oracle.spmv_csr(ptr, idx, data, x), exact_fp32=True)


def test_unsorted_duplicates_and_truncation(dev, force_xcs):
    data, idx, ptr = synthetic.build_random_csr(60000, 3000000, 400000, torch.float32,
                                                torch.int64, "cpu", seed=4)
    x = synthetic.uniform_values(4, 9, 3000000, torch.float32, "cpu")
    d, i, p, xd = data.to(dev), idx.to(dev), ptr.to(dev), x.to(dev)
    _check(fs.flagsparse_spmv_csr(d, i, p, xd, (60000, 3000000)),
           oracle.spmv_csr(ptr, idx, data, x), exact_fp32=True)
    row_len = (ptr[1:] - ptr[:-1]).numpy()
    prep = fs.prepare_spmv_csr(d, i, p, (60000, 3000000), block_nnz=4, max_segments=2)
    for use_opt in (False, True):
        caps = oracle.spmv_row_caps(row_len, use_opt, False, prep.block_nnz, prep.max_segments, 2)
        y = fs.flagsparse_spmv_csr(x=xd, prepared=prep, use_opt=use_opt)
        _check(y, oracle.spmv_csr(ptr, idx, data, x, row_cap=caps))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_coo_runs(dev, force_xcs, dtype):
    data, row, col, x, shape = synthetic.coo_uniform(1 << 17, 40 << 16, dtype=dtype)
    ref = oracle.spmv_coo(row, col, data, x, shape[0])
    p = fs.prepare_spmv_coo(data.to(dev), row.to(dev), col.to(dev), shape)
    assert p._run_layout().kind == _kind(force_xcs)
    _check(fs.flagsparse_spmv_coo(x=x.to(dev), prepared=p), ref)
    # rows without entries (run -> row map path)
    keep = (row % 3) != 0
    d2, r2, c2 = data[keep], row[keep], col[keep]
    p2 = fs.prepare_spmv_coo(d2.to(dev), r2.to(dev), c2.to(dev), shape)
    _check(fs.flagsparse_spmv_coo(x=x.to(dev), prepared=p2),
           oracle.spmv_coo(r2, c2, d2, x, shape[0]))


@pytest.mark.parametrize("count_max", [3, 8])
def test_rows_over_the_count_byte(dev, monkeypatch, count_max):
    # rows with more sums than the combine's count byte holds (ROW_COUNT_MAX, lowered here)
    # are windows of their own, summed by a whole workgroup; the others keep their windows
    monkeypatch.setattr(_spmv_layouts, "FORCE", "xcs-l2")
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANELS_PER_XCD", 2)  # 16 panels: rows of 9+ sums
    monkeypatch.setattr(_spmv_layouts, "ROW_COUNT_MAX", count_max)
    lengths = [3, 0, 400, 1, 1, 2] + [0] * 90 + [170, 5, 0, 61, 7] + [1] * 3000 + [2] * 300
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, 300000, 24, torch.float32)
    print(f"count byte {count_max}", flush=True)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(torch.int32).to(dev), ptr.to(dev), shape)
    lay = p._kernel(False)
    assert lay.kind == "xcs" and int((lay.windows.view(-1, 8)[:, 1] < 0).sum()) > 0
    ref = oracle.spmv_csr(ptr, idx, data, x)
    for use_opt in (False, True):
        _check(fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p, use_opt=use_opt), ref,
               exact_fp32=not use_opt)


def test_automatic_choice(dev):
    data, idx, ptr, x, shape = synthetic.csr_powerlaw(1 << 21, cap=5000)  # x: 8 MiB
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(dev), ptr.to(dev), shape)
    assert p._kernel(False).kind == "xstage"
    ref = oracle.spmv_csr(ptr, idx, data, x)
    _check(fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p), ref, exact_fp32=True)
    # a call without a prepared object takes the row-block layout (fastest to build)
    _check(fs.flagsparse_spmv_csr(data.to(dev), idx.to(dev), ptr.to(dev), x.to(dev), shape), ref,
           exact_fp32=True)
    rows = torch.repeat_interleave(torch.arange(shape[0]), ptr[1:] - ptr[:-1])
    _check(fs.flagsparse_spmv_coo(data.to(dev), rows.to(dev), idx.to(dev), x.to(dev), shape),
           oracle.spmv_coo(rows, idx, data, x, shape[0]))
    po = fs.prepare_spmv_coo(data.to(dev), rows.to(dev), idx.to(dev), shape)
    assert po._run_layout().kind == "xstage"
    d, i, pp, xx, sh = synthetic.csr_poisson2d(1024)
    p = fs.prepare_spmv_csr(d.to(dev), i.to(dev), pp.to(dev), sh)
    assert p._kernel(False).kind == "rowblock"
    # a heavier tail (cap 200000 as cfg3): the long rows in the staged-x layout's panel part
    data, idx, ptr, x, shape = synthetic.csr_powerlaw(1 << 21, cap=200000)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(dev), ptr.to(dev), shape)
    assert p._kernel(False).kind == "xstage" and p._kernel(False).long is not None
    _check(fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p), oracle.spmv_csr(ptr, idx, data, x),
           exact_fp32=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_combine_unaligned_windows(dev, monkeypatch, dtype):
    # runs and windows starting anywhere (not on a line); small windows, so that there are
    # hundreds, some of one long row
    monkeypatch.setattr(_spmv_layouts, "FORCE", "xcs-l2")
    monkeypatch.setattr(_spmv_layouts, "RUN_ALIGN", 1)
    monkeypatch.setattr(_spmv_layouts, "WINDOW_ALIGN", 1)
    monkeypatch.setattr(_spmv_layouts, "WINDOW_SLOTS", 128)
    monkeypatch.setattr(_spmv_layouts, "WINDOW_ROWS", 64)
    rng = np.random.default_rng(11)
    # two rows long enough to have more sums than a window holds (one-row windows) with
    # either item size
    lengths = np.concatenate([rng.zipf(1.8, 30000).clip(max=20000), [900000, 3, 900000]])
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, 1 << 21, 23, dtype)
    print(f"unaligned combine windows {dtype}", flush=True)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(torch.int32).to(dev), ptr.to(dev), shape)
    lay = p._kernel(False)
    assert lay.kind == "xcs"
    w = lay.windows.cpu().numpy().reshape(-1, 8)
    assert (w[:, 2] % 4 != 0).any() and (w[:, 2] % 4 == 0).any() and (w[:, 1] < 0).any()
    ref = oracle.spmv_csr(ptr, idx, data, x)
    for use_opt in (False, True):
        y = fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p, use_opt=use_opt)
        _check(y, ref, exact_fp32=(dtype == torch.float32 and not use_opt))


@pytest.mark.parametrize("layout", ["rowblock", "xcs-l2", "xcs-hybrid", "xstage"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_unaligned_x_and_out(dev, monkeypatch, layout, dtype):
    # x and out as views one element into their buffers (not 16-byte aligned): the panel
    # kernel then copies its x panels element by element, and the result goes through a
    # temporary into out, which is what the call returns
    monkeypatch.setattr(_spmv_layouts, "FORCE", layout)
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANEL_ROW_MIN", 32)
    lengths = [40, 0, 3, 100, 1] * 600
    n_cols = 70001  # the last panel narrower than the others
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, n_cols, 29, dtype)
    print(f"unaligned x/out {layout} {dtype}", flush=True)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(torch.int32).to(dev), ptr.to(dev), shape)
    assert p._kernel(False).kind == {"xcs-l2": "xcs"}.get(layout, layout)
    x_buf = torch.zeros(n_cols + 1, dtype=dtype, device=dev)
    x_buf[1:] = x.to(dev)
    x_view = x_buf[1:]
    assert x_view.data_ptr() % 16 != 0
    out_buf = torch.full((shape[0] + 1,), float("nan"), dtype=dtype, device=dev)
    out = out_buf[1:]
    ref = oracle.spmv_csr(ptr, idx, data, x)
    for use_opt in (False, True):
        y = fs.flagsparse_spmv_csr(x=x_view, prepared=p, out=out, use_opt=use_opt)
        assert y is out
        _check(y, ref, exact_fp32=(dtype == torch.float32 and not use_opt))
        assert torch.isnan(out_buf[0])
        # the same as with aligned x and no out, bit for bit
        assert torch.equal(y, fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p, use_opt=use_opt))


@pytest.mark.parametrize("bad", [float("inf"), float("nan")])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("mode", ["xcs-hybrid", "xstage"])
def test_panel_padding_with_nonfinite_x(dev, monkeypatch, bad, dtype, mode):
    # x infinite or NaN in every panel's first column: the panel layout's padding entries point
    # there with value 0 and must add exactly 0 (0 * inf would be NaN).  Without entries in
    # those columns every row is finite; with them, the rows holding one are inf / NaN exactly
    # as in the oracle (inf or NaN of a row does not depend on the summation order).  In the
    # staged-x layout the staged part's padding (up to 7 entries per panel) stages that x too,
    # and must never be read.
    monkeypatch.setattr(_spmv_layouts, "FORCE", mode)
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANEL_ROW_MIN", 32)
    rng = np.random.default_rng(17)
    lengths = np.concatenate([rng.integers(0, 30, 4000), rng.integers(32, 3000, 400)])
    rng.shuffle(lengths)
    n_cols = 300001
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, n_cols, 31, dtype)
    cb = _spmv_layouts._panel_col_bits(n_cols, data.element_size())
    x[::1 << cb] = bad
    print(f"non-finite x at panel bases {bad} {dtype}", flush=True)
    keep = (idx & ((1 << cb) - 1)) != 0
    row = torch.repeat_interleave(torch.arange(len(lengths)), ptr[1:] - ptr[:-1])
    for drop in (True, False):
        if drop:
            d, i = data[keep], idx[keep]
            p = torch.zeros_like(ptr)
            p[1:] = torch.cumsum(torch.bincount(row[keep], minlength=len(lengths)), 0)
        else:
            d, i, p = data, idx, ptr
        prep = fs.prepare_spmv_csr(d.to(dev), i.to(torch.int32).to(dev), p.to(dev), shape)
        lay = prep._kernel(False)
        assert lay.kind == mode
        assert int(lay.long.chunk_info[:, 1].min()) < 512  # padding present
        ref = oracle.spmv_csr(p, i, d, x)
        for use_opt in (False, True):
            y = fs.flagsparse_spmv_csr(x=x.to(dev), prepared=prep, use_opt=use_opt).cpu().numpy()
            fin = np.isfinite(ref)
            assert drop == bool(fin.all())
            assert np.array_equal(np.isnan(y), np.isnan(ref))
            assert np.array_equal(y[np.isinf(ref)], ref[np.isinf(ref)].astype(y.dtype))
            name = "float64" if dtype == torch.float64 else "float32"
            assert oracle.rel_l2(torch.as_tensor(y[fin]), ref[fin]) <= oracle.REL_L2_BOUND[name]


@pytest.mark.parametrize("n_rows,n_cols,lengths", [
    (1000, 7, [0] * 1000),          # no entries
    (3, 1, [1, 0, 1]),              # one column
    (1, 5, [5]),                    # one row holding every column
    (5, 3, [0, 3, 0, 0, 3]),
    (2, 100000, [0, 0]),            # wide, empty
])
@pytest.mark.parametrize("layout", ["xcs-l2", "xcs-hybrid", "xstage"])
def test_degenerate_shapes(dev, monkeypatch, n_rows, n_cols, lengths, layout):
    monkeypatch.setattr(_spmv_layouts, "FORCE", layout)
    monkeypatch.setattr(_spmv_layouts, "FORCE_PANEL_ROW_MIN", 2)
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, n_cols, 37, torch.float32)
    print(f"degenerate {layout} {shape} nnz={data.numel()}", flush=True)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(torch.int32).to(dev), ptr.to(dev), shape)
    ref = oracle.spmv_csr(ptr, idx, data, x)
    for use_opt in (False, True):
        y = fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p, use_opt=use_opt)
        assert y.shape == (n_rows,)
        np.testing.assert_allclose(y.cpu().numpy(), ref, rtol=1e-6, atol=1e-6)
