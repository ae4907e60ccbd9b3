"""CSR SpMV on the GPU against the CPU oracle (fp64 row sums).

Bars: relative L2 error <= 1e-5 (float32) / 1e-12 (float64) against the fp64 oracle
(north_star), and the reference test scripts' allclose ratio <= 1 with (1e-4, 1e-2) /
(1e-12, 1e-10) (tests/test_spmv_opt.py:204-207).  The default float32 path must equal
float32(oracle) to within one ulp (the reference returns fp32 of an fp64 sum,
spmv_csr.py:498-536; only the fp64 summation order differs).
"""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu


def _name(dtype):
    return str(dtype).replace("torch.", "")


def _check(y, ref64, dtype, exact_fp32=False):
    name = _name(dtype)
    err = oracle.rel_l2(y, ref64)
    assert err <= oracle.REL_L2_BOUND[name], f"rel_l2 {err:.3e}"
    atol, rtol = oracle.REF_SCRIPT_TOL[name]
    ratio = oracle.allclose_ratio(y, ref64, atol, rtol)
    assert ratio <= 1.0, f"allclose ratio {ratio:.3e}"
    if exact_fp32:
        ulp = _ulp_distance(y.detach().cpu().numpy(), ref64.astype(np.float32))
        assert ulp.size == 0 or ulp.max() <= 1, f"max ulp {ulp.max()}"


def _ulp_distance(a, b):
    """Distance in float32 units in the last place (sign-magnitude bits -> ordered ints)."""
    def ordered(v):
        i = np.ascontiguousarray(v, dtype=np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(ordered(a) - ordered(b))


def _csr_from_lengths(lengths, n_cols, seed, dtype):
    keys = synthetic._distinct_sorted_columns(torch.as_tensor(lengths, dtype=torch.int64), n_cols,
                                              seed, 1)
    ip, cols = synthetic._csr_from_keys(keys, len(lengths), n_cols)
    vals = synthetic.uniform_values(seed, 2, cols.numel(), dtype, "cpu")
    x = synthetic.uniform_values(seed, 3, n_cols, dtype, "cpu")
    return vals, cols, ip, x, (len(lengths), n_cols)


def _run(dev, data, idx, ptr, x, shape, use_opt, index_dtype=torch.int32, **kw):
    y = fs.flagsparse_spmv_csr(data.to(dev), idx.to(index_dtype).to(dev), ptr.to(dev), x.to(dev),
                               shape, use_opt=use_opt, **kw)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("use_opt", [False, True])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_cfg1_uniform_rows(dev, use_opt, index_dtype):
    data, idx, ptr, x, shape = synthetic.csr_uniform_rows()
    print(f"cfg1 use_opt={use_opt} idx={index_dtype}", flush=True)
    y = _run(dev, data, idx, ptr, x, shape, use_opt, index_dtype)
    _check(y, oracle.spmv_csr(ptr, idx, data, x), torch.float32, exact_fp32=not use_opt)


@pytest.mark.parametrize("use_opt", [False, True])
def test_poisson_fp64(dev, use_opt):
    data, idx, ptr, x, shape = synthetic.csr_poisson2d(256)
    y = _run(dev, data, idx, ptr, x, shape, use_opt)
    _check(y, oracle.spmv_csr(ptr, idx, data, x), torch.float64)


@pytest.mark.parametrize("grid", [1024, 1536])
def test_poisson_band_launch_order(dev, monkeypatch, grid):
    # a stencil's far diagonals (+-grid rows, 2.5 and 3.75 blocks of ~409 rows here) are
    # detected and the descriptors reordered; the order changes nothing in the result, bit for
    # bit
    from flagsparse_amd import _spmv_layouts

    data, idx, ptr, x, shape = synthetic.csr_poisson2d(grid)
    d, i, p, xd = data.to(dev), idx.to(dev), ptr.to(dev), x.to(dev)
    prep = fs.prepare_spmv_csr(d, i, p, shape)
    lay = prep._kernel(False)
    assert lay.kind == "rowblock" and lay.band_offset is not None
    y = fs.flagsparse_spmv_csr(x=xd, prepared=prep)
    _check(y, oracle.spmv_csr(ptr, idx, data, x), torch.float64)
    monkeypatch.setattr(_spmv_layouts, "BAND_ORDER", False)
    plain = fs.prepare_spmv_csr(d, i, p, shape)
    assert plain._kernel(False).band_offset is None
    assert torch.equal(y, fs.flagsparse_spmv_csr(x=xd, prepared=plain))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("use_opt", [False, True])
def test_powerlaw_split_rows(dev, dtype, use_opt):
    # 2^17 rows, cap 60000: rows beyond 4093 entries are split across workgroups.
    data, idx, ptr, x, shape = synthetic.csr_powerlaw(1 << 17, cap=60000, dtype=dtype)
    lengths = (ptr[1:] - ptr[:-1]).numpy()
    assert lengths.max() > 8 * 4093
    y = _run(dev, data, idx, ptr, x, shape, use_opt, torch.int64)
    _check(y, oracle.spmv_csr(ptr, idx, data, x), dtype,
           exact_fp32=(dtype == torch.float32 and not use_opt))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_random_unsorted_duplicates_empty_rows(dev, dtype):
    # reference generator shape: unsorted columns, repeated (row, col), many empty rows
    data, idx, ptr = synthetic.build_random_csr(50000, 3000, 20000, dtype, torch.int32, "cpu", seed=3)
    x = synthetic.build_random_dense(3000, dtype, "cpu", seed=3)
    lengths = (ptr[1:] - ptr[:-1])
    assert int((lengths == 0).sum()) > 1000
    for use_opt in (False, True):
        y = _run(dev, data, idx, ptr, x, (50000, 3000), use_opt)
        _check(y, oracle.spmv_csr(ptr, idx, data, x), dtype)


@pytest.mark.parametrize("lengths", [
    [2045, 2046, 1, 4093, 4094, 3, 8186, 8187, 2, 12279],       # chunk boundaries
    [1021, 1022, 1, 1020, 3, 1021, 1021, 2, 1023, 4093, 1022],    # short-row block capacity
    [1, 2, 3, 5000, 7, 1, 1, 9000, 2045, 1, 2045],              # misaligned row starts
    [0] * 100 + [200000] + [0] * 100,                           # one very long row, empty rows
    [1] * 5000 + [0] * 3000 + [2] * 2000,                       # block row cap (1024 rows)
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_block_edges(dev, lengths, dtype):
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, 1000000, 11, dtype)
    for use_opt in (False, True):
        y = _run(dev, data, idx, ptr, x, shape, use_opt)
        _check(y, oracle.spmv_csr(ptr, idx, data, x), dtype,
               exact_fp32=(dtype == torch.float32 and not use_opt))


def test_deterministic_repeat(dev):
    data, idx, ptr, x, shape = _csr_from_lengths([3] * 1000 + [150000] + [5] * 1000, 300000, 5,
                                                 torch.float32)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(torch.int32).to(dev), ptr.to(dev), shape)
    xd = x.to(dev)
    ys = [fs.flagsparse_spmv_csr(x=xd, prepared=p, use_opt=True) for _ in range(5)]
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


def test_empty_and_zero_rows(dev):
    for n_rows, n_cols in ((0, 5), (1000, 7), (3, 0)):
        ptr = torch.zeros(n_rows + 1, dtype=torch.int64, device=dev)
        data = torch.empty(0, dtype=torch.float32, device=dev)
        idx = torch.empty(0, dtype=torch.int32, device=dev)
        x = torch.randn(n_cols, device=dev)
        y = fs.flagsparse_spmv_csr(data, idx, ptr, x, (n_rows, n_cols))
        assert y.shape == (n_rows,) and torch.count_nonzero(y) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_max_segments_truncation(dev, dtype):
    lengths = [0, 5, 64, 65, 200, 300, 513, 700, 1100, 4097, 9000]
    data, idx, ptr, x, shape = _csr_from_lengths(lengths, 20000, 9, dtype)
    row_len = (ptr[1:] - ptr[:-1]).numpy()
    d, i, p, xd = data.to(dev), idx.to(torch.int32).to(dev), ptr.to(dev), x.to(dev)
    for block_nnz, max_segments in ((64, 3), (256, 1), (32, 2)):
        prep = fs.prepare_spmv_csr(d, i, p, shape, block_nnz=block_nnz, max_segments=max_segments)
        b_use, s_use = oracle.spmv_prepare_knobs(int(row_len.max()), block_nnz, max_segments)
        assert (prep.block_nnz, prep.max_segments) == (b_use, s_use)
        for use_opt in (False, True):
            caps = oracle.spmv_row_caps(row_len, use_opt, dtype == torch.float64, b_use, s_use,
                                        max_segments)
            assert np.any(caps < row_len)
            y = fs.flagsparse_spmv_csr(x=xd, prepared=prep, use_opt=use_opt)
            _check(y, oracle.spmv_csr(ptr, idx, data, x, row_cap=caps), dtype)


def test_block_nnz_doubling_attributes(dev):
    data, idx, ptr, x, shape = _csr_from_lengths([600000, 3], 2000000, 2, torch.float32)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(dev), ptr.to(dev), shape)
    assert (p.block_nnz, p.max_segments) == oracle.spmv_prepare_knobs(600000)
    assert p.max_row_nnz == 600000
    y = fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p)
    _check(y, oracle.spmv_csr(ptr, idx, data, x), torch.float32, exact_fp32=True)


def test_opt_buckets_attribute(dev):
    data, idx, ptr, x, shape = _csr_from_lengths([0, 10, 64, 65, 600, 5000], 9000, 4,
                                                 torch.float32)
    p = fs.prepare_spmv_csr(data.to(dev), idx.to(dev), ptr.to(dev), shape)
    got = p.opt_buckets
    want = oracle.spmv_opt_buckets((ptr[1:] - ptr[:-1]).numpy(), 5000, False)
    assert len(got) == len(want)
    for g, w in zip(got, want):
        assert g["rows"].dtype == torch.int32
        assert g["rows"].cpu().tolist() == w["rows"].tolist()
        assert (g["block_size"], g["max_segs"], g["batch_rows"]) == (
            w["block_size"], w["max_segs"], w["batch_rows"])


def test_out_and_return_time(dev):
    data, idx, ptr, x, shape = synthetic.csr_uniform_rows(512, 512, 8)
    d, i, p, xd = data.to(dev), idx.to(dev), ptr.to(dev), x.to(dev)
    out = torch.empty(512, device=dev)
    y, ms = fs.flagsparse_spmv_csr(d, i, p, xd, shape, out=out, return_time=True)
    assert y is out and isinstance(ms, float) and ms >= 0.0
    _check(out, oracle.spmv_csr(ptr, idx, data, x), torch.float32)
    # out aliasing x: result must still be A @ x
    xs = torch.zeros(512, device=dev)
    xs.copy_(xd)
    y = fs.flagsparse_spmv_csr(d, i, p, xs, shape, out=xs)
    _check(y, oracle.spmv_csr(ptr, idx, data, x), torch.float32)
    # non-contiguous x
    xbig = torch.zeros(1024, device=dev)
    xbig[::2] = xd
    y = fs.flagsparse_spmv_csr(d, i, p, xbig[::2], shape)
    _check(y, oracle.spmv_csr(ptr, idx, data, x), torch.float32)
    with pytest.raises(ValueError):
        fs.flagsparse_spmv_csr(d, i, p, xd, shape, out=torch.empty(511, device=dev))


def test_validation_errors(dev):
    d = torch.tensor([1.0, 2.0, 3.0], device=dev)
    i = torch.tensor([0, 1, 1], dtype=torch.int32, device=dev)
    p = torch.tensor([0, 2, 3], dtype=torch.int64, device=dev)
    x = torch.ones(2, device=dev)
    cases = [
        (lambda: fs.flagsparse_spmv_csr(d, i, p[:-1], x, (2, 2)), ValueError),
        (lambda: fs.flagsparse_spmv_csr(d, i, torch.tensor([1, 2, 3], device=dev), x, (2, 2)),
         ValueError),
        (lambda: fs.flagsparse_spmv_csr(d, i, torch.tensor([0, 2, 2], device=dev), x, (2, 2)),
         ValueError),
        (lambda: fs.flagsparse_spmv_csr(d, i, torch.tensor([0, 4, 3], device=dev), x, (2, 2)),
         ValueError),
        (lambda: fs.flagsparse_spmv_csr(d, torch.tensor([0, 3, 1], dtype=torch.int32, device=dev),
                                        p, x, (2, 2)), IndexError),
        (lambda: fs.flagsparse_spmv_csr(d, i.float(), p, x, (2, 2)), TypeError),
        (lambda: fs.flagsparse_spmv_csr(d, i, p, x.double(), (2, 2)), TypeError),
        (lambda: fs.flagsparse_spmv_csr(d, i, p, torch.ones(3, device=dev), (2, 2)), ValueError),
        (lambda: fs.flagsparse_spmv_csr(d, i, p, x.cpu(), (2, 2)), ValueError),
        (lambda: fs.flagsparse_spmv_csr(d, i, p, None, (2, 2)), TypeError),
        (lambda: fs.flagsparse_spmv_csr(x=x), ValueError),
    ]
    for fn, exc in cases:
        with pytest.raises(exc):
            fn()
    with pytest.raises(NotImplementedError):
        fs.flagsparse_spmv_csr(d.half(), i, p, x.half(), (2, 2))


def test_coo_tocsr_route(dev):
    data, row, col, x, shape = synthetic.coo_uniform(3000, 50000)
    perm = synthetic.randint(7, 1, data.numel(), 1 << 40, "cpu").argsort()
    d, r, c = data[perm], row[perm], col[perm]  # unsorted input
    ref = oracle.spmv_coo(r, c, d, x, shape[0])
    for use_opt in (True, False):
        y = fs.flagsparse_spmv_coo_tocsr(d.to(dev), r.to(dev), c.to(dev), x.to(dev), shape,
                                         use_opt=use_opt)
        _check(y, ref, torch.float32)
    p = fs.prepare_spmv_coo_tocsr(data.to(dev), row.to(dev), col.to(dev), shape, assume_sorted=True)
    y = fs.flagsparse_spmv_coo_tocsr(x=x.to(dev), prepared=p)
    _check(y, ref, torch.float32)
