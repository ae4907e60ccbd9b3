"""The benchmark configurations at their full sizes on the GPU, through the public API, against
the fp64 C oracle on the same seeded arrays (the oracle finishes these in seconds), plus
size-independent properties that hold exactly:

  cfg2  Poisson 2048^2 fp64: A * 1 = 4 - (number of neighbours) for every row, exactly;
        random x against the oracle (both paths); linearity A(2x - z) = 2Ax - Az
  cfg3  8M power-law fp32, int64 indices (the default staged-x layout, and the XCS + panel
        hybrid): oracle bars incl. <= 1 ulp from float32(fp64 oracle) on the default path; two
        calls bit-identical
  cfg3  the same in fp64 (staged-x): oracle bars, two calls bit-identical, linearity
  cfg4  COO 2M, 41.9M entries (staged-x): oracle bars for x and x = 1; A * 0 = 0; two calls
        bit-identical
  cfg5  SpMM N=64 fp32 (opt), N=16 fp32 (base and opt) and N=16 fp64 (base): oracle bars;
        column j of A B = A B[:, j] (the SpMV of the same matrix), within 1 ulp where both
        round an fp64 sum of the same products to float32 (the fp32 base path);
        the column-tiled launches (fp32 N=256, fp64 N=64 and N=256: B of 512 MiB - 2 GiB): a
        strided sample of C's rows against the oracle over the same rows, columns of C in
        different tiles against the SpMV of those columns
  sddmm cfg5's pattern, K = 64 fp32: oracle bars

Bars as everywhere: relative L2 error <= 1e-5 (fp32) / 1e-12 (fp64) and the reference scripts'
allclose ratio."""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _spmv_layouts, synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu


def _bars(y, ref64, dtype):
    name = "float64" if dtype == torch.float64 else "float32"
    err = oracle.rel_l2(y, ref64)
    assert err <= oracle.REL_L2_BOUND[name], f"rel_l2 {err:.3e}"
    atol, rtol = oracle.REF_SCRIPT_TOL[name]
    assert oracle.allclose_ratio(y, ref64, atol, rtol) <= 1.0


def _ulp(a, b):
    def ordered(v):
        i = np.ascontiguousarray(v, dtype=np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(ordered(a) - ordered(b))


def test_cfg2_full(dev):
    print("full size cfg2", flush=True)
    data, idx, ptr, x, shape = synthetic.csr_poisson2d(2048, device=dev)
    p = fs.prepare_spmv_csr(data, idx, ptr, shape)
    ones = torch.ones(shape[1], dtype=torch.float64, device=dev)
    y1 = fs.flagsparse_spmv_csr(x=ones, prepared=p).cpu().numpy()
    g = 2048
    r, c = np.divmod(np.arange(shape[0]), g)
    neighbours = (r > 0).astype(int) + (r < g - 1) + (c > 0) + (c < g - 1)
    assert np.array_equal(y1, 4.0 - neighbours)
    ptr_h, idx_h, data_h, x_h = ptr.cpu(), idx.cpu(), data.cpu(), x.cpu()
    ref = oracle.spmv_csr(ptr_h, idx_h, data_h, x_h)
    for use_opt in (False, True):
        _bars(fs.flagsparse_spmv_csr(x=x, prepared=p, use_opt=use_opt), ref, torch.float64)
    z = synthetic.uniform_values(5, 7, shape[1], torch.float64, dev)
    lhs = fs.flagsparse_spmv_csr(x=2 * x - z, prepared=p).cpu().numpy()
    rhs = 2 * ref - oracle.spmv_csr(ptr_h, idx_h, data_h, z.cpu())
    assert oracle.rel_l2(lhs, rhs) <= 1e-12


@pytest.mark.parametrize("mode", [None, "xcs"])
def test_cfg3_full(dev, monkeypatch, mode):
    print(f"full size cfg3 {mode or 'default'}", flush=True)
    monkeypatch.setattr(_spmv_layouts, "FORCE", mode)
    data, idx, ptr, x, shape = synthetic.csr_powerlaw(device=dev)
    assert idx.dtype == torch.int64 and data.numel() == 100663296
    p = fs.prepare_spmv_csr(data, idx, ptr, shape)
    assert p._kernel(False).kind == ("xstage" if mode is None else "xcs-hybrid")
    ref = oracle.spmv_csr(ptr.cpu(), idx.cpu(), data.cpu(), x.cpu())
    y = fs.flagsparse_spmv_csr(x=x, prepared=p)
    _bars(y, ref, torch.float32)
    u = _ulp(y.cpu().numpy(), ref.astype(np.float32))
    assert u.max() <= 1, u.max()
    assert torch.equal(y, fs.flagsparse_spmv_csr(x=x, prepared=p))
    _bars(fs.flagsparse_spmv_csr(x=x, prepared=p, use_opt=True), ref, torch.float32)


def test_cfg3_full_fp64(dev):
    # the staged-x layout with float64 entries (14-bit panel columns, fp64 staged values)
    print("full size cfg3 fp64", flush=True)
    data, idx, ptr, x, shape = synthetic.csr_powerlaw(dtype=torch.float64, device=dev)
    p = fs.prepare_spmv_csr(data, idx, ptr, shape)
    assert p._kernel(False).kind == "xstage"
    ref = oracle.spmv_csr(ptr.cpu(), idx.cpu(), data.cpu(), x.cpu())
    y = fs.flagsparse_spmv_csr(x=x, prepared=p)
    _bars(y, ref, torch.float64)
    assert torch.equal(y, fs.flagsparse_spmv_csr(x=x, prepared=p))
    # linearity: A(2x - z) = 2Ax - Az to fp64 rounding
    z = synthetic.uniform_values(5, 8, shape[1], torch.float64, dev)
    lhs = fs.flagsparse_spmv_csr(x=2 * x - z, prepared=p).cpu().numpy()
    rhs = 2 * ref - oracle.spmv_csr(ptr.cpu(), idx.cpu(), data.cpu(), z.cpu())
    assert oracle.rel_l2(lhs, rhs) <= 1e-12


def test_cfg4_full(dev):
    print("full size cfg4", flush=True)
    data, row, col, x, shape = synthetic.coo_uniform(device=dev)
    p = fs.prepare_spmv_coo(data, row, col, shape)
    assert p._run_layout().kind == "xstage"
    ref = oracle.spmv_coo(row.cpu(), col.cpu(), data.cpu(), x.cpu(), shape[0])
    y = fs.flagsparse_spmv_coo(x=x, prepared=p)
    _bars(y, ref, torch.float32)
    assert torch.equal(y, fs.flagsparse_spmv_coo(x=x, prepared=p))
    zero = torch.zeros_like(x)
    assert int(torch.count_nonzero(fs.flagsparse_spmv_coo(x=zero, prepared=p))) == 0
    # x = 1: every row's sum of values, against the oracle's
    ones = torch.ones_like(x)
    ref1 = oracle.spmv_coo(row.cpu(), col.cpu(), data.cpu(), ones.cpu(), shape[0])
    _bars(fs.flagsparse_spmv_coo(x=ones, prepared=p), ref1, torch.float32)


@pytest.mark.parametrize("dtype,N,paths", [(torch.float32, 64, ("opt",)),
                                           (torch.float32, 16, ("base", "opt")),
                                           (torch.float64, 16, ("base",))])
def test_cfg5_full(dev, dtype, N, paths):
    print(f"full size cfg5 {dtype} N={N} {paths}", flush=True)
    data, idx, ptr, shape = synthetic.csr_banded_random(dtype=dtype, device=dev)
    B = synthetic.dense_uniform(shape[1], N, dtype=dtype, device=dev)
    ref = oracle.spmm_csr(ptr.cpu(), idx.cpu(), data.cpu(), B.cpu())
    # a column of the product is the SpMV of that column of B
    j = N // 3
    col = fs.flagsparse_spmv_csr(data, idx, ptr, B[:, j].contiguous(), shape)
    _bars(col, ref[:, j], dtype)
    for path in paths:
        if path == "opt":  # native accumulation
            p = fs.prepare_spmm_csr_opt(data, idx, ptr, shape)
            C = fs.flagsparse_spmm_csr_opt(B=B, prepared=p)
        else:  # the base path: float32 computed in float64
            C = fs.flagsparse_spmm_csr(data, idx, ptr, B, shape)
        _bars(C, ref, dtype)
        name = "float64" if dtype == torch.float64 else "float32"
        assert oracle.rel_l2(C[:, j], col) <= oracle.REL_L2_BOUND[name]
        if path == "base" and dtype == torch.float32:
            # both round an fp64 sum of the same products (in their own orders) to float32
            u = _ulp(C[:, j].cpu().numpy(), col.cpu().numpy())
            assert u.max() <= 1, u.max()
        del C


def _sampled_rows(ptr, idx, data, rows):
    """The CSR arrays of the listed rows only (host numpy), for an oracle over a row sample."""
    ip = ptr.cpu().numpy().astype(np.int64)
    starts, lengths = ip[rows], ip[rows + 1] - ip[rows]
    sub_ptr = np.zeros(rows.size + 1, dtype=np.int64)
    np.cumsum(lengths, out=sub_ptr[1:])
    pos = np.arange(sub_ptr[-1]) - np.repeat(sub_ptr[:-1], lengths) + np.repeat(starts, lengths)
    return sub_ptr, idx.cpu().numpy()[pos], data.cpu().numpy()[pos]


@pytest.mark.parametrize("dtype,N,opt", [(torch.float32, 256, True), (torch.float64, 64, False),
                                         (torch.float64, 256, True)])
def test_cfg5_full_column_tiled(dev, dtype, N, opt):
    # B of 512 MiB - 2 GiB: the launch reads B in column tiles (spmm_csr.SPMM_B_TILE_BYTES);
    # a strided sample of C's rows against the oracle over the same rows, and a column of C
    # against the SpMV of that column of B
    from flagsparse_amd import spmm_csr

    print(f"full size cfg5 column-tiled {dtype} N={N} opt={opt}", flush=True)
    data, idx, ptr, shape = synthetic.csr_banded_random(dtype=dtype, device=dev)
    B = synthetic.dense_uniform(shape[1], N, dtype=dtype, device=dev)
    assert spmm_csr._auto_tile_cols(B) is not None
    if opt:
        C = fs.flagsparse_spmm_csr_opt(B=B, prepared=fs.prepare_spmm_csr_opt(data, idx, ptr,
                                                                               shape))
    else:
        C = fs.flagsparse_spmm_csr(data, idx, ptr, B, shape)
    rows = np.unique(np.concatenate([np.arange(0, shape[0], 61), [shape[0] - 1]]))
    sp, si, sd = _sampled_rows(ptr, idx, data, rows)
    ref = oracle.spmm_csr(sp, si, sd, B.cpu())
    got = C[torch.from_numpy(rows).to(dev)]
    _bars(got, ref, dtype)
    for j in (0, N // 2 + 1, N - 1):  # first, middle (another tile) and last column
        col = fs.flagsparse_spmv_csr(data, idx, ptr, B[:, j].contiguous(), shape)
        name = "float64" if dtype == torch.float64 else "float32"
        assert oracle.rel_l2(C[:, j], col) <= oracle.REL_L2_BOUND[name]
    del C, B
    torch.cuda.empty_cache()


def test_sddmm_full(dev):
    print("full size sddmm K=64", flush=True)
    _, idx, ptr, shape = synthetic.csr_banded_random(device=dev)
    x = synthetic.dense_uniform(shape[0], 64, seed=1, device=dev)
    y = synthetic.dense_uniform(shape[1], 64, seed=2, device=dev)
    p = fs.prepare_sddmm_csr(idx, ptr, shape, k_hint=64)
    out = fs.flagsparse_sddmm_csr(x=x, y=y, prepared=p)
    ref = oracle.sddmm_csr(ptr.cpu(), idx.cpu(), x.cpu(), y.cpu())
    _bars(out, ref, torch.float32)
