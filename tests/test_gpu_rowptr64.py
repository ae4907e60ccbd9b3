"""The 64-bit row-pointer kernels on the GPU.  Matrices with 2^31 or more entries read int64 row
pointers (and int64 entry ranges); the threshold is lowered to 0 here so that small matrices
take those kernel instantiations.  Each result is checked against the fp64 CPU oracle and
against the 32-bit row-pointer run of the same call, which must agree bit for bit (the two
differ only in the width of the row-pointer loads)."""

import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _common, _spmv_layouts, synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu

# short rows, empty rows and rows long enough to be cut into chunks (> 4093 entries)
LENGTHS = [3, 0, 9000, 1, 17, 0, 0, 5000] + [7] * 3000 + [0] * 500 + [12000, 2] + [40] * 700


def _csr(lengths, n_cols, seed, dtype):
    keys = synthetic._distinct_sorted_columns(torch.as_tensor(lengths, dtype=torch.int64),
                                              n_cols, seed, 1)
    ip, cols = synthetic._csr_from_keys(keys, len(lengths), n_cols)
    vals = synthetic.uniform_values(seed, 2, cols.numel(), dtype, "cpu")
    return vals, cols.to(torch.int32), ip.to(torch.int64)


def _bound(dtype):
    return oracle.REL_L2_BOUND["float64" if dtype == torch.float64 else "float32"]


def _both(monkeypatch, fn):
    """(result with 32-bit row pointers, result with 64-bit row pointers, the 64-bit layout)."""
    y32, _ = fn()
    monkeypatch.setattr(_common, "ROWPTR32_MAX_NNZ", 0)
    y64, layout = fn()
    monkeypatch.setattr(_common, "ROWPTR32_MAX_NNZ", _common._INDEX_LIMIT_INT32)
    return y32, y64, layout


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("use_opt", [False, True])
def test_spmv_csr_rowptr64(dev, monkeypatch, dtype, use_opt):
    monkeypatch.setattr(_spmv_layouts, "FORCE", "rowblock")
    vals, cols, ip = _csr(LENGTHS, 50000, 5, dtype)
    x = synthetic.uniform_values(5, 3, 50000, dtype, "cpu")
    shape = (len(LENGTHS), 50000)
    print(f"rowptr64 spmv csr {dtype} use_opt={use_opt}", flush=True)

    def run():
        p = fs.prepare_spmv_csr(vals.to(dev), cols.to(dev), ip.to(dev), shape)
        y = fs.flagsparse_spmv_csr(x=x.to(dev), prepared=p, use_opt=use_opt)
        return y, p._kernel(use_opt)

    y32, y64, lay = _both(monkeypatch, run)
    assert lay.kind == "rowblock" and lay.rowptr_bits == 64 and lay.plan.n_split_rows == 3
    assert oracle.rel_l2(y64, oracle.spmv_csr(ip, cols, vals, x)) <= _bound(dtype)
    assert torch.equal(y32, y64)


def test_spmv_coo_rowptr64(dev, monkeypatch):
    monkeypatch.setattr(_spmv_layouts, "FORCE", "rowblock")
    vals, cols, ip = _csr(LENGTHS, 50000, 6, torch.float32)
    row = torch.repeat_interleave(torch.arange(len(LENGTHS), dtype=torch.int32),
                                  torch.as_tensor(LENGTHS))
    x = synthetic.uniform_values(6, 3, 50000, torch.float32, "cpu")
    shape = (len(LENGTHS), 50000)
    print("rowptr64 spmv coo", flush=True)

    def run():
        p = fs.prepare_spmv_coo(vals.to(dev), row.to(dev), cols.to(dev), shape)
        return fs.flagsparse_spmv_coo(x=x.to(dev), prepared=p), p._run_layout()

    y32, y64, lay = _both(monkeypatch, run)
    assert lay.kind == "rowblock" and lay.rowptr_bits == 64
    assert oracle.rel_l2(y64, oracle.spmv_coo(row, cols, vals, x, shape[0])) <= 1e-5
    assert torch.equal(y32, y64)


@pytest.mark.parametrize("dtype,N", [(torch.float32, 64), (torch.float32, 5), (torch.float64, 16)])
def test_spmm_csr_rowptr64(dev, monkeypatch, dtype, N):
    vals, cols, ip = _csr(LENGTHS, 20000, 7, dtype)
    B = synthetic.dense_uniform(20000, N, dtype, seed=7, device="cpu")
    shape = (len(LENGTHS), 20000)
    ref = oracle.spmm_csr(ip, cols, vals, B)
    print(f"rowptr64 spmm csr {dtype} N={N}", flush=True)

    def run():
        p = fs.prepare_spmm_csr_opt(vals.to(dev), cols.to(dev), ip.to(dev), shape)
        return fs.flagsparse_spmm_csr_opt(B=B.to(dev), prepared=p), p._kernel_csr()

    C32, C64, kc = _both(monkeypatch, run)
    assert kc.rowptr_bits == 64
    assert oracle.rel_l2(C64, ref) <= _bound(dtype)
    assert torch.equal(C32, C64)

    def run_base():
        return fs.flagsparse_spmm_csr(vals.to(dev), cols.to(dev), ip.to(dev), B.to(dev),
                                      shape), None

    C32, C64, _ = _both(monkeypatch, run_base)
    assert oracle.rel_l2(C64, ref) <= _bound(dtype)
    assert torch.equal(C32, C64)


def test_spmm_coo_rowptr64(dev, monkeypatch):
    vals, cols, ip = _csr(LENGTHS, 20000, 8, torch.float64)
    row = torch.repeat_interleave(torch.arange(len(LENGTHS), dtype=torch.int32),
                                  torch.as_tensor(LENGTHS))
    B = synthetic.dense_uniform(20000, 24, torch.float64, seed=8, device="cpu")
    shape = (len(LENGTHS), 20000)
    print("rowptr64 spmm coo", flush=True)

    def run():
        return fs.flagsparse_spmm_coo(vals.to(dev), row.to(dev), cols.to(dev), B.to(dev),
                                      shape), None

    C32, C64, _ = _both(monkeypatch, run)
    assert oracle.rel_l2(C64, oracle.spmm_coo(row, cols, vals, B, shape[0])) <= 1e-12
    assert torch.equal(C32, C64)


@pytest.mark.parametrize("dtype,K", [(torch.float32, 64), (torch.float64, 33)])
def test_sddmm_rowptr64(dev, monkeypatch, dtype, K):
    vals, cols, ip = _csr(LENGTHS, 20000, 9, dtype)
    x = synthetic.dense_uniform(len(LENGTHS), K, dtype, seed=10, device="cpu")
    y = synthetic.dense_uniform(20000, K, dtype, seed=11, device="cpu")
    shape = (len(LENGTHS), 20000)
    print(f"rowptr64 sddmm {dtype} K={K}", flush=True)

    def run():
        p = fs.prepare_sddmm_csr(cols.to(dev), ip.to(dev), shape, k_hint=K)
        out = fs.flagsparse_sddmm_csr(x=x.to(dev), y=y.to(dev), prepared=p)
        return out, p

    o32, o64, p = _both(monkeypatch, run)
    assert p._kernel_ptr.dtype == torch.int64
    assert oracle.rel_l2(o64, oracle.sddmm_csr(ip, cols, x, y)) <= _bound(dtype)
    assert torch.equal(o32, o64)
