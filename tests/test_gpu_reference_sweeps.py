"""The reference test scripts' synthetic sweeps, on the GPU, with their own pass rules.

- tests/test_spmv.py:19-24 (shapes and nnz), :211-218 (tolerances): CSR SpMV on the reference
  generator's matrices (_common.py:166-181: unsorted columns, repeated (row, col)), float32 and
  float64, int32 indices, both accumulation paths and the COO -> CSR route.
- tests/test_spmv_coo.py:19, :171-176 (a dense N(0,1) matrix with 10 % of it kept, in row-major
  order), :323-326 (tolerances): COO SpMV by both routes (row runs and atomics).
- tests/test_spmm.py:41-46 (shapes, nnz and N), :138-151 (the library's float32 (1e-6, 1e-5) /
  float64 (1e-10, 1e-8) rule), int32 and int64 indices; tests/test_spmm_opt.py:202-224
  ((1e-4, 1e-2) / (1e-12, 1e-10) for the opt path).

The reference draws unseeded inputs; here every case is seeded (flagsparse_amd/synthetic.py).
A case passes when max |y - ref| / (atol + rtol |ref|) <= 1 against the fp64 oracle, as in the
scripts.
"""

import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu

SPMV_CASES = [(512, 512, 4096), (1024, 1024, 16384), (2048, 2048, 65536), (4096, 4096, 131072)]
SPMV_TOL = {torch.float32: (1.25e-4, 1.25e-2), torch.float64: (1e-12, 1e-10)}
COO_SIZES = [(512, 512), (1024, 1024), (2048, 2048)]
COO_TOL = {torch.float32: (1e-4, 1e-2), torch.float64: (1e-12, 1e-10)}
SPMM_CASES = [(512, 512, 4096, 16), (1024, 1024, 16384, 32), (2048, 2048, 65536, 64),
              (4096, 4096, 131072, 64)]
SPMM_TOL = {torch.float32: (1e-6, 1e-5), torch.float64: (1e-10, 1e-8)}
SPMM_OPT_TOL = {torch.float32: (1e-4, 1e-2), torch.float64: (1e-12, 1e-10)}


def _ratio(out, ref, tol):
    atol, rtol = tol
    return oracle.allclose_ratio(out, ref, atol, rtol)


@pytest.mark.parametrize("case", SPMV_CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_spmv_script_sweep(dev, case, dtype):
    m, n, nnz = case
    data, idx, ptr = synthetic.build_random_csr(m, n, nnz, dtype, torch.int32, "cpu",
                                                seed=m + nnz)
    x = synthetic.normal_values(m + nnz, 76, n, dtype, "cpu")
    print(f"spmv sweep {case} {dtype}", flush=True)
    ref = oracle.spmv_csr(ptr, idx, data, x)
    d, i, p, xd = data.to(dev), idx.to(dev), ptr.to(dev), x.to(dev)
    for use_opt in (False, True):
        y = fs.flagsparse_spmv_csr(d, i, p, xd, (m, n), use_opt=use_opt)
        assert _ratio(y, ref, SPMV_TOL[dtype]) <= 1.0
    rows = torch.repeat_interleave(torch.arange(m), ptr[1:] - ptr[:-1])
    y = fs.flagsparse_spmv_coo_tocsr(d, rows.to(dev), i, xd, (m, n))
    assert _ratio(y, ref, SPMV_TOL[dtype]) <= 1.0


@pytest.mark.parametrize("size", COO_SIZES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_spmv_coo_script_sweep(dev, size, dtype):
    m, n = size
    seed = m + 7
    A = synthetic.normal_values(seed, 77, m * n, dtype, "cpu").reshape(m, n)
    keep = synthetic.uniform_values(seed, 90, m * n, torch.float64, "cpu", 0.0, 1.0) < 0.1
    A = A * keep.reshape(m, n).to(dtype)
    row, col = torch.nonzero(A, as_tuple=True)  # row-major order, as the script's dense -> COO
    data = A[row, col]
    x = synthetic.normal_values(seed, 79, n, dtype, "cpu")
    print(f"coo sweep {size} {dtype} nnz={data.numel()}", flush=True)
    ref = oracle.spmv_coo(row, col, data, x, m)
    d, r, c, xd = data.to(dev), row.to(dev), col.to(dev), x.to(dev)
    for sort_by_row in (True, False):
        p = fs.prepare_spmv_coo(d, r, c, (m, n), sort_by_row=sort_by_row)
        y = fs.flagsparse_spmv_coo(x=xd, prepared=p)
        assert _ratio(y, ref, COO_TOL[dtype]) <= 1.0


@pytest.mark.parametrize("case", SPMM_CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_spmm_script_sweep(dev, case, dtype, index_dtype):
    m, n, nnz, N = case
    data, idx, ptr = synthetic.build_random_csr(m, n, nnz, dtype, index_dtype, "cpu",
                                                seed=m + N)
    B = synthetic.normal_values(m + N, 81, n * N, dtype, "cpu").reshape(n, N)
    print(f"spmm sweep {case} {dtype} {index_dtype}", flush=True)
    ref = oracle.spmm_csr(ptr, idx, data, B)
    d, i, p, Bd = data.to(dev), idx.to(dev), ptr.to(dev), B.to(dev)
    assert _ratio(fs.flagsparse_spmm_csr(d, i, p, Bd, (m, n)), ref, SPMM_TOL[dtype]) <= 1.0
    prep = fs.prepare_spmm_csr_opt(d, i, p, (m, n))
    C = fs.flagsparse_spmm_csr_opt(B=Bd, prepared=prep)
    assert _ratio(C, ref, SPMM_OPT_TOL[dtype]) <= 1.0
