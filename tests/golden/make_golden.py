"""Writes the golden fixtures in tests/golden/*.npz.

Inputs come from the seeded SplitMix64 generators (flagsparse_amd/synthetic.py, bit-stable
across torch/numpy versions and devices for uniform-derived arrays).  Expected outputs are
computed here with scipy.sparse in float64 - an implementation independent of both the
oracle (oracle/fsp_oracle.c) and the HIP kernels - which is the reference's own definition of
correctness for this path (fp64 accumulation: tests/test_spmv.py:143-174,
tests/test_spmv_coo.py:56-71, tests/test_spmm.py:270-311).

Cases:
  cfg1_csr_f32     BASELINE configs[0]: 4096 x 4096, 16 distinct uniform columns per row,
                   int32, values and x ~ U(-1, 1), seed 0
  poisson64_f64    5-point Poisson on a 64 x 64 grid (configs[1] at reduced size)
  ragged_f32/f64   reference-generator shape: empty rows, unsorted and repeated columns
  longrow_spmm_f32 the reference's long-row API case shape (tests/test_spmm.py:383-395):
                   (2, 2048), a 1536-entry row and a 4-entry row, N = 48
  coo_dups_f32     unsorted COO with repeated (row, col) pairs and empty rows
  coo_spmm_ref_f32/f64
                   the reference's duplicate/unsorted COO SpMM case (tests/test_spmm_coo.py:
                   497-503: shape (4, 6), its fixed row/col lists, N = 48), seeded values
  coo_spmm_dups_f32/f64
                   unsorted COO with repeated (row, col) pairs and empty rows @ B, N = 24
  sddmm_f32_k64 / sddmm_f64_k33
                   SDDMM on a ragged CSR pattern (empty rows, repeated columns), alpha 1.25,
                   beta -0.5 with data; expected values from numpy row gathers in float64
  spmm_f32/f64_N   small CSR @ B for N in {1, 3, 4, 16, 64}

Run from the repository root:  python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import scipy.sparse as sp
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from flagsparse_amd import synthetic  # noqa: E402


def _np(t):
    return t.detach().cpu().numpy()


def _csr_expected(data, indices, indptr, shape, rhs):
    A = sp.csr_matrix((_np(data).astype(np.float64), _np(indices).astype(np.int64),
                       _np(indptr).astype(np.int64)), shape=shape)
    return A @ rhs.astype(np.float64)


def _save(name, **arrays):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    print(f"{path}: " + ", ".join(f"{k}{list(v.shape)}" for k, v in arrays.items()))


def _csr_case(name, data, indices, indptr, x, shape):
    y = _csr_expected(data, indices, indptr, shape, _np(x))
    _save(name, data=_np(data), indices=_np(indices), indptr=_np(indptr), x=_np(x),
          shape=np.array(shape, dtype=np.int64), y=y)


def main():
    d, i, p, x, shape = synthetic.csr_uniform_rows()
    _csr_case("cfg1_csr_f32", d, i, p, x, shape)

    d, i, p, x, shape = synthetic.csr_poisson2d(64)
    _csr_case("poisson64_f64", d, i, p, x, shape)

    for dtype, tag in ((torch.float32, "f32"), (torch.float64, "f64")):
        d, i, p = synthetic.build_random_csr(3000, 700, 5000, dtype, torch.int32, "cpu", seed=21)
        x = synthetic.uniform_values(21, 9, 700, dtype, "cpu")
        _csr_case(f"ragged_{tag}", d, i, p, x, (3000, 700))

    # long-row SpMM case
    cols = torch.cat([torch.arange(1536), torch.tensor([7, 129, 511, 1024])]).to(torch.int32)
    data = synthetic.uniform_values(3, 1, cols.numel(), torch.float32, "cpu")
    indptr = torch.tensor([0, 1536, 1540], dtype=torch.int64)
    B = synthetic.dense_uniform(2048, 48, torch.float32, seed=3)
    C = _csr_expected(data, cols, indptr, (2, 2048), _np(B))
    _save("longrow_spmm_f32", data=_np(data), indices=_np(cols), indptr=_np(indptr), B=_np(B),
          shape=np.array([2, 2048], dtype=np.int64), C=C)

    # unsorted COO with duplicates
    n_rows, n_cols, nnz = 900, 800, 6000
    row = synthetic.randint(4, 1, nnz, n_rows - 100, "cpu")  # rows >= 800 stay empty
    col = synthetic.randint(4, 2, nnz, n_cols, "cpu")
    row[:300] = row[300:600]
    col[:300] = col[300:600]
    vals = synthetic.uniform_values(4, 3, nnz, torch.float32, "cpu")
    x = synthetic.uniform_values(4, 4, n_cols, torch.float32, "cpu")
    y = sp.coo_matrix((_np(vals).astype(np.float64), (_np(row), _np(col))),
                      shape=(n_rows, n_cols)) @ _np(x).astype(np.float64)
    _save("coo_dups_f32", data=_np(vals), row=_np(row).astype(np.int32),
          col=_np(col).astype(np.int32), x=_np(x), shape=np.array([n_rows, n_cols]), y=y)

    # COO SpMM: the reference's duplicate/unsorted case and a larger unsorted one
    for dtype, tag in ((torch.float32, "f32"), (torch.float64, "f64")):
        row = torch.tensor([2, 0, 2, 1, 2, 0, 3, 2], dtype=torch.int32)
        col = torch.tensor([1, 4, 1, 3, 0, 4, 2, 5], dtype=torch.int32)
        vals = synthetic.uniform_values(5, 1, row.numel(), dtype, "cpu")
        B = synthetic.dense_uniform(6, 48, dtype, seed=5)
        C = sp.coo_matrix((_np(vals).astype(np.float64), (_np(row), _np(col))),
                          shape=(4, 6)) @ _np(B).astype(np.float64)
        _save(f"coo_spmm_ref_{tag}", data=_np(vals), row=_np(row), col=_np(col), B=_np(B),
              shape=np.array([4, 6], dtype=np.int64), C=C)

        n_rows, n_cols, nnz = 500, 400, 4000
        row = synthetic.randint(6, 1, nnz, n_rows - 50, "cpu")  # rows >= 450 stay empty
        col = synthetic.randint(6, 2, nnz, n_cols, "cpu")
        row[:200] = row[200:400]
        col[:200] = col[200:400]
        vals = synthetic.uniform_values(6, 3, nnz, dtype, "cpu")
        B = synthetic.dense_uniform(n_cols, 24, dtype, seed=6)
        C = sp.coo_matrix((_np(vals).astype(np.float64), (_np(row), _np(col))),
                          shape=(n_rows, n_cols)) @ _np(B).astype(np.float64)
        _save(f"coo_spmm_dups_{tag}", data=_np(vals), row=_np(row).astype(np.int32),
              col=_np(col).astype(np.int32), B=_np(B),
              shape=np.array([n_rows, n_cols], dtype=np.int64), C=C)

    # SDDMM: out[p] = alpha * dot(x[row(p)], y[col(p)]) + beta * data[p]
    for dtype, tag, K in ((torch.float32, "f32", 64), (torch.float64, "f64", 33)):
        d, i, p = synthetic.build_random_csr(400, 300, 5000, dtype, torch.int32, "cpu", seed=41)
        x = synthetic.dense_uniform(400, K, dtype, seed=42)
        y = synthetic.dense_uniform(300, K, dtype, seed=43)
        rows = np.repeat(np.arange(400), np.diff(_np(p)))
        xs, ys = _np(x).astype(np.float64), _np(y).astype(np.float64)
        out = 1.25 * np.einsum("pk,pk->p", xs[rows], ys[_np(i).astype(np.int64)]) \
            - 0.5 * _np(d).astype(np.float64)
        _save(f"sddmm_{tag}_k{K}", data=_np(d), indices=_np(i), indptr=_np(p), x=_np(x),
              y=_np(y), shape=np.array([400, 300], dtype=np.int64), alpha=np.array(1.25),
              beta=np.array(-0.5), out=out)

    # small SpMM
    for dtype, tag in ((torch.float32, "f32"), (torch.float64, "f64")):
        d, i, p = synthetic.build_random_csr(300, 200, 3000, dtype, torch.int32, "cpu", seed=31)
        for N in (1, 3, 4, 16, 64):
            B = synthetic.dense_uniform(200, N, dtype, seed=31 + N)
            C = _csr_expected(d, i, p, (300, 200), _np(B))
            _save(f"spmm_{tag}_n{N}", data=_np(d), indices=_np(i), indptr=_np(p), B=_np(B),
                  shape=np.array([300, 200], dtype=np.int64), C=C)


if __name__ == "__main__":
    main()
