"""Matrix Market (.mtx) loaders: the on-disk format of the reference's SuiteSparse drivers.

The file is parsed by the library's native reader (``fsp_mtx_read``, flagsparse_amd/csrc/
mtx.cpp); the expansion and summation rules follow the reference's loaders:

  load_mtx_to_csr_torch   tests/test_spmv.py:29-103 (and its copies in test_spmv_opt.py,
                          test_spmm.py, test_spmm_opt.py): pattern entries are 1.0; a
                          symmetric / hermitian entry off the diagonal is mirrored, a
                          skew-symmetric one mirrored with the opposite sign; entries outside
                          the shape are dropped; duplicates are summed (float64, in file order);
                          columns sorted in each row; int64 indices and indptr
  load_mtx_to_coo_torch   tests/test_spmm_coo.py:156-249 with coalesce=True (the same summed
                          entries in (row, col) order; complex files need a complex dtype),
                          tests/test_spmv_coo.py:257-305 with coalesce=False (entries in file
                          order, each mirrored entry right after its source, no summation)

Only coordinate files are read; dense "array" files raise NotImplementedError.
"""

import ctypes
import os

import numpy as np
import torch

from . import _abi

_FIELD_PATTERN, _FIELD_COMPLEX = 1, 2
_SYM_SYMMETRIC, _SYM_SKEW, _SYM_HERMITIAN = 1, 2, 3


def read_mtx_entries(file_path):
    """Raw entries of a coordinate .mtx file: (rows int64, cols int64, vals, shape, info) with
    0-based indices in file order; vals is float64, or complex128 for complex files; info holds
    the header nnz, field, symmetry and the number of entries lacking a value."""
    L = _abi.lib()
    path = os.fsencode(os.fspath(file_path))
    info = (ctypes.c_int64 * 7)()

    def _raise_on(rc):
        if rc != 0:
            msg = L.fsp_last_error().decode(errors="replace")
            if rc == -3:
                raise NotImplementedError(msg)
            raise ValueError(msg)

    _raise_on(L.fsp_mtx_read(path, ctypes.cast(info, ctypes.c_void_p), None, None, None, 0))
    n_rows, n_cols, nnz = int(info[0]), int(info[1]), int(info[2])
    cap = max(nnz, 0)
    field = int(info[3])
    rows = np.empty(cap, dtype=np.int64)
    cols = np.empty(cap, dtype=np.int64)
    vals = np.empty(cap * (2 if field == _FIELD_COMPLEX else 1), dtype=np.float64)
    if cap > 0:
        _raise_on(L.fsp_mtx_read(path, ctypes.cast(info, ctypes.c_void_p),
                                 rows.ctypes.data_as(ctypes.c_void_p),
                                 cols.ctypes.data_as(ctypes.c_void_p),
                                 vals.ctypes.data_as(ctypes.c_void_p), cap))
    n = int(info[5]) if cap > 0 else 0
    rows, cols = rows[:n], cols[:n]
    if field == _FIELD_COMPLEX:
        vals = vals[:2 * n].view(np.complex128)
    else:
        vals = vals[:n]
        if field == _FIELD_PATTERN:
            vals = np.ones(n, dtype=np.float64)
    meta = {"nnz": nnz, "field": field, "symmetry": int(info[4]), "missing_values": int(info[6])}
    return rows, cols, vals, (n_rows, n_cols), meta


def _expand(rows, cols, vals, shape, symmetry):
    """Drop entries outside the shape; add the mirrored twin of every off-diagonal entry of
    symmetric / skew-symmetric / hermitian storage right after its source."""
    n_rows, n_cols = shape
    keep = (rows >= 0) & (rows < n_rows) & (cols >= 0) & (cols < n_cols)
    rows, cols, vals = rows[keep], cols[keep], vals[keep]
    if symmetry == 0:
        return rows, cols, vals
    twin = (rows != cols) & (cols < n_rows) & (rows < n_cols)
    if symmetry == _SYM_SKEW:
        tv = -vals
    elif symmetry == _SYM_HERMITIAN and np.iscomplexobj(vals):
        tv = np.conj(vals)
    else:
        tv = vals
    # interleave source / twin, then drop the twins that do not exist
    r2 = np.stack([rows, cols], axis=1).reshape(-1)
    c2 = np.stack([cols, rows], axis=1).reshape(-1)
    v2 = np.stack([vals, tv], axis=1).reshape(-1)
    m2 = np.stack([np.ones_like(twin), twin], axis=1).reshape(-1)
    return r2[m2], c2[m2], v2[m2]


def _coalesce(rows, cols, vals, n_cols):
    """Sum duplicate (row, col) keys in file order (a stable sort, then left-to-right sums,
    the order in which the reference's dictionaries accumulate) and return the entries in
    (row, col) order."""
    if rows.size == 0:
        return rows, cols, vals
    key = rows * max(int(n_cols), 1) + cols
    order = np.argsort(key, kind="stable")
    key, vals = key[order], vals[order]
    start = np.flatnonzero(np.concatenate([[True], key[1:] != key[:-1]]))
    sums = np.add.reduceat(vals, start)
    ukey = key[start]
    return ukey // max(int(n_cols), 1), ukey % max(int(n_cols), 1), sums


def _device(device):
    if device is None:
        return torch.device("cuda" if torch.cuda.is_available() else "cpu")
    return torch.device(device)


def load_mtx_to_csr_torch(file_path, dtype=torch.float32, device=None):
    """.mtx -> (data, indices int64, indptr int64, shape) on ``device`` (the rules of
    tests/test_spmv.py:29-103)."""
    device = _device(device)
    rows, cols, vals, shape, meta = read_mtx_entries(file_path)
    n_rows, n_cols = shape
    if meta["nnz"] == 0:
        return (torch.tensor([], dtype=dtype, device=device),
                torch.tensor([], dtype=torch.int64, device=device),
                torch.zeros(n_rows + 1, dtype=torch.int64, device=device), (n_rows, n_cols))
    rows, cols, vals = _expand(rows, cols, vals, shape, meta["symmetry"])
    rows, cols, vals = _coalesce(rows, cols, vals, n_cols)
    indptr = np.zeros(n_rows + 1, dtype=np.int64)
    np.cumsum(np.bincount(rows, minlength=n_rows), out=indptr[1:])
    return (torch.from_numpy(np.ascontiguousarray(vals)).to(device=device, dtype=dtype),
            torch.from_numpy(cols).to(device), torch.from_numpy(indptr).to(device),
            (n_rows, n_cols))


def load_mtx_to_coo_torch(file_path, dtype=torch.float32, device=None, coalesce=True):
    """.mtx -> (data, row int64, col int64, shape) on ``device``.  coalesce=True: summed
    entries in (row, col) order (tests/test_spmm_coo.py:156-249); coalesce=False: entries in
    file order with mirrored twins, duplicates kept (tests/test_spmv_coo.py:257-305)."""
    device = _device(device)
    rows, cols, vals, shape, meta = read_mtx_entries(file_path)
    n_rows, n_cols = shape
    if meta["nnz"] == 0:
        empty = torch.tensor([], dtype=torch.int64, device=device)
        return torch.tensor([], dtype=dtype, device=device), empty, empty.clone(), shape
    if np.iscomplexobj(vals) and not dtype.is_complex:
        raise TypeError(f"Matrix Market file {file_path} stores complex values but requested "
                        f"dtype {dtype}")
    if coalesce and meta["missing_values"]:
        raise ValueError(f"Matrix Market file {file_path}: an entry is missing its value")
    rows, cols, vals = _expand(rows, cols, vals, shape, meta["symmetry"])
    if coalesce:
        rows, cols, vals = _coalesce(rows, cols, vals, n_cols)
    return (torch.from_numpy(np.ascontiguousarray(vals)).to(device=device, dtype=dtype),
            torch.from_numpy(np.ascontiguousarray(rows)).to(device),
            torch.from_numpy(np.ascontiguousarray(cols)).to(device), shape)
