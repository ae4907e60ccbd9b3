""".mtx loaders (flagsparse_amd/mtx.py over the native reader fsp_mtx_read), on the CPU.

Pinned by scipy.io.mmread (an independent Matrix Market reader) for the storage kinds scipy
accepts - general, symmetric, skew-symmetric, hermitian, pattern, integer - and by explicit
expected arrays for the reference-specific rules scipy does not share: entries outside the
shape are dropped, only the first nnz entry lines count, duplicates are summed in file order
(tests/test_spmv.py:29-103, tests/test_spmm_coo.py:156-249, tests/test_spmv_coo.py:257-305).
"""

import numpy as np
import pytest
import scipy.io
import scipy.sparse as sp
import torch

from flagsparse_amd import mtx


def _write(tmp_path, name, text):
    p = tmp_path / name
    p.write_text(text)
    return str(p)


def _scipy_csr(path):
    A = sp.csr_matrix(scipy.io.mmread(path))
    A.sum_duplicates()
    A.sort_indices()
    return A


def _check_csr(path, dtype=torch.float64):
    data, indices, indptr, shape = mtx.load_mtx_to_csr_torch(path, dtype=dtype, device="cpu")
    A = _scipy_csr(path)
    assert shape == A.shape
    assert indices.dtype == torch.int64 and indptr.dtype == torch.int64
    assert np.array_equal(indptr.numpy(), A.indptr)
    assert np.array_equal(indices.numpy(), A.indices)
    np.testing.assert_allclose(data.numpy(), A.data, rtol=1e-15, atol=0)
    # the COO loader gives the same summed entries in (row, col) order
    v, r, c, shape2 = mtx.load_mtx_to_coo_torch(path, dtype=dtype, device="cpu")
    Ac = A.tocoo()
    assert shape2 == A.shape
    assert np.array_equal(r.numpy(), Ac.row) and np.array_equal(c.numpy(), Ac.col)
    np.testing.assert_allclose(v.numpy(), Ac.data, rtol=1e-15, atol=0)


GENERAL = """%%MatrixMarket matrix coordinate real general
% a comment
4 5 7

1 1 1.5
2 3 -2.25
4 5 3e-1
1 1 0.5
3 2 7
2 3 1.0
4 1 -1
"""


def test_general_with_duplicates_comments_and_blank_lines(tmp_path):
    _check_csr(_write(tmp_path, "g.mtx", GENERAL))


@pytest.mark.parametrize("symmetry", ["symmetric", "skew-symmetric"])
def test_symmetric_storage(tmp_path, symmetry):
    diag = "" if symmetry == "skew-symmetric" else "1 1 2.0\n3 3 -4\n"
    n_diag = 0 if symmetry == "skew-symmetric" else 2
    text = (f"%%MatrixMarket matrix coordinate real {symmetry}\n4 4 {4 + n_diag}\n" + diag +
            "2 1 1.25\n3 1 -0.5\n4 2 6\n4 3 1e2\n")
    _check_csr(_write(tmp_path, "s.mtx", text))


def test_pattern_and_integer(tmp_path):
    _check_csr(_write(tmp_path, "p.mtx", "%%MatrixMarket matrix coordinate pattern general\n"
                                         "3 3 4\n1 2\n2 2\n3 1\n3 3\n"))
    _check_csr(_write(tmp_path, "ps.mtx", "%%MatrixMarket matrix coordinate pattern symmetric\n"
                                          "3 3 3\n2 1\n3 3\n3 2\n"))
    _check_csr(_write(tmp_path, "i.mtx", "%%MatrixMarket matrix coordinate integer general\n"
                                         "2 3 3\n1 3 -7\n2 1 4\n2 2 12\n"))


def test_hermitian_complex(tmp_path):
    path = _write(tmp_path, "h.mtx", "%%MatrixMarket matrix coordinate complex hermitian\n"
                                     "3 3 3\n1 1 2.0 0.0\n2 1 1.0 -3.0\n3 2 0.5 4.0\n")
    v, r, c, shape = mtx.load_mtx_to_coo_torch(path, dtype=torch.complex128, device="cpu")
    A = sp.coo_matrix(scipy.io.mmread(path)).tocsr()
    A.sort_indices()
    Ac = A.tocoo()
    assert np.array_equal(r.numpy(), Ac.row) and np.array_equal(c.numpy(), Ac.col)
    np.testing.assert_allclose(v.numpy(), Ac.data, rtol=1e-15, atol=0)
    with pytest.raises(TypeError, match="complex"):
        mtx.load_mtx_to_coo_torch(path, dtype=torch.float32, device="cpu")


def test_random_file_written_by_scipy(tmp_path):
    rng = np.random.default_rng(3)
    A = sp.random(700, 500, density=0.02, random_state=rng, format="coo")
    path = str(tmp_path / "r.mtx")
    scipy.io.mmwrite(path, A)
    _check_csr(path)
    S = sp.random(400, 400, density=0.03, random_state=rng, format="csr")
    S = (S + S.T).tocoo()
    path = str(tmp_path / "rs.mtx")
    scipy.io.mmwrite(path, S, symmetry="symmetric")
    _check_csr(path)


def test_reference_rules_scipy_does_not_share(tmp_path):
    # out-of-range entries are dropped; only the first nnz entry lines count; a line with one
    # token is skipped
    path = _write(tmp_path, "o.mtx", "%%MatrixMarket matrix coordinate real general\n"
                                     "3 3 4\n1 1 1\n4 1 9\n7\n2 2 2\n3 5 9\n3 3 3\n")
    data, indices, indptr, shape = mtx.load_mtx_to_csr_torch(path, dtype=torch.float64,
                                                             device="cpu")
    assert shape == (3, 3)
    assert indptr.tolist() == [0, 1, 2, 2]  # "3 3 3" is the fifth entry line: not read
    assert indices.tolist() == [0, 1] and data.tolist() == [1.0, 2.0]
    # duplicates are summed in file order: (1e16 + 1) - 1e16 == 0 in float64
    path = _write(tmp_path, "d.mtx", "%%MatrixMarket matrix coordinate real general\n"
                                     "1 1 3\n1 1 1e16\n1 1 1\n1 1 -1e16\n")
    data, _, _, _ = mtx.load_mtx_to_csr_torch(path, dtype=torch.float64, device="cpu")
    assert data.tolist() == [((0.0 + 1e16) + 1.0) - 1e16]
    # a comment between entry lines is skipped (scipy's reader rejects it)
    path = _write(tmp_path, "c.mtx", "%%MatrixMarket matrix coordinate real general\n"
                                     "2 2 2\n1 2 5\n% note\n2 1 6\n")
    data, indices, indptr, _ = mtx.load_mtx_to_csr_torch(path, dtype=torch.float64, device="cpu")
    assert data.tolist() == [5.0, 6.0] and indices.tolist() == [1, 0]
    # no entries
    path = _write(tmp_path, "e.mtx", "%%MatrixMarket matrix coordinate real general\n5 4 0\n")
    data, indices, indptr, shape = mtx.load_mtx_to_csr_torch(path, device="cpu")
    assert data.numel() == 0 and indptr.tolist() == [0] * 6 and shape == (5, 4)


def test_uncoalesced_order_keeps_file_order_and_twins(tmp_path):
    path = _write(tmp_path, "u.mtx", "%%MatrixMarket matrix coordinate real skew-symmetric\n"
                                     "3 3 3\n2 1 1.5\n3 2 -2\n2 1 0.25\n")
    v, r, c, _ = mtx.load_mtx_to_coo_torch(path, dtype=torch.float64, device="cpu",
                                           coalesce=False)
    assert r.tolist() == [1, 0, 2, 1, 1, 0]
    assert c.tolist() == [0, 1, 1, 2, 0, 1]
    assert v.tolist() == [1.5, -1.5, -2.0, 2.0, 0.25, -0.25]


def test_errors(tmp_path):
    with pytest.raises(ValueError, match="cannot open"):
        mtx.read_mtx_entries(str(tmp_path / "missing.mtx"))
    with pytest.raises(NotImplementedError, match="array"):
        mtx.read_mtx_entries(_write(tmp_path, "a.mtx",
                                    "%%MatrixMarket matrix array real general\n2 2\n1\n2\n3\n4\n"))
    with pytest.raises(ValueError, match="header"):
        mtx.read_mtx_entries(_write(tmp_path, "h.mtx", "% only comments\n"))
    with pytest.raises(ValueError, match="entry"):
        mtx.read_mtx_entries(_write(tmp_path, "b.mtx",
                                    "%%MatrixMarket matrix coordinate real general\n"
                                    "2 2 1\n1 x 2.0\n"))
    path = _write(tmp_path, "m.mtx", "%%MatrixMarket matrix coordinate real general\n"
                                     "2 2 2\n1 1\n2 2 3\n")
    with pytest.raises(ValueError, match="missing"):
        mtx.load_mtx_to_coo_torch(path, device="cpu")
    v, r, c, _ = mtx.load_mtx_to_coo_torch(path, dtype=torch.float64, device="cpu",
                                           coalesce=False)
    assert v.tolist() == [0.0, 3.0]  # a missing value reads as 0 in this loader


@pytest.mark.parametrize("text", ["   %%Matrix", "\t%%MatrixMarke", "  %", "%%MatrixMarket"])
def test_truncated_header_at_end_of_file(tmp_path, text):
    # a header cut short after leading blanks at the very end of the file (no newline): the
    # reader compares only the bytes that exist, and reports a missing header
    with pytest.raises(ValueError, match="header"):
        mtx.read_mtx_entries(_write(tmp_path, "t.mtx", text))
