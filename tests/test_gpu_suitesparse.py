"""The .mtx batch harness (flagsparse_amd.suitesparse) end to end on the GPU: Matrix Market
files written by scipy (general, symmetric, pattern) through SpMV, SpMM and SDDMM, checked
against float64 torch products with the reference scripts' tolerance."""

import csv

import numpy as np
import pytest
import scipy.io
import scipy.sparse as sp
import torch

from flagsparse_amd import suitesparse

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mtx_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("mtx")
    rng = np.random.default_rng(11)
    scipy.io.mmwrite(str(d / "general.mtx"), sp.random(900, 700, density=0.01, random_state=rng))
    S = sp.random(600, 600, density=0.02, random_state=rng, format="csr")
    scipy.io.mmwrite(str(d / "symmetric.mtx"), (S + S.T).tocoo(), symmetry="symmetric")
    P = sp.random(500, 800, density=0.01, random_state=rng, format="coo")
    P.data[:] = 1.0
    scipy.io.mmwrite(str(d / "pattern.mtx"), P, field="pattern")
    (d / "notes.txt").write_text("not a matrix")
    return d


@pytest.mark.parametrize("op", ["spmv", "spmm", "sddmm"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_batch(dev, mtx_dir, op, dtype, tmp_path):
    out_csv = tmp_path / "res.csv"
    rows = suitesparse.run_mtx_batch([str(mtx_dir)], op=op, value_dtype=dtype, dense_cols=24,
                                     warmup=1, iters=2, csv_path=str(out_csv))
    assert [r["path"].rsplit("/", 1)[1] for r in rows] == ["general.mtx", "pattern.mtx",
                                                           "symmetric.mtx"]
    for r in rows:
        assert r["error"] is None, r
        assert r["ok"], r
        assert r["ms"] > 0 and r["nnz"] > 0
    with open(out_csv) as fh:
        got = list(csv.DictReader(fh))
    assert len(got) == 3 and set(got[0]) == set(suitesparse.CSV_FIELDS)


def test_cli_and_bad_files(dev, mtx_dir, tmp_path):
    bad = tmp_path / "bad.mtx"
    bad.write_text("%%MatrixMarket matrix coordinate real general\n2 2 1\n1 x 2\n")
    rows = suitesparse.run_mtx_batch([str(bad), str(mtx_dir / "general.mtx")], warmup=1, iters=1)
    assert rows[0]["error"] and "ValueError" in rows[0]["error"] and rows[1]["ok"]
    assert suitesparse.main([str(mtx_dir / "general.mtx"), "--op", "spmm", "--dense-cols", "8",
                             "--warmup", "1", "--iters", "1"]) == 0
    assert suitesparse.expand_mtx_paths([str(mtx_dir), str(mtx_dir / "general.mtx")]) == \
        suitesparse.expand_mtx_paths([str(mtx_dir)])
