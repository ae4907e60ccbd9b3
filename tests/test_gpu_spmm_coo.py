"""COO SpMM on the GPU: flagsparse_spmm_coo (row-run route through spmm_rowblock_kernel) and the
atomic route (spmm_coo_atomic_kernel) against the fp64 C oracle, plus the reference's API
cases (tests/test_spmm_coo.py:942-1060) and its dense-column coverage table (:47-54).

Bar: relative L2 error <= 1e-5 (fp32) / 1e-12 (fp64) against the oracle's fp64 product, and
the reference script's allclose (tests/test_spmm_coo.py:134-143: fp32 atol 1e-4 rtol 1e-2,
fp64 atol 1e-12 rtol 1e-10).
"""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import spmm_coo, synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu

SCRIPT_TOL = {torch.float32: (1e-4, 1e-2), torch.float64: (1e-12, 1e-10)}


def _check(C, row, col, data, B, n_rows):
    ref = oracle.spmm_coo(row, col, data, B, n_rows)
    assert tuple(C.shape) == ref.shape
    if C.numel() == 0:
        return
    name = "float64" if C.dtype == torch.float64 else "float32"
    assert oracle.rel_l2(C, ref) <= oracle.REL_L2_BOUND[name]
    atol, rtol = SCRIPT_TOL[C.dtype]
    assert oracle.allclose_ratio(C, ref, atol, rtol) <= 1.0


def _random_coo(dev, n_rows, n_cols, nnz, dtype, index_dtype, seed, sort=False, dups=0):
    data, row, col = synthetic.build_random_coo(n_rows, n_cols, nnz, dtype, index_dtype, dev,
                                                seed=seed)
    if dups:
        row[:dups] = row[dups:2 * dups]
        col[:dups] = col[dups:2 * dups]
    if sort:
        key = row.to(torch.int64) * n_cols + col.to(torch.int64)
        order = torch.argsort(key)
        data, row, col = data[order], row[order], col[order]
    return data, row, col


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("sort", [False, True])
def test_spmm_coo_random(dev, dtype, index_dtype, sort):
    n_rows, n_cols, N = 700, 500, 40
    data, row, col = _random_coo(dev, n_rows, n_cols, 9000, dtype, index_dtype, seed=11,
                                 sort=sort, dups=500)
    B = synthetic.dense_uniform(n_cols, N, dtype, seed=12, device=dev)
    print(f"coo spmm {dtype} {index_dtype} sort={sort}", flush=True)
    C = fs.flagsparse_spmm_coo(data, row, col, B, (n_rows, n_cols))
    assert C.dtype == dtype and C.is_cuda
    _check(C, row, col, data, B, n_rows)
    Ca = spmm_coo._run_spmm_coo_route(data, row, col, B, (n_rows, n_cols), route="atomic")
    _check(Ca, row, col, data, B, n_rows)


@pytest.mark.parametrize("n_dense_cols", [4, 5, 12, 24, 48, 96])
def test_spmm_coo_dense_column_coverage(dev, n_dense_cols):
    # the reference's COO_TILE_CASES: 256 x 256, 4096 entries, N in {4, 5, 12, 24, 48, 96}
    data, row, col = _random_coo(dev, 256, 256, 4096, torch.float32, torch.int32, seed=n_dense_cols)
    B = synthetic.dense_uniform(256, n_dense_cols, torch.float32, seed=1, device=dev)
    C = fs.flagsparse_spmm_coo(data, row, col, B, (256, 256))
    _check(C, row, col, data, B, 256)


@pytest.mark.parametrize("block_n", [1, 8, 32, 100])
def test_spmm_coo_block_n_tiles(dev, block_n):
    data, row, col = _random_coo(dev, 300, 200, 3000, torch.float64, torch.int32, seed=3)
    B = synthetic.dense_uniform(200, 70, torch.float64, seed=4, device=dev)
    C = fs.flagsparse_spmm_coo(data, row, col, B, (300, 200), block_n=block_n, block_nnz=64)
    _check(C, row, col, data, B, 300)


def test_spmm_coo_long_rows_and_empty_rows(dev):
    # rows longer than the row-part threshold (split with a second pass) next to empty rows
    n_rows, n_cols = 64, 5000
    rows = [torch.full((4000,), 3), torch.full((1500,), 40), torch.arange(50, 60)]
    row = torch.cat(rows).to(torch.int32).to(dev)
    col = synthetic.randint(9, 1, row.numel(), n_cols, dev).to(torch.int32)
    data = synthetic.uniform_values(9, 2, row.numel(), torch.float32, dev)
    perm = torch.argsort(synthetic.uniform01(9, 3, row.numel(), dev))  # seeded shuffle
    data, row, col = data[perm], row[perm], col[perm]
    B = synthetic.dense_uniform(n_cols, 20, torch.float32, seed=9, device=dev)
    C = fs.flagsparse_spmm_coo(data, row, col, B, (n_rows, n_cols))
    _check(C, row, col, data, B, n_rows)
    assert torch.count_nonzero(C[0]) == 0 and torch.count_nonzero(C[63]) == 0


def test_spmm_coo_reference_api_cases(dev):
    # tests/test_spmm_coo.py:950-969 (negative cases on device tensors)
    data = torch.tensor([1.0, 2.0, 3.0], dtype=torch.float32, device=dev)
    row = torch.tensor([0, 0, 1], dtype=torch.int32, device=dev)
    col = torch.tensor([0, 1, 1], dtype=torch.int32, device=dev)
    B = torch.randn((2, 4), dtype=torch.float32, device=dev)
    cases = [
        (lambda: fs.flagsparse_spmm_coo(data, row, col, B, (2,)), ValueError),
        (lambda: fs.flagsparse_spmm_coo(data, row, col, B[0], (2, 2)), ValueError),
        (lambda: fs.flagsparse_spmm_coo(data, row, col, B.to(torch.float64), (2, 2)), TypeError),
        (lambda: fs.flagsparse_spmm_coo(data, row, col, torch.randn((3, 4), device=dev), (2, 2)),
         ValueError),
        (lambda: fs.flagsparse_spmm_coo(data, row[:-1], col, B, (2, 2)), ValueError),
        (lambda: fs.flagsparse_spmm_coo(data, row, col[:-1], B, (2, 2)), ValueError),
        (lambda: fs.flagsparse_spmm_coo(
            data, torch.tensor([0, 2, 1], dtype=torch.int32, device=dev), col, B, (2, 2)),
         IndexError),
        (lambda: fs.flagsparse_spmm_coo(
            data, row, torch.tensor([0, 3, 1], dtype=torch.int32, device=dev), B, (2, 2)),
         IndexError),
        (lambda: fs.flagsparse_spmm_coo(data, row, col, B, (2, 2), block_n=0), ValueError),
        (lambda: fs.flagsparse_spmm_coo(data, row, col, B, (2, 2), block_nnz=0), ValueError),
        (lambda: fs.flagsparse_spmm_coo(
            data, row, col, B, (2, 2), out=torch.empty((3, 4), dtype=torch.float32, device=dev)),
         ValueError),
        (lambda: fs.flagsparse_spmm_coo(
            data, row, col, B, (2, 2), out=torch.empty((2, 4), dtype=torch.float32)), ValueError),
        (lambda: fs.flagsparse_spmm_coo(data, row.to(torch.int16), col, B, (2, 2)), TypeError),
    ]
    for fn, exc in cases:
        with pytest.raises(exc):
            fn()


def test_spmm_coo_reference_positive_cases(dev):
    # tests/test_spmm_coo.py:993-1050: out path, empty matrix, N = 0, non-contiguous B,
    # unsorted duplicates (:497-503)
    data = torch.tensor([1.0, 2.0, 3.0], dtype=torch.float32, device=dev)
    row = torch.tensor([0, 0, 1], dtype=torch.int32, device=dev)
    col = torch.tensor([0, 1, 1], dtype=torch.int32, device=dev)
    B = synthetic.dense_uniform(2, 4, torch.float32, seed=2, device=dev)
    out = torch.empty((2, 4), dtype=torch.float32, device=dev)
    C = fs.flagsparse_spmm_coo(data, row, col, B, (2, 2), out=out)
    assert C.data_ptr() == out.data_ptr()
    _check(C, row, col, data, B, 2)

    empty = torch.tensor([], dtype=torch.float32, device=dev)
    eidx = torch.tensor([], dtype=torch.int32, device=dev)
    C = fs.flagsparse_spmm_coo(empty, eidx, eidx, B, (2, 2))
    assert C.shape == (2, 4) and torch.count_nonzero(C) == 0

    C = fs.flagsparse_spmm_coo(data, row, col, torch.empty((2, 0), device=dev), (2, 2))
    assert C.shape == (2, 0)

    Bt = synthetic.dense_uniform(4, 2, torch.float32, seed=3, device=dev).transpose(0, 1)
    assert not Bt.is_contiguous()
    _check(fs.flagsparse_spmm_coo(data, row, col, Bt, (2, 2)), row, col, data, Bt.contiguous(), 2)

    drow = torch.tensor([2, 0, 2, 1, 2, 0, 3, 2], dtype=torch.int64, device=dev)
    dcol = torch.tensor([1, 4, 1, 3, 0, 4, 2, 5], dtype=torch.int64, device=dev)
    dval = synthetic.uniform_values(8, 1, 8, torch.float64, dev)
    dB = synthetic.dense_uniform(6, 48, torch.float64, seed=8, device=dev)
    _check(fs.flagsparse_spmm_coo(dval, drow, dcol, dB, (4, 6)), drow, dcol, dval, dB, 4)


def test_spmm_coo_return_time_and_out_copy(dev):
    data, row, col = _random_coo(dev, 100, 80, 900, torch.float32, torch.int32, seed=5)
    B = synthetic.dense_uniform(80, 16, torch.float32, seed=6, device=dev)
    C, ms = fs.flagsparse_spmm_coo(data, row, col, B, (100, 80), return_time=True)
    assert ms >= 0.0
    _check(C, row, col, data, B, 100)
    # a non-contiguous out gets a copy of the result
    out = torch.empty((16, 100), dtype=torch.float32, device=dev).t()
    C2 = fs.flagsparse_spmm_coo(data, row, col, B, (100, 80), out=out)
    assert C2.data_ptr() == out.data_ptr()
    assert torch.equal(C2, C)


def test_spmm_coo_rowrun_is_deterministic(dev):
    data, row, col = _random_coo(dev, 400, 300, 6000, torch.float32, torch.int32, seed=8,
                                 dups=300)
    B = synthetic.dense_uniform(300, 33, torch.float32, seed=8, device=dev)
    C1 = fs.flagsparse_spmm_coo(data, row, col, B, (400, 300))
    C2 = fs.flagsparse_spmm_coo(data, row, col, B, (400, 300))
    assert torch.equal(C1, C2)
    # float32 inputs are summed in float64 and rounded once: equal to fp32(oracle) except where
    # the fp64 sums differ in their last bits across a rounding boundary
    ref = oracle.spmm_coo(row, col, data, B, 400).astype(np.float32)
    assert np.mean(C1.cpu().numpy() == ref) > 0.999


def test_benchmark_spmm_coo_case(dev):
    r = spmm_coo.benchmark_spmm_coo_case(n_rows=300, n_cols=250, nnz=4000, n_dense_cols=24,
                                         warmup=1, iters=3, compare_routes=True)
    assert set(r) == {"parameters", "performance", "verification", "backend_status",
                      "samples", "route_results", "parity", "route_samples"}
    assert r["verification"]["triton_match_reference"]
    assert r["parameters"]["block_n"] == 32 and r["parameters"]["n_row_runs"] > 0
    assert set(r["route_results"]) == {"rowrun", "atomic"}
    assert all(v["match_reference"] for v in r["route_results"].values())
    assert r["parity"]["rowrun_vs_atomic"]["match"]
    r = spmm_coo.comprehensive_spmm_coo_test(n_rows=128, n_cols=96, nnz=1000, n_dense_cols=5,
                                             dtype=torch.float64, warmup=1, iters=2)
    assert r["parameters"]["route"] == "rowrun" and r["verification"]["triton_match_reference"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("route", ["rowrun", "atomic"])
def test_canonical_route_as_the_reference_scripts_drive_it(dev, dtype, route):
    # tests/test_spmm_coo.py:288-375: validate, canonicalise (duplicates summed, entries in
    # (row, col) order, float32 widened to float64), time the canonical route and compare it
    # with torch.sparse.mm over the same canonical entries
    import flagsparse.sparse_operations.spmm_coo as ast_ops

    n_rows, n_cols, N = 600, 450, 24
    data, row, col = _random_coo(dev, n_rows, n_cols, 7000, dtype, torch.int64, seed=21,
                                 dups=400)
    B = synthetic.dense_uniform(n_cols, N, dtype, seed=22, device=dev)
    shape = (n_rows, n_cols)
    print(f"canonical route {dtype} {route}", flush=True)
    nd, nr, nc, nB, n_r, n_c, n_d = ast_ops._prepare_spmm_coo_inputs(data, row, col, B, shape)
    cd, cr, cc, cB, _, _, _, out_dtype, compute_dtype = \
        ast_ops._prepare_spmm_coo_canonical_prepared(nd, nr, nc, nB, n_r, n_c, n_d)
    assert out_dtype == dtype and compute_dtype == torch.float64
    assert cd.numel() < nd.numel()  # duplicates merged
    key = cr * n_cols + cc
    assert bool((key[1:] > key[:-1]).all())  # strictly increasing: sorted, no duplicates
    values, steady_ms, first_ms = ast_ops._benchmark_spmm_coo_canonical_route(
        cd, cr, cc, cB, n_r, n_d, out_dtype, 2, 5, None, 256, route)
    assert values.dtype == dtype and steady_ms > 0 and first_ms > 0
    expected = ast_ops._build_spmm_coo_pytorch_reference_from_canonical(cd, cr, cc, cB, shape,
                                                                        out_dtype)
    metrics = ast_ops._spmm_validation_metrics(values, expected)
    assert metrics["max_relative_error"] <= (1e-6 if dtype == torch.float32 else 1e-13)
    _check(values, row, col, data, B, n_rows)
