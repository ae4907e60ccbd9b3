"""CSR SpMM on the GPU against the fp64 CPU oracle, plus the reference's API checks.

Bars: relative L2 error <= 1e-5 (float32) / 1e-12 (float64) against the fp64 oracle
(north_star), and the reference scripts' allclose ratio <= 1 with (1e-4, 1e-2) / (1e-12, 1e-10)
(tests/test_spmm_opt.py:202-224).  The API cases follow tests/test_spmm.py:685-807: 15
negative cases with the expected exception types and 5 positive ones (out identity, empty
matrix, N = 0, non-contiguous B, a 1536-entry row).
"""

import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu


def _check(C, ref64):
    name = "float64" if C.dtype == torch.float64 else "float32"
    err = oracle.rel_l2(C, ref64)
    assert err <= oracle.REL_L2_BOUND[name], f"rel_l2 {err:.3e}"
    atol, rtol = oracle.REF_SCRIPT_TOL[name]
    assert oracle.allclose_ratio(C, ref64, atol, rtol) <= 1.0


def _csr_from_lengths(lengths, n_cols, seed, dtype):
    keys = synthetic._distinct_sorted_columns(torch.as_tensor(lengths, dtype=torch.int64),
                                              n_cols, seed, 1)
    ip, cols = synthetic._csr_from_keys(keys, len(lengths), n_cols)
    vals = synthetic.uniform_values(seed, 2, cols.numel(), dtype, "cpu")
    return vals, cols.to(torch.int32), ip, (len(lengths), n_cols)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("N", [16, 64, 256])
def test_banded_random_like_cfg5(dev, dtype, N):
    # cfg5's generator at 1/64 of the rows
    data, idx, ptr, shape = synthetic.csr_banded_random(1 << 14, dtype=dtype)
    B = synthetic.dense_uniform(shape[1], N, dtype=dtype)
    print(f"cfg5-like n={shape[0]} N={N} {dtype}", flush=True)
    ref = oracle.spmm_csr(ptr, idx, data, B)
    d, i, p, Bd = data.to(dev), idx.to(dev), ptr.to(dev), B.to(dev)
    _check(fs.flagsparse_spmm_csr_opt(d, i, p, Bd, shape), ref)
    _check(fs.flagsparse_spmm_csr(d, i, p, Bd, shape), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("N", [24, 64, 130])
def test_large_b_column_tiles(dev, monkeypatch, dtype, N):
    # the automatic column tiling of a B over half of SPMM_B_TILE_BYTES, with the threshold
    # lowered so that a small B takes it (tiles of 16 fp32 / 8 fp64 columns; ragged last tiles for N = 24
    # and 130)
    from flagsparse_amd import spmm_csr as mod

    monkeypatch.setattr(mod, "SPMM_B_TILE_BYTES", 256 << 10)
    data, idx, ptr, shape = synthetic.csr_banded_random(1 << 12, band_nnz=8, rand_nnz=8,
                                                        dtype=dtype)
    B = synthetic.dense_uniform(shape[1], N, dtype=dtype, seed=3)
    assert mod._auto_tile_cols(B) is not None
    print(f"column tiles N={N} {dtype} tile={mod._auto_tile_cols(B)}", flush=True)
    ref = oracle.spmm_csr(ptr, idx, data, B)
    d, i, p, Bd = data.to(dev), idx.to(dev), ptr.to(dev), B.to(dev)
    _check(fs.flagsparse_spmm_csr_opt(d, i, p, Bd, shape), ref)
    _check(fs.flagsparse_spmm_csr(d, i, p, Bd, shape), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("N", [1, 2, 3, 5, 7, 12, 24, 33, 48, 96, 130])
def test_widths_and_long_rows(dev, dtype, N):
    # short rows, rows around the part threshold (128) and block capacity (2045), split rows
    lengths = [0, 1, 2, 3, 127, 128, 129, 300, 2045, 2046, 5000, 0, 7, 20000, 4, 4]
    data, idx, ptr, shape = _csr_from_lengths(lengths, 30000, N, dtype)
    B = synthetic.dense_uniform(shape[1], N, dtype=dtype, seed=N)
    ref = oracle.spmm_csr(ptr, idx, data, B)
    d, i, p, Bd = data.to(dev), idx.to(dev), ptr.to(dev), B.to(dev)
    _check(fs.flagsparse_spmm_csr_opt(d, i, p, Bd, shape), ref)
    _check(fs.flagsparse_spmm_csr(d, i, p, Bd, shape), ref)


def test_unsorted_duplicate_columns_int64(dev):
    data, idx, ptr = synthetic.build_random_csr(4000, 900, 60000, torch.float32, torch.int64,
                                                "cpu", seed=8)
    B = synthetic.dense_uniform(900, 40, seed=8)
    ref = oracle.spmm_csr(ptr, idx, data, B)
    d, i, p, Bd = data.to(dev), idx.to(dev), ptr.to(dev), B.to(dev)
    _check(fs.flagsparse_spmm_csr_opt(d, i, p, Bd, (4000, 900)), ref)
    _check(fs.flagsparse_spmm_csr(d, i, p.to(torch.int32), Bd, (4000, 900)), ref)


def test_block_n_knob_and_alg1_attributes(dev):
    data, idx, ptr = synthetic.build_random_csr(256, 256, 4096, torch.float32, torch.int32,
                                                "cpu", seed=1)
    B = synthetic.dense_uniform(256, 96, seed=1)
    ref = oracle.spmm_csr(ptr, idx, data, B)
    d, i, p, Bd = data.to(dev), idx.to(dev), ptr.to(dev), B.to(dev)
    for block_n in (None, 8, 32, 64, 100):
        _check(fs.flagsparse_spmm_csr(d, i, p, Bd, (256, 256), block_n=block_n), ref)
    C, ms = fs.flagsparse_spmm_csr(d, i, p, Bd, (256, 256), return_time=True)
    assert isinstance(ms, float) and ms >= 0.0
    _check(C, ref)


def test_prepared_reuse_and_out(dev):
    data, idx, ptr, shape = synthetic.csr_banded_random(4096)
    B = synthetic.dense_uniform(shape[1], 64)
    ref = oracle.spmm_csr(ptr, idx, data, B)
    prep = fs.prepare_spmm_csr_opt(data.to(dev), idx.to(dev), ptr.to(dev), shape)
    Bd = B.to(dev)
    out = torch.empty((shape[0], 64), device=dev)
    for _ in range(3):
        C = fs.flagsparse_spmm_csr_opt(B=Bd, prepared=prep, out=out)
        assert C is out
        _check(C, ref)
    C1 = fs.flagsparse_spmm_csr_opt(B=Bd, prepared=prep)
    C2 = fs.flagsparse_spmm_csr_opt(B=Bd, prepared=prep)
    assert torch.equal(C1, C2)  # deterministic
    C, ms = fs.flagsparse_spmm_csr_opt(B=Bd, prepared=prep, return_time=True)
    assert ms >= 0.0
    with pytest.raises(ValueError):
        fs.flagsparse_spmm_csr_opt(B=Bd, prepared=prep, shape=(5, 5))
    with pytest.raises(ValueError):
        fs.flagsparse_spmm_csr_opt(B=Bd, prepared=prep, out=torch.empty((3, 64), device=dev))
    with pytest.raises(TypeError):
        fs.flagsparse_spmm_csr_opt(B=Bd.double(), prepared=prep)


def test_opt_reference_metadata(dev):
    lengths = [0, 32, 33, 128, 129, 512, 513, 2048, 2049, 3000, 1, 5000]
    data, idx, ptr, shape = _csr_from_lengths(lengths, 9000, 2, torch.float32)
    p = fs.prepare_spmm_csr_opt(data.to(dev), idx.to(dev), ptr.to(dev), shape)
    buckets, long_rows = oracle.spmm_opt_buckets(torch.tensor(lengths).numpy())
    assert [b["rows"].cpu().tolist() for b in p.row_buckets] == \
        [b["rows"].tolist() for b in buckets]
    assert p.long_row_ids.cpu().tolist() == long_rows.tolist()
    rows, starts, ends, rptr = oracle.spmm_opt_split_metadata(ptr.numpy(), long_rows)
    assert p.long_part_rows.cpu().tolist() == rows.tolist()
    assert p.long_part_starts.cpu().tolist() == starts.tolist()
    assert p.long_part_ends.cpu().tolist() == ends.tolist()
    assert p.long_row_part_ptr.cpu().tolist() == rptr.tolist()
    assert p.supports_opt and not p.long_row_fallback_only


def test_reference_api_checks(dev):
    """tests/test_spmm.py:685-807."""
    data = torch.tensor([1.0, 2.0, 3.0], dtype=torch.float32, device=dev)
    indices = torch.tensor([0, 1, 1], dtype=torch.int32, device=dev)
    indptr = torch.tensor([0, 2, 3], dtype=torch.int64, device=dev)
    B = synthetic.dense_uniform(2, 4, seed=5).to(dev)
    long_cols = torch.cat([torch.arange(1536), torch.tensor([7, 129, 511, 1024])]).to(torch.int32)
    long_data = synthetic.uniform_values(5, 1, long_cols.numel(), torch.float32, "cpu")
    long_indptr = torch.tensor([0, 1536, 1540], dtype=torch.int64)
    long_B = synthetic.dense_uniform(2048, 48, seed=6)
    ld, li, lp, lB = (long_data.to(dev), long_cols.to(dev), long_indptr.to(dev), long_B.to(dev))
    f = fs.flagsparse_spmm_csr
    negative = [
        (lambda: f(data, indices, indptr, B, (2,)), ValueError),
        (lambda: f(data, indices, indptr, B[0], (2, 2)), ValueError),
        (lambda: f(data, indices, indptr, B.to(torch.float64), (2, 2)), TypeError),
        (lambda: f(data, indices, indptr, torch.ones((3, 4), device=dev), (2, 2)), ValueError),
        (lambda: f(data, indices, indptr[:-1], B, (2, 2)), ValueError),
        (lambda: f(data, indices, torch.tensor([1, 2, 3], device=dev), B, (2, 2)), ValueError),
        (lambda: f(data, indices, torch.tensor([0, 2, 2], device=dev), B, (2, 2)), ValueError),
        (lambda: f(data, indices, torch.tensor([0, 3, 2], device=dev), B, (2, 2)), ValueError),
        (lambda: f(data, torch.tensor([0, 3, 1], dtype=torch.int32, device=dev), indptr, B,
                   (2, 2)), IndexError),
        (lambda: f(data, indices, indptr, B, (2, 2), block_n=0), ValueError),
        (lambda: f(data, indices, indptr, B, (2, 2), block_nnz=0), ValueError),
        (lambda: f(data, indices, indptr, B, (2, 2), max_segments=0), ValueError),
        (lambda: f(data, indices, indptr, B, (2, 2), out=torch.empty((3, 4), device=dev)),
         ValueError),
        (lambda: f(data, indices, indptr, B, (2, 2), out=torch.empty((2, 4))), ValueError),
        (lambda: f(ld, li, lp, lB, (2, 2048), block_nnz=128, max_segments=4), ValueError),
    ]
    for k, (fn, exc) in enumerate(negative):
        with pytest.raises(exc):
            fn()
    # positive cases
    out = torch.empty((2, 4), dtype=torch.float32, device=dev)
    ref = oracle.spmm_csr(indptr, indices, data, B)
    C = f(data, indices, indptr, B, (2, 2), out=out)
    assert C is out
    _check(C, ref)
    empty = f(torch.tensor([], device=dev), torch.tensor([], dtype=torch.int32, device=dev),
              torch.zeros(3, dtype=torch.int64, device=dev), B, (2, 2))
    assert empty.shape == (2, 4) and torch.count_nonzero(empty) == 0
    C0 = f(data, indices, indptr, torch.empty((2, 0), device=dev), (2, 2))
    assert C0.shape == (2, 0)
    Bt = synthetic.dense_uniform(4, 2, seed=7).to(dev).transpose(0, 1)
    assert not Bt.is_contiguous()
    _check(f(data, indices, indptr, Bt, (2, 2)), oracle.spmm_csr(indptr, indices, data, Bt))
    _check(f(ld, li, lp, lB, (2, 2048)), oracle.spmm_csr(long_indptr, long_cols, long_data, long_B))
    _check(f(ld, li, lp, lB, (2, 2048), block_nnz=128, max_segments=12),
           oracle.spmm_csr(long_indptr, long_cols, long_data, long_B))
    with pytest.raises(NotImplementedError):
        f(data.half(), indices, indptr, B.half(), (2, 2))
