"""The drop-in surface, checked without a GPU: exported names, signatures and defaults of the
reference's entry points, and the validation errors that the reference raises before it
touches the device (argument types, shapes, knobs, CPU tensors).

Reference: src/flagsparse/__init__.py:5-63 (names), sparse_operations/spmv_csr.py:379-452,
455, 557-569, 650, 687-700; spmv_coo.py:182-225, 284-297; spmm_csr.py:197-281, 480,
1057-1080, 1129-1160; spmm_coo.py:312-371, 626-694, 848-862, 1146-1158 (signatures and
checks).
"""

import inspect

import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import _abi

# (name, [(parameter, default or inspect._empty)]) as written in the reference sources
REFERENCE_SIGNATURES = {
    "prepare_spmv_csr": [("data", None), ("indices", None), ("indptr", None), ("shape", None),
                         ("block_nnz", 256), ("max_segments", None)],
    "flagsparse_spmv_csr": [("data", None), ("indices", None), ("indptr", None), ("x", None),
                            ("shape", None), ("block_nnz", 256), ("max_segments", None),
                            ("out", None), ("return_time", False), ("use_opt", False),
                            ("prepared", None)],
    "prepare_spmv_coo_tocsr": [("data", None), ("row", None), ("col", None), ("shape", None),
                               ("block_nnz", 256), ("max_segments", None),
                               ("assume_sorted", False)],
    "flagsparse_spmv_coo_tocsr": [("data", None), ("row", None), ("col", None), ("x", None),
                                  ("shape", None), ("block_nnz", 256), ("max_segments", None),
                                  ("out", None), ("return_time", False), ("use_opt", True),
                                  ("prepared", None), ("assume_sorted", False)],
    "prepare_spmv_coo": [("data", None), ("row", None), ("col", None), ("shape", None),
                         ("sort_by_row", True)],
    "flagsparse_spmv_coo": [("data", None), ("row", None), ("col", None), ("x", None),
                            ("shape", None), ("out", None), ("return_time", False),
                            ("prepared", None), ("sort_by_row", True), ("block_size", 256),
                            ("num_warps", 4), ("block_inner", 128)],
    "prepare_spmm_csr_opt": [("data", None), ("indices", None), ("indptr", None),
                             ("shape", None)],
    "flagsparse_spmm_csr": [("data", None), ("indices", None), ("indptr", None), ("B", None),
                            ("shape", None), ("block_n", None), ("block_nnz", None),
                            ("max_segments", None), ("out", None), ("return_time", False)],
    "flagsparse_spmm_csr_opt": [("data", None), ("indices", None), ("indptr", None),
                                ("B", None), ("shape", None), ("prepared", None), ("out", None),
                                ("return_time", False)],
    "benchmark_spmv_case": [("n_rows", 4096), ("n_cols", 4096), ("nnz", 65536),
                            ("value_dtype", torch.float32), ("index_dtype", torch.int32),
                            ("warmup", 20), ("iters", 200), ("block_nnz", 256),
                            ("max_segments", None), ("run_cusparse", True)],
    "benchmark_spmm_case": [("n_rows", 4096), ("n_cols", 4096), ("nnz", 65536),
                            ("n_dense_cols", 32), ("value_dtype", torch.float32),
                            ("index_dtype", torch.int32), ("warmup", 20), ("iters", 200),
                            ("block_n", None), ("block_nnz", None), ("max_segments", None),
                            ("run_cusparse", True)],
    "benchmark_spmm_opt_case": [("n_rows", 4096), ("n_cols", 4096), ("nnz", 65536),
                                ("n_dense_cols", 32), ("value_dtype", torch.float32),
                                ("index_dtype", torch.int32), ("warmup", 20), ("iters", 200),
                                ("run_cusparse", True)],
    "comprehensive_spmm_test": [("n_rows", 4096), ("n_cols", 4096), ("nnz", 65536),
                                ("n_dense_cols", 32), ("dtype", torch.float32),
                                ("index_dtype", torch.int32), ("warmup", 20), ("iters", 200),
                                ("block_n", None), ("block_nnz", None), ("max_segments", None),
                                ("run_cusparse", True)],
    "flagsparse_spmm_coo": [("data", None), ("row", None), ("col", None), ("B", None),
                            ("shape", None), ("block_n", None), ("block_nnz", 256), ("out", None),
                            ("return_time", False)],
    "spmm_coo.benchmark_spmm_coo_case": [
        ("n_rows", 4096), ("n_cols", 4096), ("nnz", 65536), ("n_dense_cols", 32),
        ("value_dtype", torch.float32), ("index_dtype", torch.int32), ("warmup", 20),
        ("iters", 200), ("block_n", None), ("block_nnz", 256), ("run_cusparse", True),
        ("route", "rowrun"), ("compare_routes", False)],
    "prepare_sddmm_csr": [("indices", None), ("indptr", None), ("shape", None), ("k_hint", 64)],
    "flagsparse_sddmm_csr": [("data", None), ("indices", None), ("indptr", None), ("x", None),
                             ("y", None), ("shape", None), ("alpha", 1.0), ("beta", 0.0),
                             ("prepared", None), ("out", None), ("return_time", False),
                             ("return_meta", False), ("allow_fallback", False)],
    "benchmark_sddmm_case": [("n_rows", 1024), ("n_cols", 1024), ("nnz", 16384), ("k_dim", 64),
                             ("value_dtype", torch.float32), ("warmup", 10), ("iters", 30),
                             ("alpha", 1.0), ("beta", 0.0), ("run_cusparse", False)],
    "spmm_coo.comprehensive_spmm_coo_test": [
        ("n_rows", 4096), ("n_cols", 4096), ("nnz", 65536), ("n_dense_cols", 32),
        ("dtype", torch.float32), ("index_dtype", torch.int32), ("warmup", 20), ("iters", 200),
        ("block_n", None), ("block_nnz", 256), ("run_cusparse", True)],
}
# Parameters without a default in the reference (positional-required).
REQUIRED = {
    "prepare_spmv_csr": 4, "prepare_spmv_coo_tocsr": 4, "prepare_spmv_coo": 4,
    "prepare_spmm_csr_opt": 4, "flagsparse_spmm_csr": 5, "flagsparse_spmm_coo": 5,
    "prepare_sddmm_csr": 3,
}


def _resolve(name):
    """``fs.<name>``, or ``flagsparse_amd.<module>.<name>`` for the benchmark cases that the
    reference reaches through its sparse_operations modules."""
    if "." in name:
        import importlib

        mod, attr = name.split(".")
        return getattr(importlib.import_module(f"flagsparse_amd.{mod}"), attr)
    return getattr(fs, name)


@pytest.mark.parametrize("name", sorted(REFERENCE_SIGNATURES))
def test_signature_matches_reference(name):
    params = list(inspect.signature(_resolve(name)).parameters.values())
    want = REFERENCE_SIGNATURES[name]
    # same parameters in the same order; trailing additions must be optional keywords
    assert [p.name for p in params[:len(want)]] == [w[0] for w in want]
    assert all(p.default is not inspect.Parameter.empty for p in params[len(want):])
    n_req = REQUIRED.get(name, 0)
    for i, (p, (_, default)) in enumerate(zip(params, want)):
        if i < n_req:
            assert p.default is inspect.Parameter.empty, p.name
        else:
            assert p.default == default, (p.name, p.default, default)


def test_export_surface():
    reference_all = {
        "flagsparse_gather", "flagsparse_scatter", "pytorch_index_gather",
        "pytorch_index_scatter", "cusparse_spmv_gather", "cusparse_spmv_scatter",
        "benchmark_gather_case", "benchmark_scatter_case", "benchmark_performance",
        "comprehensive_gather_test", "comprehensive_scatter_test", "PreparedCoo",
        "PreparedCsrSpmv", "PreparedCsrSpmmOpt", "prepare_spmv_csr", "prepare_spmm_csr_opt",
        "prepare_spmv_coo", "prepare_spmv_coo_tocsr", "flagsparse_spmv_csr",
        "flagsparse_spmv_coo", "flagsparse_spmv_coo_tocsr", "flagsparse_spmm_csr_opt",
        "flagsparse_spsv_csr", "flagsparse_spsv_coo", "flagsparse_spmm_csr",
        "flagsparse_spmm_coo", "prepare_spgemm_csr", "flagsparse_spgemm_csr", "SpGEMMPrepared",
        "prepare_sddmm_csr", "flagsparse_sddmm_csr", "SDDMMPrepared", "benchmark_spgemm_case",
        "benchmark_sddmm_case", "benchmark_spmm_case", "benchmark_spmm_opt_case",
        "comprehensive_spmm_test", "benchmark_spmv_case", "create_csr_matrix",
        "create_coo_matrix", "create_csc_matrix", "create_bsr_matrix", "create_sell_matrix",
        "create_blocked_ell_matrix", "coo_to_csr", "coo_to_csc", "coo_to_bsr", "coo_to_sell",
        "coo_to_blocked_ell", "CSRMatrix", "COOMatrix", "CSCMatrix", "BSRMatrix", "SELLMatrix",
        "BLOCKEDELLMatrix", "generate_random_sparse_matrix", "read_mtx_file",
    }
    assert set(fs.__all__) == reference_all
    for name in fs.__all__:
        assert getattr(fs, name) is not None
    assert fs.__version__ == "1.0.0"
    assert fs.SUPPORTED_INDEX_DTYPES == (torch.int32, torch.int64)
    assert fs.SUPPORTED_VALUE_DTYPES == (torch.float16, torch.bfloat16, torch.float32,
                                         torch.float64, torch.complex64, torch.complex128)


@pytest.mark.parametrize("name", ["flagsparse_gather", "flagsparse_spgemm_csr", "read_mtx_file",
                                  "CSRMatrix"])
def test_out_of_scope_names_raise(name):
    with pytest.raises(NotImplementedError):
        getattr(fs, name)()


def _csr_cpu():
    data = torch.tensor([1.0, 2.0, 3.0])
    indices = torch.tensor([0, 1, 1], dtype=torch.int32)
    indptr = torch.tensor([0, 2, 3], dtype=torch.int64)
    return data, indices, indptr


def test_spmv_csr_host_validation():
    data, indices, indptr = _csr_cpu()
    with pytest.raises(TypeError):
        fs.prepare_spmv_csr([1.0], indices, indptr, (2, 2))
    with pytest.raises(ValueError):
        fs.prepare_spmv_csr(data[None, :], indices, indptr, (2, 2))
    with pytest.raises(ValueError):
        fs.prepare_spmv_csr(data, indices, indptr[:-1], (2, 2))
    with pytest.raises(ValueError):
        fs.prepare_spmv_csr(data[:2], indices, indptr, (2, 2))
    with pytest.raises(ValueError, match="CUDA"):
        fs.prepare_spmv_csr(data, indices, indptr, (2, 2))
    with pytest.raises(ValueError, match="required"):
        fs.flagsparse_spmv_csr(x=torch.ones(2))


def test_spmv_coo_host_validation():
    data = torch.ones(3)
    row = torch.tensor([0, 1, 1])
    col = torch.tensor([0, 0, 1])
    with pytest.raises(TypeError):
        fs.prepare_spmv_coo(data, row.tolist(), col, (2, 2))
    with pytest.raises(ValueError):
        fs.prepare_spmv_coo(data, row[None], col, (2, 2))
    with pytest.raises(ValueError, match="CUDA"):
        fs.prepare_spmv_coo(data, row, col, (2, 2))
    with pytest.raises(ValueError):
        fs.flagsparse_spmv_coo(data, row, col, None, (2, 2))
    with pytest.raises(ValueError, match="CUDA"):
        fs.prepare_spmv_coo_tocsr(data, row, col, (2, 2))
    with pytest.raises(TypeError):
        fs.flagsparse_spmv_coo_tocsr(data, row, col, None, (2, 2))


def test_spmm_host_validation():
    data, indices, indptr = _csr_cpu()
    B = torch.ones(2, 4)
    # knob checks come first (spmm_csr.py:1075-1080)
    for kw in ({"block_n": 0}, {"block_nnz": 0}, {"max_segments": 0}):
        with pytest.raises(ValueError, match="positive"):
            fs.flagsparse_spmm_csr(data, indices, indptr, B, (2, 2), **kw)
    with pytest.raises(ValueError, match="2D"):
        fs.flagsparse_spmm_csr(data, indices, indptr, B[0], (2, 2))
    with pytest.raises(ValueError, match="2-tuple"):
        fs.flagsparse_spmm_csr(data, indices, indptr, B, (2,))
    with pytest.raises(ValueError, match="CUDA"):
        fs.flagsparse_spmm_csr(data, indices, indptr, B, (2, 2))
    with pytest.raises(ValueError, match="non-negative"):
        fs.prepare_spmm_csr_opt(data, indices, indptr, (-1, 2))
    with pytest.raises(TypeError, match="PreparedCsrSpmmOpt"):
        fs.flagsparse_spmm_csr_opt(B=B, prepared=object())
    with pytest.raises(ValueError, match="required"):
        fs.flagsparse_spmm_csr_opt(B=B)


def test_spmm_coo_host_validation():
    # the reference's API negative cases that fail before the device is touched
    # (tests/test_spmm_coo.py:956-969; spmm_coo.py:312-336, 655-660)
    data = torch.tensor([1.0, 2.0, 3.0])
    row = torch.tensor([0, 0, 1], dtype=torch.int32)
    col = torch.tensor([0, 1, 1], dtype=torch.int32)
    B = torch.ones(2, 4)
    for kw in ({"block_n": 0}, {"block_nnz": 0}):
        with pytest.raises(ValueError, match="positive"):
            fs.flagsparse_spmm_coo(data, row, col, B, (2, 2), **kw)
    with pytest.raises(ValueError, match="2-tuple"):
        fs.flagsparse_spmm_coo(data, row, col, B, (2,))
    with pytest.raises(ValueError, match="2D"):
        fs.flagsparse_spmm_coo(data, row, col, B[0], (2, 2))
    with pytest.raises(ValueError, match="same length"):
        fs.flagsparse_spmm_coo(data, row[:-1], col, B, (2, 2))
    with pytest.raises(ValueError, match="same length"):
        fs.flagsparse_spmm_coo(data, row, col[:-1], B, (2, 2))
    with pytest.raises(ValueError, match="n_cols=2"):
        fs.flagsparse_spmm_coo(data, row, col, torch.ones(3, 4), (2, 2))
    with pytest.raises(ValueError, match="non-negative"):
        fs.flagsparse_spmm_coo(data, row, col, torch.ones(0, 4), (-1, 0))
    with pytest.raises(ValueError, match="CUDA"):
        fs.flagsparse_spmm_coo(data, row, col, B, (2, 2))
    from flagsparse_amd import spmm_coo

    with pytest.raises(ValueError, match="route"):
        spmm_coo._normalize_spmm_coo_route("csr")
    cfg = spmm_coo._resolve_spmm_coo_launch_config(48, 1000)
    assert (cfg["block_n"], cfg["block_nnz"], cfg["required_nnz_tiles"]) == (64, 256, 4)
    assert (cfg["heuristic_warp_size"], cfg["heuristic_factor"]) == (32, 2)


def test_sddmm_host_validation():
    # sddmm_csr.py:46-66 and :361-373: checks that fail before the device is touched
    indices = torch.tensor([0, 1, 1], dtype=torch.int32)
    indptr = torch.tensor([0, 2, 3], dtype=torch.int64)
    with pytest.raises(ValueError, match="2-tuple"):
        fs.prepare_sddmm_csr(indices, indptr, (2,))
    with pytest.raises(ValueError, match="1D"):
        fs.prepare_sddmm_csr(indices[None], indptr, (2, 2))
    with pytest.raises(ValueError, match="non-negative"):
        fs.prepare_sddmm_csr(indices, indptr, (-1, 2))
    with pytest.raises(ValueError, match="n_rows\\+1=4"):
        fs.prepare_sddmm_csr(indices, indptr, (3, 2))
    with pytest.raises(ValueError, match="CUDA"):
        fs.prepare_sddmm_csr(indices, indptr, (2, 2))
    with pytest.raises(ValueError, match="required"):
        fs.flagsparse_sddmm_csr(x=torch.ones(2, 2), y=torch.ones(2, 2))
    with pytest.raises(TypeError, match="SDDMMPrepared"):
        fs.flagsparse_sddmm_csr(x=torch.ones(2, 2), y=torch.ones(2, 2), prepared=object())
    from flagsparse_amd import sddmm_csr

    with pytest.raises(ValueError, match="variant"):
        sddmm_csr._normalize_sddmm_diagnostic_variant("fast")
    assert sddmm_csr._normalize_sddmm_diagnostic_variant(None) == "baseline"
    assert sddmm_csr._normalize_sddmm_diagnostic_variant(" ACC64 ") == "acc64"
    # the reference's launch table (sddmm_csr.py:36-43)
    assert [sddmm_csr._resolve_sddmm_launch_config(k) for k in (1, 32, 33, 64, 65, 128, 129)] == \
        [(32, 2), (32, 2), (64, 4), (64, 4), (64, 4), (64, 4), (128, 8)]


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_abi, "LIB_PATH", str(tmp_path / "libmissing.so"))
    monkeypatch.setattr(_abi, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _abi.lib()
