"""Benchmark harness entry points on the GPU: result dictionaries keep the reference's schema
and the flagsparse results verify.

Key sets follow the reference's returned dictionaries:
  benchmark_spmv_case      sparse_operations/benchmarks.py:349-374
  benchmark_spmm_opt_case  sparse_operations/spmm_csr.py:1281-1317
  benchmark_spmm_case      sparse_operations/spmm_csr.py:1469-1533
  comprehensive_spmm_test  sparse_operations/spmm_csr.py:1534-1562 (delegates to the above)
"""

import pytest
import torch

import flagsparse_amd as fs

pytestmark = pytest.mark.gpu

SPMV_KEYS = {
    "parameters": {"n_rows", "n_cols", "nnz", "value_dtype", "index_dtype", "warmup", "iters"},
    "performance": {"triton_ms", "cusparse_ms", "triton_speedup_vs_cusparse"},
    "verification": {"triton_match_reference", "triton_max_error", "cusparse_match_reference",
                     "cusparse_max_error"},
    "backend_status": {"cusparse_unavailable_reason"},
    "samples": {"triton", "reference"},
}

SPMM_OPT_KEYS = {
    "parameters": {"n_rows", "n_cols", "nnz", "n_dense_cols", "value_dtype", "index_dtype"},
    "performance": {"base_ms", "base_first_call_ms", "opt_ms", "opt_first_call_ms", "pt_ms",
                    "cu_ms", "opt_vs_base", "opt_vs_pt", "opt_vs_cu"},
    "verification": {"err_base", "err_opt", "base_ok", "opt_ok", "status"},
    "backend_status": {"long_row_fallback_used", "flagsparse_internal_route"},
    "samples": {"base", "opt", "reference"},
}

SPMM_KEYS = {
    "parameters": {"format", "n_rows", "n_cols", "nnz", "n_dense_cols", "value_dtype",
                   "index_dtype", "warmup", "iters", "block_n", "block_nnz", "max_segments",
                   "required_segments", "alg1_warp_size", "alg1_factor", "auto_max_segments",
                   "run_cusparse"},
    "performance": {"pytorch_ms", "triton_ms", "triton_first_call_ms", "cusparse_ms",
                    "triton_speedup_vs_pytorch", "triton_speedup_vs_cusparse"},
    "verification": {
        "triton_match_reference", "triton_match_pytorch", "triton_max_error",
        "triton_max_abs_error", "triton_max_relative_error", "triton_sum_relative_error",
        "triton_relative_threshold", "triton_strict_allclose_match", "pytorch_match_reference",
        "pytorch_max_error", "pytorch_max_abs_error", "pytorch_max_relative_error",
        "pytorch_sum_relative_error", "pytorch_relative_threshold", "cusparse_match_reference",
        "cusparse_match_pytorch", "cusparse_max_error", "cusparse_max_abs_error",
        "cusparse_max_relative_error", "cusparse_sum_relative_error",
        "cusparse_relative_threshold", "cusparse_strict_allclose_match"},
    "backend_status": {"pytorch_unavailable_reason", "pytorch_sparse_format",
                       "cusparse_unavailable_reason", "flagsparse_internal_route"},
    "samples": {"pytorch", "triton", "reference", "cusparse"},
}


def _check_schema(result, schema):
    assert set(result) == set(schema)
    for section, keys in schema.items():
        assert set(result[section]) == keys, section


@pytest.mark.parametrize("value_dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_benchmark_spmv_case(dev, value_dtype, index_dtype):
    r = fs.benchmark_spmv_case(n_rows=1500, n_cols=1300, nnz=20000, value_dtype=value_dtype,
                               index_dtype=index_dtype, warmup=2, iters=5)
    _check_schema(r, SPMV_KEYS)
    assert r["verification"]["triton_match_reference"] is True
    assert r["performance"]["triton_ms"] > 0
    assert r["samples"]["triton"].shape == (1500,)
    assert r["samples"]["triton"].dtype == value_dtype
    assert r["parameters"]["value_dtype"] == str(value_dtype)


@pytest.mark.parametrize("value_dtype", [torch.float32, torch.float64])
def test_benchmark_spmm_opt_case(dev, value_dtype):
    r = fs.benchmark_spmm_opt_case(n_rows=900, n_cols=700, nnz=12000, n_dense_cols=24,
                                   value_dtype=value_dtype, warmup=2, iters=5)
    _check_schema(r, SPMM_OPT_KEYS)
    v = r["verification"]
    assert v["base_ok"] and v["opt_ok"] and v["status"] == "PASS"
    assert r["samples"]["opt"].shape == (900, 24)


def test_benchmark_spmm_opt_case_rejects_half(dev):
    with pytest.raises(TypeError):
        fs.benchmark_spmm_opt_case(n_rows=16, n_cols=16, nnz=32, value_dtype=torch.float16)


@pytest.mark.parametrize("n_dense_cols", [1, 7, 64, 130])
def test_benchmark_spmm_case(dev, n_dense_cols):
    r = fs.benchmark_spmm_case(n_rows=800, n_cols=600, nnz=9000, n_dense_cols=n_dense_cols,
                               warmup=2, iters=5)
    _check_schema(r, SPMM_KEYS)
    v = r["verification"]
    assert v["triton_match_reference"] and v["triton_strict_allclose_match"]
    assert v["triton_max_relative_error"] <= v["triton_relative_threshold"]
    assert r["samples"]["triton"].shape == (800, n_dense_cols)
    assert r["parameters"]["block_n"] >= 1


def test_comprehensive_spmm_test(dev):
    r = fs.comprehensive_spmm_test(n_rows=512, n_cols=512, nnz=4096, n_dense_cols=32,
                                   dtype=torch.float64, warmup=2, iters=5)
    _check_schema(r, SPMM_KEYS)
    assert r["parameters"]["value_dtype"] == str(torch.float64)
    assert r["verification"]["triton_match_reference"]


def test_measurement_probes(dev):
    # bench.py's probes: the gather probe sums what it gathered (x of ones: one per gather), the
    # row probe likewise (rows of ones: 64 per row), the stream probe counts per workgroup the
    # parity of what it read (a buffer of zeros: 0), over every workgroup's share
    from flagsparse_amd import _abi

    L = _abi.lib()
    s = _abi.raw_stream(dev)
    n = 4096 * 3 + 8
    x = torch.ones(1000, dtype=torch.float32, device=dev)
    idx = torch.randint(0, 1000, (n,), dtype=torch.int32, device=dev)
    out = torch.zeros(int(L.fsp_probe_gather_blocks(n)), dtype=torch.float32, device=dev)
    print("probe gather", flush=True)
    _abi.check(L.fsp_probe_gather(x.data_ptr(), 1000, idx.data_ptr(), n, out.data_ptr(), s), "g")
    torch.cuda.synchronize()
    assert float(out.sum()) == n
    b = torch.ones((300, 64), dtype=torch.float32, device=dev)
    rows = torch.randint(0, 300, (777,), dtype=torch.int32, device=dev)
    out = torch.zeros(int(L.fsp_probe_rows_blocks(777)), dtype=torch.float32, device=dev)
    print("probe rows", flush=True)
    _abi.check(L.fsp_probe_rows(b.data_ptr(), 300, 64, rows.data_ptr(), 777, out.data_ptr(), s),
               "r")
    torch.cuda.synchronize()
    assert float(out.sum()) == 777 * 64
    n16 = 2048 * 5 + 3
    src = torch.zeros(n16 * 16, dtype=torch.uint8, device=dev)
    out = torch.full((int(L.fsp_probe_stream_blocks(n16)),), -1.0, device=dev)
    assert out.numel() == 6
    print("probe stream", flush=True)
    _abi.check(L.fsp_probe_stream(src.data_ptr(), n16, out.data_ptr(), s), "s")
    torch.cuda.synchronize()
    assert torch.equal(out, torch.zeros_like(out))
    assert L.fsp_probe_stream(src.data_ptr() + 4, n16, out.data_ptr(), s) == -1  # misaligned
