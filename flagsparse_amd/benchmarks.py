"""SpMV benchmark case (mirrors benchmark_spmv_case, sparse_operations/benchmarks.py:230-374).

The result dictionary keeps the reference's keys; the "triton_*" entries describe the
flagsparse kernel and the cuSPARSE/CuPy baseline is reported unavailable (it is not part of
the MI355X build).  The expected values come from torch.sparse on the same device, as in the
reference when CuPy is absent (benchmarks.py:284-301).
"""

import torch

from ._common import _benchmark_cuda_op, _tolerance_for_dtype
from .spmv_csr import flagsparse_spmv_csr, prepare_spmv_csr
from .synthetic import build_random_csr, build_random_dense


def benchmark_spmv_case(n_rows=4096, n_cols=4096, nnz=65536, value_dtype=torch.float32,
                        index_dtype=torch.int32, warmup=20, iters=200, block_nnz=256,
                        max_segments=None, run_cusparse=True, seed=0):
    """Time flagsparse CSR SpMV on a random matrix and check it against torch.sparse."""
    device = torch.device("cuda")
    data, indices, indptr = build_random_csr(n_rows, n_cols, nnz, value_dtype, index_dtype,
                                             device, seed=seed)
    x = build_random_dense(n_cols, value_dtype, device, seed=seed)
    shape = (n_rows, n_cols)
    prepared = prepare_spmv_csr(data, indices, indptr, shape, block_nnz=block_nnz,
                                max_segments=max_segments)
    op = lambda: flagsparse_spmv_csr(x=x, prepared=prepared, return_time=False)  # noqa: E731
    triton_y, triton_ms = _benchmark_cuda_op(op, warmup=warmup, iters=iters)
    row_indices = torch.repeat_interleave(
        torch.arange(n_rows, device=device, dtype=torch.int64), indptr[1:] - indptr[:-1])
    coo = torch.sparse_coo_tensor(torch.stack([row_indices, indices.to(torch.int64)]), data,
                                  shape, device=device).coalesce()
    expected = torch.sparse.mm(coo, x.unsqueeze(1)).squeeze(1)
    atol, rtol = _tolerance_for_dtype(value_dtype)
    triton_match = torch.allclose(triton_y, expected, atol=atol, rtol=rtol)
    triton_max_error = (float(torch.max(torch.abs(triton_y - expected)).item())
                        if n_rows > 0 else 0.0)
    return {
        "parameters": {"n_rows": n_rows, "n_cols": n_cols, "nnz": nnz,
                       "value_dtype": str(value_dtype), "index_dtype": str(index_dtype),
                       "warmup": warmup, "iters": iters},
        "performance": {"triton_ms": triton_ms, "cusparse_ms": None,
                        "triton_speedup_vs_cusparse": None},
        "verification": {"triton_match_reference": triton_match,
                         "triton_max_error": triton_max_error,
                         "cusparse_match_reference": None, "cusparse_max_error": None},
        "backend_status": {"cusparse_unavailable_reason": (
            "CuPy/cuSPARSE is not part of the MI355X build" if run_cusparse else None)},
        "samples": {"triton": triton_y, "reference": expected},
    }
