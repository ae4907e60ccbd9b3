"""COO SpMM C = A @ B on gfx950, behind the reference's entry point.

Public API and error behaviour mirror ``src/flagsparse/sparse_operations/spmm_coo.py``:
``flagsparse_spmm_coo`` (:671-694) with its validation (:312-371) and launch knobs (:374-391,
:626-668), and the benchmark cases ``benchmark_spmm_coo_case`` / ``comprehensive_spmm_coo_test``
(:848-1171).

The reference coalesces duplicate (row, col) entries, sorts them lexicographically and runs one
program per row run (:136-180, :394-461), in float64 for float32 inputs (:11-18).  Here the
entries are brought into row order (no sort when they already are), a row pointer found by
binary search turns them into CSR - a row run is a CSR row, and a row without entries is an empty row that
the kernel writes as 0 - and ``spmm_rowblock_kernel`` computes C with float64 accumulation for
float32 (duplicates are summed by the accumulation itself).  The reference's "atomic" route
(:244-271, :464-523), reachable through the benchmark case, runs ``spmm_coo_atomic_kernel``.
"""

import time

import torch

from . import _abi
from ._index_stats import index_stats
from ._common import (
    SUPPORTED_INDEX_DTYPES,
    _INDEX_LIMIT_INT32,
    _benchmark_cuda_op,
    _require_kernel_dtype,
)
from .spmm_csr import (
    SUPPORTED_SPMM_VALUE_DTYPES,
    _out_ok_direct,
    _run_spmm,
    _select_spmm_alg1_warp_and_factor,
    _spmm_coo_reference_tolerance,
    _spmm_relative_threshold,
    _spmm_validation_metrics,
    _SpmmKernelCsr,
)
from .synthetic import build_random_coo, build_random_dense


def _prepare_spmm_coo_inputs_checked(data, row, col, B, shape):
    """Validation and narrowing of spmm_coo.py:312-371 (same checks, messages and types), plus
    whether the rows are already in order (from the same pass over the indices)."""
    if len(shape) != 2:
        raise ValueError("shape must be a 2-tuple: (n_rows, n_cols)")
    if data.ndim != 1 or row.ndim != 1 or col.ndim != 1:
        raise ValueError("data, row, and col must be 1D tensors")
    if B.ndim != 2:
        raise ValueError("B must be a 2D dense tensor")
    n_rows, n_cols = int(shape[0]), int(shape[1])
    if n_rows < 0 or n_cols < 0:
        raise ValueError("shape dimensions must be non-negative")
    if data.numel() != row.numel() or data.numel() != col.numel():
        raise ValueError("data, row, and col must have the same length (nnz)")
    if B.shape[0] != n_cols:
        raise ValueError(f"B.shape[0] must be n_cols={n_cols}, got {B.shape[0]}")
    if not all(t.is_cuda for t in (data, row, col, B)):
        raise ValueError("data, row, col, and B must be CUDA tensors")
    if not all(t.device == data.device for t in (row, col, B)):
        raise ValueError("data, row, col, and B must be on the same CUDA device")
    if data.dtype not in SUPPORTED_SPMM_VALUE_DTYPES:
        raise TypeError(
            "data dtype must be one of: float16, bfloat16, float32, float64, complex64, "
            "complex128")
    if B.dtype != data.dtype:
        raise TypeError("B dtype must match data dtype")
    if row.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("row dtype must be torch.int32 or torch.int64")
    if col.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("col dtype must be torch.int32 or torch.int64")
    nnz = data.numel()
    if nnz > _INDEX_LIMIT_INT32:
        raise ValueError("nnz exceeds the int32 range supported by the Triton COO kernel")
    row, col = row.contiguous(), col.contiguous()
    row_sorted = True
    if nnz > 0:
        # one pass over both arrays and one host sync for the four bounds and the row order
        min_row, max_row, min_col, max_col, descents = index_stats(row, col)
        row_sorted = descents == 0
        if min_row < 0 or max_row >= n_rows:
            raise IndexError("row indices out of range for n_rows")
        if min_col < 0 or max_col >= n_cols:
            raise IndexError("col indices out of range for n_cols")
        if max_row > _INDEX_LIMIT_INT32:
            raise ValueError("row indices exceed the int32 range supported by the Triton kernel")
        if max_col > _INDEX_LIMIT_INT32:
            raise ValueError(
                "column indices exceed the int32 range supported by the Triton kernel")
    data = data.contiguous()
    kernel_row = row.contiguous().to(torch.int32)
    kernel_col = col.contiguous().to(torch.int32)
    B = B.contiguous()
    return data, kernel_row, kernel_col, B, n_rows, n_cols, int(B.shape[1]), row_sorted


def _prepare_spmm_coo_inputs(data, row, col, B, shape):
    """spmm_coo.py:312-371: the validated, narrowed inputs (data, row int32, col int32, B,
    n_rows, n_cols, n_dense_cols) - the seven values the reference's scripts unpack
    (tests/test_spmm_coo.py:290)."""
    return _prepare_spmm_coo_inputs_checked(data, row, col, B, shape)[:7]


def _resolve_spmm_coo_launch_config(n_dense_cols, nnz, block_n=None, block_nnz=256):
    """spmm_coo.py:374-391: block_n defaults to the ALG1 warp * factor, block_nnz to 256."""
    warp_size, factor = _select_spmm_alg1_warp_and_factor(n_dense_cols)
    if block_n is None:
        block_n = warp_size * factor
    if block_nnz is None:
        block_nnz = 256
    if block_n <= 0 or block_nnz <= 0:
        raise ValueError("block_n and block_nnz must be positive when provided")
    return {
        "block_n": int(block_n),
        "block_nnz": int(block_nnz),
        "required_nnz_tiles": int(-(-nnz // block_nnz) if nnz > 0 else 0),
        "heuristic_warp_size": int(warp_size),
        "heuristic_factor": int(factor),
    }


def _normalize_spmm_coo_route(route):
    route = "rowrun" if route is None else str(route).lower()
    if route not in ("rowrun", "atomic"):
        raise ValueError("route must be 'rowrun' or 'atomic'")
    return route


class _CooRowOrder:
    """Row-ordered COO (int32 rows and columns) plus its CSR view for the SpMM kernel."""

    __slots__ = ("data", "row", "col", "n_rows", "n_cols", "_kc")

    def __init__(self, data, row, col, n_rows, n_cols, row_sorted=None):
        nnz = int(data.numel())
        if row_sorted is None:
            row_sorted = nnz <= 1 or bool((row[1:] >= row[:-1]).all().item())
        if not row_sorted:
            # (row, col) order, stable, so equal keys keep their input order
            key = row.to(torch.int64) * max(1, n_cols) + col.to(torch.int64)
            order = torch.sort(key, stable=True).indices
            data, row, col = data[order], row[order], col[order]
        self.data = data.contiguous()
        self.row = row.contiguous()
        self.col = col.contiguous()
        self.n_rows, self.n_cols = n_rows, n_cols
        self._kc = None

    def kernel_csr(self):
        if self._kc is None:
            # rows are in order, so row r's entries start at the first position whose row
            # is >= r: one binary search per row (no atomics, unlike a bincount)
            bounds = torch.arange(self.n_rows + 1, dtype=self.row.dtype, device=self.row.device)
            indptr = torch.searchsorted(self.row, bounds).to(torch.int64)
            self._kc = _SpmmKernelCsr(self.data, self.col, indptr, window_blocks=1)
        return self._kc


def _spmm_coo_rowrun(coo, B, C, tile_cols=None):
    """C (n_rows x N, contiguous, output dtype) = A @ B through the CSR kernel."""
    _run_spmm(coo.kernel_csr(), B, C, acc_f64=True, tile_cols=tile_cols)
    return C


def _spmm_coo_atomic(data, row, col, n_rows, B, n_dense_cols):
    """The atomic route, entries in any order: an fp64 accumulation buffer (fp32 inputs are
    computed in fp64, as in the reference), rounded to the input dtype at the end."""
    dtype = data.dtype
    C_acc = torch.empty((n_rows, n_dense_cols), dtype=torch.float64, device=B.device)
    L = _abi.lib()
    _abi.check(
        L.fsp_spmm_coo_atomic(_abi.dtype_code(dtype), 1, _abi.ptr(data), _abi.ptr(row),
                              _abi.ptr(col), int(data.numel()), _abi.ptr(B), B.stride(0),
                              n_dense_cols, _abi.ptr(C_acc), n_dense_cols, n_rows,
                              _abi.stream_handle(B.device)),
        "fsp_spmm_coo_atomic")
    return C_acc if dtype == torch.float64 else C_acc.to(dtype)


def _run_spmm_coo_route(data, row, col, B, shape, block_n=None, block_nnz=256, out=None,
                        return_time=False, route="rowrun"):
    """Validation, ordering and launch (spmm_coo.py:572-668)."""
    route = _normalize_spmm_coo_route(route)
    if block_n is not None and block_n <= 0:
        raise ValueError("block_n must be positive when provided")
    if block_nnz is not None and block_nnz <= 0:
        raise ValueError("block_nnz must be positive when provided")
    data, row, col, B, n_rows, n_cols, n_dense_cols, row_sorted = \
        _prepare_spmm_coo_inputs_checked(data, row, col, B, shape)
    launch = _resolve_spmm_coo_launch_config(n_dense_cols, data.numel(), block_n=block_n,
                                             block_nnz=block_nnz)
    dtype = data.dtype
    if out is not None:
        if not out.is_cuda:
            raise ValueError("out must be a CUDA tensor")
        if out.device != data.device:
            raise ValueError("out must be on the same CUDA device as the inputs")
        if out.shape != (n_rows, n_dense_cols) or out.dtype != dtype:
            raise ValueError("out shape/dtype must match result")
    t0 = None
    if return_time:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
    direct = False
    if n_rows == 0 or n_dense_cols == 0 or n_cols == 0 or data.numel() == 0:
        C = torch.zeros((n_rows, n_dense_cols), dtype=dtype, device=data.device)
    else:
        _require_kernel_dtype(dtype, "flagsparse_spmm_coo")
        if route == "atomic":
            C = _spmm_coo_atomic(data, row, col, n_rows, B, n_dense_cols)
        else:
            coo = _CooRowOrder(data, row, col, n_rows, n_cols, row_sorted)
            direct = _out_ok_direct(out, (B, data))
            C = out if direct else torch.empty((n_rows, n_dense_cols), dtype=dtype,
                                               device=data.device)
            tile = launch["block_n"] if block_n is not None else None
            _spmm_coo_rowrun(coo, B, C, tile_cols=tile)
    elapsed_ms = None
    if return_time:
        torch.cuda.synchronize()
        elapsed_ms = (time.perf_counter() - t0) * 1000.0
    if out is not None and not direct:
        out.copy_(C)
        C = out
    if return_time:
        return C, elapsed_ms
    return C


def flagsparse_spmm_coo(data, row, col, B, shape, block_n=None, block_nnz=256, out=None,
                        return_time=False):
    """COO SpMM C = A @ B (spmm_coo.py:671-694): the row-run route.

    Duplicate (row, col) entries are summed; float32 is accumulated in float64 and rounded
    once, as in the reference.  ``block_n`` sets the column tile of a workgroup; ``block_nnz``
    is validated (positive) as in the reference.  Returns C, or (C, elapsed_ms) with
    ``return_time``.
    """
    return _run_spmm_coo_route(data, row, col, B, shape, block_n=block_n, block_nnz=block_nnz,
                               out=out, return_time=return_time, route="rowrun")


# ------------------------------------------------------------------------------------------
# The canonical route of the reference's benchmark scripts (spmm_coo.py:11-18, 54-119,
# 572-624, 697-713, 754-790): duplicates summed, entries in (row, col) order, float32 data and
# B widened to float64 before the product, the result rounded back.  The helpers keep the
# reference's argument lists and return tuples, which tests/test_spmm_coo.py:288-375 unpacks.
# ------------------------------------------------------------------------------------------


def _spmm_coo_compute_dtype(value_dtype):
    """spmm_coo.py:11-18: float32 is computed in float64; fp16/bf16 in float32."""
    if value_dtype in (torch.complex64, torch.complex128):
        return torch.complex128 if value_dtype == torch.complex64 else value_dtype
    if value_dtype in (torch.float16, torch.bfloat16):
        return torch.float32
    if value_dtype == torch.float32:
        return torch.float64
    return value_dtype


def _build_torch_sparse_coo(data, row, col, shape):
    """A coalesced torch COO tensor (int64 indices) for torch.sparse.mm (spmm_coo.py:54-75)."""
    n_rows, n_cols = int(shape[0]), int(shape[1])
    idx = torch.stack([row.to(torch.int64), col.to(torch.int64)]) if data.numel() else \
        torch.empty((2, 0), dtype=torch.int64, device=data.device)
    t = torch.sparse_coo_tensor(idx, data, size=(n_rows, n_cols), device=data.device,
                                dtype=data.dtype)
    return t.coalesce() if data.numel() else t


def _prepare_spmm_coo_canonical_prepared(data, row, col, B, n_rows, n_cols, n_dense_cols):
    """(data, row int64, col int64, B, n_rows, n_cols, n_dense_cols, output dtype, compute
    dtype): the entries in the compute dtype with duplicate (row, col) pairs summed, in
    (row, col) order; B in the compute dtype (spmm_coo.py:78-105)."""
    output_dtype = data.dtype
    compute_dtype = _spmm_coo_compute_dtype(output_dtype)
    d = data if compute_dtype == output_dtype else data.to(compute_dtype)
    Bc = B if compute_dtype == output_dtype else B.to(compute_dtype)
    if d.numel() == 0:
        z = torch.empty(0, dtype=torch.int64, device=data.device)
        return (d.contiguous(), z, z.clone(), Bc, n_rows, n_cols, n_dense_cols, output_dtype,
                compute_dtype)
    coo = _build_torch_sparse_coo(d, row, col, (n_rows, n_cols))  # sums duplicates, sorts
    idx = coo.indices()
    return (coo.values().contiguous(), idx[0].contiguous(), idx[1].contiguous(), Bc, n_rows,
            n_cols, n_dense_cols, output_dtype, compute_dtype)


def _prepare_spmm_coo_canonical_inputs(data, row, col, B, shape):
    """Validation, then the canonical entries (spmm_coo.py:108-118)."""
    return _prepare_spmm_coo_canonical_prepared(*_prepare_spmm_coo_inputs(data, row, col, B,
                                                                           shape))


def _run_spmm_coo_canonical_route(canonical_data, canonical_row, canonical_col, canonical_B,
                                  n_rows, n_dense_cols, output_dtype, block_n=None,
                                  block_nnz=256, out=None, return_time=False, route="rowrun"):
    """The product over canonical entries, in their dtype, rounded to ``output_dtype``, with
    the reference's out checks and host timing (spmm_coo.py:572-624)."""
    route = _normalize_spmm_coo_route(route)
    n_cols = int(canonical_B.shape[0])
    if out is not None:
        if not out.is_cuda:
            raise ValueError("out must be a CUDA tensor")
        if out.device != canonical_data.device:
            raise ValueError("out must be on the same CUDA device as the inputs")
        if out.shape != (n_rows, n_dense_cols) or out.dtype != output_dtype:
            raise ValueError("out shape/dtype must match result")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    C = _run_spmm_coo_route(canonical_data, canonical_row, canonical_col, canonical_B,
                            (n_rows, n_cols), block_n=block_n, block_nnz=block_nnz, route=route)
    if C.dtype != output_dtype:
        C = C.to(output_dtype)
    torch.cuda.synchronize()
    elapsed_ms = (time.perf_counter() - t0) * 1000.0
    if out is not None:
        out.copy_(C)
        C = out
    return (C, elapsed_ms) if return_time else C


def _build_spmm_coo_pytorch_reference_from_canonical(canonical_data, canonical_row,
                                                     canonical_col, canonical_B, shape,
                                                     output_dtype):
    """torch.sparse.mm over the canonical entries, rounded to ``output_dtype``
    (spmm_coo.py:697-713) - the scripts' correctness reference."""
    coo = _build_torch_sparse_coo(canonical_data, canonical_row, canonical_col, shape)
    expected = torch.sparse.mm(coo, canonical_B)
    return expected if expected.dtype == output_dtype else expected.to(output_dtype)


def _benchmark_spmm_coo_canonical_route(canonical_data, canonical_row, canonical_col,
                                        canonical_B, n_rows, n_dense_cols, output_dtype, warmup,
                                        iters, block_n, block_nnz, route):
    """(values, steady ms, first-call ms) of the canonical route (spmm_coo.py:754-790)."""
    route = _normalize_spmm_coo_route(route)

    def op():
        return _run_spmm_coo_canonical_route(canonical_data, canonical_row, canonical_col,
                                             canonical_B, n_rows, n_dense_cols, output_dtype,
                                             block_n=block_n, block_nnz=block_nnz, route=route)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    op()
    torch.cuda.synchronize()
    first_call_ms = (time.perf_counter() - t0) * 1000.0
    values, steady_ms = _benchmark_cuda_op(op, warmup=warmup, iters=iters)
    return values, steady_ms, first_call_ms


# ------------------------------------------------------------------------------------------
# Benchmark cases (spmm_coo.py:697-1171): same result dictionaries; the "triton_*" keys
# name the flagsparse kernel as in the reference, cuSPARSE/CuPy is reported unavailable.
# ------------------------------------------------------------------------------------------


def _torch_coo_reference(data, row, col, B, shape):
    """fp64 (for float32) torch.sparse.mm over the coalesced entries, rounded to the input
    dtype (spmm_coo.py:697-713 with the compute dtype of :11-18)."""
    ref_dtype = torch.float64 if data.dtype == torch.float32 else data.dtype
    coo = torch.sparse_coo_tensor(torch.stack([row.to(torch.int64), col.to(torch.int64)]),
                                  data.to(ref_dtype), size=shape, device=data.device).coalesce()
    return torch.sparse.mm(coo, B.to(ref_dtype)).to(data.dtype)


def _spmm_coo_pairwise_summary(candidate, reference, value_dtype):
    """spmm_coo.py:830-845."""
    metrics = _spmm_validation_metrics(candidate, reference)
    atol, rtol = _spmm_coo_reference_tolerance(value_dtype)
    if candidate.numel() == 0:
        error_ratio = 0.0
    else:
        diff = torch.abs(candidate - reference)
        error_ratio = float(torch.max(diff / (atol + rtol * torch.abs(reference))).item())
    return {
        "match": torch.allclose(candidate, reference, atol=atol, rtol=rtol),
        "error_ratio": error_ratio,
        "max_abs_error": metrics["max_abs_error"],
        "max_relative_error": metrics["max_relative_error"],
        "sum_relative_error": metrics["sum_relative_error"],
    }


def _timed_route(data, row, col, B, shape, warmup, iters, block_n, block_nnz, route):
    op = lambda: _run_spmm_coo_route(data, row, col, B, shape, block_n=block_n,  # noqa: E731
                                     block_nnz=block_nnz, route=route)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    op()
    torch.cuda.synchronize()
    first_call_ms = (time.perf_counter() - t0) * 1000.0
    values, ms = _benchmark_cuda_op(op, warmup=warmup, iters=iters)
    return values, ms, first_call_ms


def benchmark_spmm_coo_case(n_rows=4096, n_cols=4096, nnz=65536, n_dense_cols=32,
                            value_dtype=torch.float32, index_dtype=torch.int32, warmup=20,
                            iters=200, block_n=None, block_nnz=256, run_cusparse=True,
                            route="rowrun", compare_routes=False, seed=0):
    """flagsparse COO SpMM vs torch.sparse.mm (spmm_coo.py:848-1143); CuPy/cuSPARSE is not
    part of this build and is reported unavailable."""
    selected_route = _normalize_spmm_coo_route(route)
    device = torch.device("cuda")
    data, row, col = build_random_coo(n_rows, n_cols, nnz, value_dtype, index_dtype, device,
                                      seed=seed)
    B = build_random_dense((n_cols, n_dense_cols), value_dtype, device, seed=seed)
    shape = (n_rows, n_cols)
    launch = _resolve_spmm_coo_launch_config(n_dense_cols, nnz, block_n=block_n,
                                             block_nnz=block_nnz)
    n_row_runs = int(torch.unique(row).numel()) if nnz > 0 else 0
    expected = _torch_coo_reference(data, row, col, B, shape)
    triton_C, triton_ms, triton_first_ms = _timed_route(
        data, row, col, B, shape, warmup, iters, block_n, block_nnz, selected_route)
    triton_summary = _spmm_coo_pairwise_summary(triton_C, expected, value_dtype)
    triton_match = triton_summary["match"]

    pytorch_values, pytorch_ms, pytorch_reason = expected, None, None
    try:
        native = torch.sparse_coo_tensor(torch.stack([row.to(torch.int64), col.to(torch.int64)]),
                                         data, size=shape, device=device).coalesce()
        pytorch_values, pytorch_ms = _benchmark_cuda_op(lambda: torch.sparse.mm(native, B),
                                                        warmup=warmup, iters=iters)
    except Exception as exc:  # torch.sparse may not support the dtype on this device
        pytorch_reason = str(exc)

    route_results = parity = route_samples = None
    if compare_routes:
        outputs = {selected_route: triton_C}
        route_results = {selected_route: {
            "route": selected_route, "ms": triton_ms, "first_call_ms": triton_first_ms,
            "match_reference": triton_summary["match"],
            "error_ratio": triton_summary["error_ratio"],
            "max_abs_error": triton_summary["max_abs_error"],
            "max_relative_error": triton_summary["max_relative_error"],
            "match_cusparse": None, "error": None}}
        for extra in ("rowrun", "atomic"):
            if extra in outputs:
                continue
            try:
                vals, ms, first_ms = _timed_route(data, row, col, B, shape, warmup, iters,
                                                  block_n, block_nnz, extra)
                summary = _spmm_coo_pairwise_summary(vals, expected, value_dtype)
                outputs[extra] = vals
                route_results[extra] = {
                    "route": extra, "ms": ms, "first_call_ms": first_ms,
                    "match_reference": summary["match"], "error_ratio": summary["error_ratio"],
                    "max_abs_error": summary["max_abs_error"],
                    "max_relative_error": summary["max_relative_error"],
                    "match_cusparse": None, "error": None}
            except Exception as exc:
                route_results[extra] = {
                    "route": extra, "ms": None, "first_call_ms": None, "match_reference": False,
                    "error_ratio": None, "max_abs_error": None, "max_relative_error": None,
                    "match_cusparse": None, "error": str(exc)}
        if "rowrun" in outputs and "atomic" in outputs:
            rr = _spmm_coo_pairwise_summary(outputs["rowrun"], outputs["atomic"], value_dtype)
        else:
            rr = {"match": None, "error_ratio": None, "max_abs_error": None,
                  "max_relative_error": None, "sum_relative_error": None}
        parity = {"rowrun_vs_atomic": rr}
        route_samples = outputs

    threshold = _spmm_relative_threshold(value_dtype)
    return {
        "parameters": {
            "format": "coo", "internal_format": f"native-{selected_route}",
            "route": selected_route, "compare_routes": bool(compare_routes), "n_rows": n_rows,
            "n_cols": n_cols, "nnz": nnz, "n_dense_cols": n_dense_cols,
            "value_dtype": str(value_dtype), "index_dtype": str(index_dtype), "warmup": warmup,
            "iters": iters, "block_n": launch["block_n"], "block_nnz": launch["block_nnz"],
            "required_nnz_tiles": launch["required_nnz_tiles"],
            "heuristic_warp_size": launch["heuristic_warp_size"],
            "heuristic_factor": launch["heuristic_factor"], "n_row_runs": n_row_runs,
            "run_cusparse": run_cusparse,
        },
        "performance": {
            "pytorch_ms": pytorch_ms, "triton_ms": triton_ms,
            "triton_first_call_ms": triton_first_ms, "cusparse_ms": None,
            "triton_speedup_vs_pytorch": (pytorch_ms / triton_ms
                                          if pytorch_ms is not None and triton_ms > 0 else None),
            "triton_speedup_vs_cusparse": None,
        },
        "verification": {
            "triton_match_reference": triton_match, "triton_match_pytorch": triton_match,
            "triton_max_error": triton_summary["max_abs_error"],
            "triton_max_abs_error": triton_summary["max_abs_error"],
            "triton_max_relative_error": triton_summary["max_relative_error"],
            "triton_sum_relative_error": triton_summary["sum_relative_error"],
            "triton_relative_threshold": threshold, "triton_strict_allclose_match": triton_match,
            "pytorch_match_reference": True, "pytorch_max_error": 0.0,
            "pytorch_max_abs_error": 0.0, "pytorch_max_relative_error": 0.0,
            "pytorch_sum_relative_error": 0.0, "pytorch_relative_threshold": threshold,
            "cusparse_match_reference": None, "cusparse_match_pytorch": None,
            "cusparse_max_error": None, "cusparse_max_abs_error": None,
            "cusparse_max_relative_error": None, "cusparse_sum_relative_error": None,
            "cusparse_relative_threshold": threshold, "cusparse_strict_allclose_match": None,
        },
        "backend_status": {
            "pytorch_unavailable_reason": pytorch_reason, "pytorch_sparse_format": "COO",
            "cusparse_unavailable_reason": (
                "CuPy/cuSPARSE is not part of the MI355X build" if run_cusparse else None),
            "flagsparse_internal_route": f"coo-native-{selected_route}",
        },
        "samples": {"pytorch": pytorch_values, "triton": triton_C, "reference": expected,
                    "cusparse": None},
        "route_results": route_results,
        "parity": parity,
        "route_samples": route_samples,
    }


def comprehensive_spmm_coo_test(n_rows=4096, n_cols=4096, nnz=65536, n_dense_cols=32,
                                dtype=torch.float32, index_dtype=torch.int32, warmup=20,
                                iters=200, block_n=None, block_nnz=256, run_cusparse=True):
    """Full COO SpMM benchmark entry for one configuration (spmm_coo.py:1146-1171)."""
    return benchmark_spmm_coo_case(n_rows=n_rows, n_cols=n_cols, nnz=nnz,
                                   n_dense_cols=n_dense_cols, value_dtype=dtype,
                                   index_dtype=index_dtype, warmup=warmup, iters=iters,
                                   block_n=block_n, block_nnz=block_nnz,
                                   run_cusparse=run_cusparse)
