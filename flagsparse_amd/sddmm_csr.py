"""CSR SDDMM on gfx950, behind the reference's entry points.

Public API and error behaviour mirror ``src/flagsparse/sparse_operations/sddmm_csr.py``:
``SDDMMPrepared`` (:9-33), ``prepare_sddmm_csr`` (:93-104) with its pattern validation
(:46-79), ``flagsparse_sddmm_csr`` (:350-422) with the dense-input checks (:205-240), the
diagnostic variants of ``_run_sddmm_prepared`` (:243-347) and ``benchmark_sddmm_case``
(:472-572).

out[p] = alpha * dot(x[row(p)], y[col(p)]) + beta * data[p] for every stored entry p, computed
by flagsparse_amd/csrc/sddmm.hip in the input precision (float64 for the "acc64" variants) with
a fixed reduction order: ``sddmm_rowblock_kernel`` over a row-block plan built on the device
(one lane group per row, the row of x held in registers) when K <= 4 * 64 lanes * vector
width, ``sddmm_flat_kernel`` (one lane group per entry) otherwise.
"""

import time

import torch

from . import _abi, _common
from ._common import (  # noqa: F401  (cp and the converters: the reference scripts' names)
    _aligned,
    _benchmark_cuda_op,
    _cupy_from_torch,
    _tolerance_for_dtype,
    _torch_from_cupy,
    cp,
)
from ._plan import build_row_block_plan_device
from .synthetic import build_random_csr, build_random_dense

SUPPORTED_SDDMM_VALUE_DTYPES = (torch.float32, torch.float64)
SUPPORTED_SDDMM_DIAGNOSTIC_VARIANTS = ("baseline", "acc64", "acc64_out64", "altreduce")

_BLOCK_THREADS = 256
# Rows longer than this are cut into chunks that all lane groups of a workgroup share.
_SDDMM_ROW_SPLIT_THRESHOLD = 128
# The row-block plan is built in windows of this many blocks' rows (windows of one block's
# rows add a tiny block whenever the entry cap ends a block before the row cap does; wider
# windows plan more slowly), as for SpMM.
SDDMM_PLAN_WINDOW_BLOCKS = 4


class SDDMMPrepared:
    """Prepared CSR pattern for SDDMM (sddmm_csr.py:9-33): int32 columns, int64 row pointers,
    one int32 row id per entry, and the reference's launch attributes (block_k, num_warps)."""

    __slots__ = ("indices", "indptr", "shape", "n_rows", "n_cols", "nnz", "row_ids", "block_k",
                 "num_warps", "_plans", "_kernel_ptr", "_window_blocks")

    def __init__(self, indices, indptr, shape, row_ids, block_k, num_warps):
        self.indices = indices
        self.indptr = indptr
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows = self.shape[0]
        self.n_cols = self.shape[1]
        self.nnz = int(indices.numel())
        self.row_ids = row_ids
        self.block_k = int(block_k)
        self.num_warps = int(num_warps)
        self._plans = {}
        self._kernel_ptr = None
        self._window_blocks = SDDMM_PLAN_WINDOW_BLOCKS  # 1 for a prepared object of one call

    def _row_plan(self, lanes):
        """Row-block plan for ``lanes`` lanes per entry (built on the device, cached)."""
        plan = self._plans.get(lanes)
        if plan is None:
            if self._kernel_ptr is None:
                self._kernel_ptr = (self.indptr.to(torch.int32)
                                    if self.nnz <= _common.ROWPTR32_MAX_NNZ
                                    else self.indptr.to(torch.int64))
            cap = _abi.caps()["spmm_block_nnz"]
            rows_cap = _BLOCK_THREADS // lanes
            plan = build_row_block_plan_device(self._kernel_ptr, cap, rows_cap,
                                               min(_SDDMM_ROW_SPLIT_THRESHOLD, cap), cap,
                                               window_rows=self._window_blocks * rows_cap)
            self._plans[lanes] = plan
        return plan



def _resolve_sddmm_launch_config(k):
    """(block_k, num_warps) of sddmm_csr.py:36-43, kept as attributes and metadata."""
    if k <= 32:
        return 32, 2
    if k <= 64:
        return 64, 4
    if k <= 128:
        return 64, 4
    return 128, 8


def _prepare_sddmm_csr_pattern(indices, indptr, shape):
    """Validation of sddmm_csr.py:46-79 (same checks, order, messages and types)."""
    if len(shape) != 2:
        raise ValueError("shape must be a 2-tuple")
    if indices.ndim != 1 or indptr.ndim != 1:
        raise ValueError("indices and indptr must be 1D tensors")
    n_rows, n_cols = int(shape[0]), int(shape[1])
    if n_rows < 0 or n_cols < 0:
        raise ValueError("shape dimensions must be non-negative")
    if indptr.numel() != n_rows + 1:
        raise ValueError(f"indptr length must be n_rows+1={n_rows + 1}, got {indptr.numel()}")
    if not indices.is_cuda or not indptr.is_cuda:
        raise ValueError("indices and indptr must be CUDA tensors")
    if indices.dtype != torch.int32:
        raise TypeError("indices dtype must be torch.int32")
    if indptr.dtype not in (torch.int32, torch.int64):
        raise TypeError("indptr dtype must be torch.int32 or torch.int64")
    indptr64 = indptr.to(torch.int64).contiguous()
    indices = _aligned(indices.contiguous())  # 16-byte loads of the columns
    nnz = int(indices.numel())
    # one host sync for the structural checks: first, last, monotone
    first, last, bad = torch.stack([
        indptr64[0], indptr64[-1],
        (indptr64[1:] < indptr64[:-1]).any().to(torch.int64) if n_rows > 0
        else torch.zeros((), dtype=torch.int64, device=indptr64.device)]).tolist()
    if first != 0:
        raise ValueError("indptr[0] must be 0")
    if last != nnz:
        raise ValueError(f"indptr[-1] must equal nnz={nnz}")
    if bad:
        raise ValueError("indptr must be nondecreasing")
    if nnz > 0:
        min_col, max_col = torch.stack([indices.min(), indices.max()]).tolist()
        if min_col < 0 or max_col >= n_cols:
            raise IndexError("indices out of range for shape[1]")
    return indices, indptr64, (n_rows, n_cols)


def _build_row_ids(indptr):
    n_rows = int(indptr.numel()) - 1
    if n_rows <= 0:
        return torch.empty(0, dtype=torch.int32, device=indptr.device)
    return torch.repeat_interleave(torch.arange(n_rows, dtype=torch.int32, device=indptr.device),
                                   indptr[1:] - indptr[:-1])


def prepare_sddmm_csr(indices, indptr, shape, k_hint=64):
    """Validate a CSR pattern and build its per-entry row ids (sddmm_csr.py:93-104)."""
    indices, indptr, shape = _prepare_sddmm_csr_pattern(indices, indptr, shape)
    row_ids = _build_row_ids(indptr)
    block_k, num_warps = _resolve_sddmm_launch_config(int(k_hint))
    return SDDMMPrepared(indices=indices, indptr=indptr, shape=shape, row_ids=row_ids,
                         block_k=block_k, num_warps=num_warps)


def _validate_sddmm_dense_inputs(data, prepared, x, y):
    """sddmm_csr.py:205-226."""
    if x.ndim != 2 or y.ndim != 2:
        raise ValueError("x and y must be 2D dense tensors")
    if not x.is_cuda or not y.is_cuda:
        raise ValueError("x and y must be CUDA tensors")
    if x.device != y.device or x.device != prepared.indices.device:
        raise ValueError("x, y, and sparse pattern must be on the same CUDA device")
    if x.dtype not in SUPPORTED_SDDMM_VALUE_DTYPES:
        raise TypeError("x dtype must be torch.float32 or torch.float64")
    if y.dtype != x.dtype:
        raise TypeError("y dtype must match x dtype")
    if data is not None and data.dtype != x.dtype:
        raise TypeError("data dtype must match x/y dtype")
    if x.shape[0] != prepared.n_rows:
        raise ValueError(f"x.shape[0] must be n_rows={prepared.n_rows}, got {x.shape[0]}")
    if y.shape[0] != prepared.n_cols:
        raise ValueError(f"y.shape[0] must be n_cols={prepared.n_cols}, got {y.shape[0]}")
    if x.shape[1] != y.shape[1]:
        raise ValueError("x and y must have the same K dimension")
    if data is not None and data.numel() != prepared.nnz:
        raise ValueError("data length must equal nnz of sparse pattern")
    return int(x.shape[1])


def _prepare_validated_sddmm_out(prepared, x, out, out_dtype=None):
    """sddmm_csr.py:229-240."""
    nnz = prepared.nnz
    target_dtype = x.dtype if out_dtype is None else out_dtype
    if out is None:
        return torch.empty(nnz, dtype=target_dtype, device=x.device)
    if out.ndim != 1 or out.numel() != nnz:
        raise ValueError("out must be a 1D tensor with length nnz")
    if not out.is_cuda or out.device != x.device:
        raise ValueError("out must be a CUDA tensor on the same device as x")
    if out.dtype != target_dtype:
        raise TypeError("out dtype must match the requested output dtype")
    return out


def _normalize_sddmm_diagnostic_variant(variant):
    if variant is None:
        return "baseline"
    variant = str(variant).strip().lower()
    if variant not in SUPPORTED_SDDMM_DIAGNOSTIC_VARIANTS:
        supported = ", ".join(SUPPORTED_SDDMM_DIAGNOSTIC_VARIANTS)
        raise ValueError(
            f"Unsupported SDDMM diagnostic variant {variant!r}; expected one of: {supported}")
    return variant


def _resolve_sddmm_diagnostic_out_dtype(variant, value_dtype):
    return torch.float64 if _normalize_sddmm_diagnostic_variant(variant) == "acc64_out64" \
        else value_dtype


def _sddmm_lane_shape(K, x, y):
    """(lanes per entry G, elements per lane vec): 16-byte loads when K, the row strides and
    the base pointers allow it; G covers K in one step up to 64 lanes."""
    vmax = 4 if x.dtype == torch.float32 else 2
    vec = 1
    for v in (vmax, 2):
        if (K % v == 0 and x.stride(0) % v == 0 and y.stride(0) % v == 0
                and x.data_ptr() % 16 == 0 and y.data_ptr() % 16 == 0):
            vec = v
            break
    steps = -(-K // vec)
    lanes = 1
    while lanes < steps and lanes < 64:
        lanes <<= 1
    # At most 16 lanes while the row-block schedule still holds K (K <= 4 * lanes * vec): wider
    # groups spend more on the cross-lane sum than their loads gain.  Measured on MI355X, cfg5's
    # pattern: fp32 K=128 1747 -> 1625 us (32 -> 16 lanes), fp64 K=64 2259 -> 1932 us; fp32
    # K=64 stays at 16 (8 lanes: 846 vs 807 us).
    while lanes > 16 and K <= 4 * (lanes // 2) * vec:
        lanes >>= 1
    return lanes, vec


def _launch_sddmm(prepared, x, y, data, alpha, beta, out, acc_f64):
    """fsp_sddmm_csr with the row-block schedule when K fits four steps of the lane group
    (x rows kept in registers), else one lane group per entry."""
    K = int(x.shape[1])
    lanes, vec = _sddmm_lane_shape(K, x, y)
    L = _abi.lib()
    cols = prepared.indices
    if K <= 4 * lanes * vec and cols.data_ptr() % 16 == 0:
        plan = prepared._row_plan(lanes)
        rp = prepared._kernel_ptr
        sched = (_abi.ptr(rp), 32 if rp.dtype == torch.int32 else 64, _abi.ptr(plan.desc),
                 _abi.ptr(plan.ranges), plan.n_desc)
    else:
        sched = (None, 32, None, None, 0)
    rowptr, bits, desc, ranges, n_desc = sched
    _abi.check(
        L.fsp_sddmm_csr(_abi.dtype_code(x.dtype), int(acc_f64),
                        int(out.dtype == torch.float64 and x.dtype == torch.float32),
                        _abi.ptr(cols), _abi.ptr(prepared.row_ids), rowptr, bits, prepared.nnz,
                        _abi.ptr(x), x.stride(0), _abi.ptr(y), y.stride(0), K, _abi.ptr(data),
                        float(alpha), float(beta), _abi.ptr(out), desc, ranges, n_desc, lanes,
                        vec, _abi.stream_handle(x.device)),
        "fsp_sddmm_csr")


def _sddmm_reference(indices, indptr, x, y, data, alpha, beta):
    """torch sampled dot (sddmm_csr.py:425-437), used by the benchmark case and the fallback."""
    n_rows = int(indptr.numel()) - 1
    row_ids = torch.repeat_interleave(
        torch.arange(n_rows, dtype=torch.int64, device=indices.device), indptr[1:] - indptr[:-1])
    if row_ids.numel() == 0:
        return torch.empty(0, dtype=x.dtype, device=x.device)
    vals = torch.sum(x[row_ids] * y[indices.to(torch.int64)], dim=1)
    vals = alpha * vals
    if data is not None:
        vals = vals + beta * data
    return vals


def _run_sddmm_prepared(prepared, x, y, data, alpha, beta, out, allow_fallback=False,
                        variant="baseline", out_dtype=None):
    """Launch with a diagnostic variant (sddmm_csr.py:271-347).  "acc64" accumulates float32 in
    float64, "acc64_out64" also returns float64, "altreduce" (the reference's per-k loop) is
    the baseline here: this kernel has one reduction order.  With ``allow_fallback`` a failing
    kernel call (not a missing library) is replaced by the torch sampled dot, as in the
    reference, and reported in the metadata."""
    nnz = prepared.nnz
    variant = _normalize_sddmm_diagnostic_variant(variant)
    target = (_resolve_sddmm_diagnostic_out_dtype(variant, x.dtype) if out_dtype is None
              else out_dtype)
    out = _prepare_validated_sddmm_out(prepared, x, out, out_dtype=target)
    acc_f64 = variant in ("acc64", "acc64_out64") or x.dtype == torch.float64
    block_k, num_warps = _resolve_sddmm_launch_config(int(x.shape[1]))
    meta = {"block_k": block_k if nnz else prepared.block_k,
            "num_warps": num_warps if nnz else prepared.num_warps, "fallback_used": False,
            "variant": variant, "acc_dtype": "float64" if acc_f64 else "float32",
            "out_dtype": str(out.dtype).replace("torch.", "")}
    if nnz == 0:
        return out, meta
    if out.dtype == torch.float64 and x.dtype == torch.float32 and not acc_f64:
        acc_f64 = True  # a float64 result of float32 inputs is accumulated in float64
    try:
        _launch_sddmm(prepared, x, y, data, alpha, beta, out, acc_f64)
    except _abi.HipLibraryError:
        if not allow_fallback:
            raise
        out.copy_(_sddmm_reference(prepared.indices, prepared.indptr, x, y, data, alpha,
                                   beta).to(out.dtype))
        meta["fallback_used"] = True
    return out, meta


def flagsparse_sddmm_csr(data=None, indices=None, indptr=None, x=None, y=None, shape=None,
                         alpha=1.0, beta=0.0, prepared=None, out=None, return_time=False,
                         return_meta=False, allow_fallback=False):
    """CSR SDDMM: out[p] = alpha * dot(x[row(p)], y[col(p)]) + beta * data[p]
    (sddmm_csr.py:350-422; returns out, optionally with the elapsed ms and/or metadata)."""
    prepare_ms = 0.0
    if prepared is None:
        if any(v is None for v in (indices, indptr, shape)):
            raise ValueError(
                "indices, indptr, and shape are required when prepared is not provided")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        k_hint = int(x.shape[1]) if (x is not None and x.ndim == 2) else 64
        prepared = prepare_sddmm_csr(indices, indptr, shape, k_hint=k_hint)
        prepared._window_blocks = 1  # planned for this call only: the fastest plan to build
        torch.cuda.synchronize()
        prepare_ms = (time.perf_counter() - t0) * 1000.0
    elif not isinstance(prepared, SDDMMPrepared):
        raise TypeError("prepared must be a SDDMMPrepared instance")
    if x is None or y is None:
        raise ValueError("x and y are required")
    if data is None and float(beta) != 0.0:
        raise ValueError("data is required when beta is non-zero")
    k_dim = _validate_sddmm_dense_inputs(data, prepared, x, y)
    if k_dim == 0:
        out = _prepare_validated_sddmm_out(prepared, x, out)
        if beta == 0.0 or data is None:
            out.zero_()
        else:
            out.copy_(data * beta)
        meta = {"prepare_ms": prepare_ms, "block_k": prepared.block_k,
                "num_warps": prepared.num_warps, "fallback_used": False}
        if return_time and return_meta:
            return out, 0.0, meta
        if return_time:
            return out, 0.0
        if return_meta:
            return out, meta
        return out
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out_tensor, launch_meta = _run_sddmm_prepared(
        prepared, x.contiguous(), y.contiguous(),
        data.contiguous() if data is not None else None, alpha, beta, out,
        allow_fallback=allow_fallback)
    torch.cuda.synchronize()
    elapsed_ms = (time.perf_counter() - t0) * 1000.0
    meta = {"prepare_ms": prepare_ms, **launch_meta}
    if return_time and return_meta:
        return out_tensor, elapsed_ms, meta
    if return_time:
        return out_tensor, elapsed_ms
    if return_meta:
        return out_tensor, meta
    return out_tensor


def benchmark_sddmm_case(n_rows=1024, n_cols=1024, nnz=16384, k_dim=64,
                         value_dtype=torch.float32, warmup=10, iters=30, alpha=1.0, beta=0.0,
                         run_cusparse=False, seed=0):
    """SDDMM vs the torch sampled dot (sddmm_csr.py:472-572); CuPy is not part of this build."""
    if value_dtype not in SUPPORTED_SDDMM_VALUE_DTYPES:
        raise TypeError("value_dtype must be torch.float32 or torch.float64")
    device = torch.device("cuda")
    data, indices, indptr = build_random_csr(n_rows, n_cols, nnz, value_dtype, torch.int32,
                                             device, seed=seed)
    x = build_random_dense((n_rows, k_dim), value_dtype, device, seed=seed, stream=81)
    y = build_random_dense((n_cols, k_dim), value_dtype, device, seed=seed, stream=82)
    prepared = prepare_sddmm_csr(indices, indptr, (n_rows, n_cols), k_hint=k_dim)
    op = lambda: flagsparse_sddmm_csr(data=data, x=x, y=y, alpha=alpha, beta=beta,  # noqa: E731
                                      prepared=prepared, return_time=False)
    triton_values, triton_ms = _benchmark_cuda_op(op, warmup=warmup, iters=iters)
    ref_op = lambda: _sddmm_reference(indices, indptr.to(torch.int64), x, y, data,  # noqa: E731
                                      alpha, beta)
    ref_values, pytorch_ms = _benchmark_cuda_op(ref_op, warmup=warmup, iters=iters)
    atol, rtol = _tolerance_for_dtype(value_dtype)
    match = bool(torch.allclose(triton_values, ref_values, atol=atol, rtol=rtol))
    max_abs = (float(torch.max(torch.abs(triton_values - ref_values)).item())
               if triton_values.numel() > 0 else 0.0)
    return {
        "parameters": {"n_rows": n_rows, "n_cols": n_cols, "nnz": nnz, "k_dim": k_dim,
                       "value_dtype": str(value_dtype), "warmup": warmup, "iters": iters,
                       "alpha": alpha, "beta": beta},
        "performance": {"triton_ms": triton_ms, "pytorch_ms": pytorch_ms, "cusparse_ms": None,
                        "triton_speedup_vs_pytorch": (pytorch_ms / triton_ms
                                                      if triton_ms > 0 else None),
                        "triton_speedup_vs_cusparse": None},
        "verification": {"triton_match_pytorch": match, "triton_max_abs_error": max_abs,
                         "cusparse_match_pytorch": None},
        "backend_status": {"cusparse_unavailable_reason": (
            "CuPy is not part of the MI355X build" if run_cusparse else None)},
        "samples": {"triton": triton_values, "pytorch": ref_values},
    }
