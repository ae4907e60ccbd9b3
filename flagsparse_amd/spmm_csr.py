"""CSR SpMM C = A @ B on gfx950, behind the reference's entry points.

Public API and error behaviour mirror ``src/flagsparse/sparse_operations/spmm_csr.py``:
``flagsparse_spmm_csr`` (:1057-1126, base "ALG1" path, float32 computed in float64),
``prepare_spmm_csr_opt`` (:480-522) and ``flagsparse_spmm_csr_opt`` (:1129-1183, native
precision), the validation metrics (:6-90, :1186-1192) and the benchmark cases
(:1195-1562).

Both paths run ``spmm_rowblock_kernel`` (flagsparse_amd/csrc/spmm.hip): G lanes share each
B row with 16-byte loads along N, short rows are one row per lane group, rows longer than
128 entries are cut into parts whose sums are added in part order (deterministic).
"""

import time

import torch

from . import _abi, _common
from ._common import (
    SUPPORTED_INDEX_DTYPES,
    SUPPORTED_VALUE_DTYPES,
    _INDEX_LIMIT_INT32,
    _aligned,
    _benchmark_cuda_op,
    _is_complex_dtype,
    _require_kernel_dtype,
    _tolerance_for_dtype,
)
from ._index_stats import index_stats_device
from ._plan import StreamOrder, build_row_block_plan_device
from .synthetic import build_random_csr, build_random_dense

SUPPORTED_SPMM_VALUE_DTYPES = SUPPORTED_VALUE_DTYPES

XCD_REMAP = 1
# The row-block plan is built in windows of SPMM_PLAN_WINDOW_BLOCKS x the block row cap (each
# window's last block may be short).  Windows of one block's rows cut a block after every
# row-cap rows even when the entry cap ended the one before, adding a tiny block per window;
# wider windows make the planner (one thread per window) slower, which the paths that plan
# on every call pay each time.  Measured on MI355X, cfg5's matrix, fp32 N=16, per call
# (prepared / COO / base): 380 / 813 / 633 us with windows of 1 block, 329 / 840 / 657 with 4,
# 327 / 1124 / 957 with 16; N=64: 663 / 1087 / 924, 663 / 1099 / 930, 662 / 1174 / 1006.  So
# prepared matrices plan with 4 and the per-call paths with 1.
SPMM_PLAN_WINDOW_BLOCKS = 4
# Rows longer than this go to the part path (several lane groups per row).
_SPMM_ROW_SPLIT_THRESHOLD = 128


# ------------------------------------------------------------------------------------------
# Validation metrics (spmm_csr.py:6-90)
# ------------------------------------------------------------------------------------------


def _spmm_relative_threshold(value_dtype):
    if value_dtype == torch.float16:
        return 5e-3
    if value_dtype == torch.bfloat16:
        return 1e-2
    if value_dtype in (torch.float32, torch.complex64):
        return 1e-6
    if value_dtype in (torch.float64, torch.complex128):
        return 1e-12
    return 1e-6


def _spmm_coo_reference_tolerance(value_dtype):
    if value_dtype == torch.float16:
        return 2e-3, 2e-3
    if value_dtype == torch.bfloat16:
        return 1e-1, 1e-1
    if value_dtype in (torch.float32, torch.complex64):
        return 1e-4, 1e-2
    if value_dtype in (torch.float64, torch.complex128):
        return 1e-12, 1e-10
    return 1e-6, 1e-5


def _spmm_error_metrics(candidate, reference):
    if candidate.shape != reference.shape:
        raise ValueError(
            f"candidate and reference must have the same shape, got {candidate.shape} vs "
            f"{reference.shape}")
    if candidate.numel() == 0:
        return {"max_abs_error": 0.0, "max_relative_error": 0.0, "sum_relative_error": 0.0,
                "reference_max_magnitude": 0.0, "reference_sum_magnitude": 0.0}
    if _is_complex_dtype(reference.dtype):
        reference_compare = torch.abs(reference)
        abs_diff = torch.abs(torch.abs(candidate) - reference_compare)
    else:
        reference_compare = torch.abs(reference)
        abs_diff = torch.abs(candidate - reference)
    max_abs_error = float(torch.max(abs_diff).item())
    reference_max_magnitude = float(torch.max(reference_compare).item())
    sum_abs_error = float(torch.sum(abs_diff).item())
    reference_sum_magnitude = float(torch.sum(reference_compare).item())
    if reference_max_magnitude == 0.0:
        max_relative_error = 0.0 if max_abs_error == 0.0 else float("inf")
    else:
        max_relative_error = max_abs_error / reference_max_magnitude
    if reference_sum_magnitude == 0.0:
        sum_relative_error = 0.0 if sum_abs_error == 0.0 else float("inf")
    else:
        sum_relative_error = sum_abs_error / reference_sum_magnitude
    return {"max_abs_error": max_abs_error, "max_relative_error": max_relative_error,
            "sum_relative_error": sum_relative_error,
            "reference_max_magnitude": reference_max_magnitude,
            "reference_sum_magnitude": reference_sum_magnitude}


def _spmm_validation_metrics(candidate, reference):
    metrics = _spmm_error_metrics(candidate, reference)
    threshold = _spmm_relative_threshold(reference.dtype)
    atol, rtol = _tolerance_for_dtype(reference.dtype)
    metrics.update({
        "relative_threshold": threshold,
        "matches_threshold": metrics["max_relative_error"] <= threshold,
        "strict_allclose_match": torch.allclose(candidate, reference, atol=atol, rtol=rtol),
    })
    return metrics


def _spmm_opt_reference_error(candidate, reference, value_dtype):
    atol, rtol = _spmm_coo_reference_tolerance(value_dtype)
    if candidate.numel() == 0:
        return 0.0
    diff = torch.abs(candidate - reference)
    denom = atol + rtol * torch.abs(reference)
    return float(torch.max(diff / denom).item())


# ------------------------------------------------------------------------------------------
# Validation and launch configuration
# ------------------------------------------------------------------------------------------


def _prepare_spmm_csr_matrix(data, indices, indptr, shape):
    """spmm_csr.py:197-255 (same checks, order and exceptions; the device-side checks are
    gathered into one host synchronisation)."""
    if len(shape) != 2:
        raise ValueError("shape must be a 2-tuple: (n_rows, n_cols)")
    if data.ndim != 1 or indices.ndim != 1 or indptr.ndim != 1:
        raise ValueError("data, indices, and indptr must be 1D tensors")
    n_rows, n_cols = int(shape[0]), int(shape[1])
    if n_rows < 0 or n_cols < 0:
        raise ValueError("shape dimensions must be non-negative")
    if indptr.numel() != n_rows + 1:
        raise ValueError(f"indptr length must be n_rows+1={n_rows + 1}, got {indptr.numel()}")
    if data.numel() != indices.numel():
        raise ValueError("data and indices must have the same length (nnz)")
    if not all(t.is_cuda for t in (data, indices, indptr)):
        raise ValueError("data, indices, and indptr must be CUDA tensors")
    if not all(t.device == data.device for t in (indices, indptr)):
        raise ValueError("data, indices, and indptr must be on the same CUDA device")
    if data.dtype not in SUPPORTED_SPMM_VALUE_DTYPES:
        raise TypeError(
            "data dtype must be one of: float16, bfloat16, float32, float64, complex64, complex128"
        )
    if indices.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("indices dtype must be torch.int32 or torch.int64")
    if indptr.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("indptr dtype must be torch.int32 or torch.int64")

    nnz = data.numel()
    probes = [indptr[0].to(torch.int64), indptr[-1].to(torch.int64)]
    if indptr.numel() > 1:
        probes.append(torch.any(indptr[1:] < indptr[:-1]).to(torch.int64))
        probes.append(torch.max(indptr[1:] - indptr[:-1]).to(torch.int64))
    if nnz > 0:
        probes += list(index_stats_device(indices.contiguous(), indices.contiguous())[:2])
    vals = torch.stack(probes).tolist()
    if vals[0] != 0:
        raise ValueError("indptr[0] must be 0")
    if vals[1] != nnz:
        raise ValueError(f"indptr[-1] must equal nnz={nnz}, got {vals[1]}")
    pos = 2
    max_row_nnz = 0
    if indptr.numel() > 1:
        if vals[2]:
            raise ValueError("indptr must be nondecreasing")
        max_row_nnz = vals[3]
        pos = 4
    if nnz > 0:
        min_col, max_col = vals[pos], vals[pos + 1]
        if min_col < 0 or max_col >= n_cols:
            raise IndexError("indices out of range for n_cols")
        if max_col > _INDEX_LIMIT_INT32:
            raise ValueError(
                "column indices exceed the int32 range supported by the Triton kernel")

    data = data.contiguous()
    indices = indices.contiguous()
    indptr = indptr.contiguous()
    kernel_indices = indices.to(torch.int32) if indices.dtype == torch.int64 else indices
    kernel_indptr = indptr.to(torch.int64)
    row_lengths = (kernel_indptr[1:] - kernel_indptr[:-1] if n_rows > 0
                   else kernel_indptr.new_empty((0,)))
    return data, kernel_indices, kernel_indptr, n_rows, n_cols, row_lengths, int(max_row_nnz)


def _prepare_spmm_csr_inputs(data, indices, indptr, B, shape):
    """spmm_csr.py:258-281."""
    if B.ndim != 2:
        raise ValueError("B must be a 2D dense tensor")
    (data, kernel_indices, kernel_indptr, n_rows, n_cols, _row_lengths,
     max_row_nnz) = _prepare_spmm_csr_matrix(data, indices, indptr, shape)
    if B.shape[0] != n_cols:
        raise ValueError(f"B.shape[0] must be n_cols={n_cols}, got {B.shape[0]}")
    if not B.is_cuda:
        raise ValueError("B must be a CUDA tensor")
    if B.device != data.device:
        raise ValueError("B must be on the same CUDA device as the sparse matrix")
    if B.dtype != data.dtype:
        raise TypeError("B dtype must match data dtype")
    B = B.contiguous()
    return (data, kernel_indices, kernel_indptr, B, n_rows, n_cols, int(B.shape[1]),
            max_row_nnz)


def _select_spmm_alg1_warp_and_factor(n_dense_cols):
    """spmm_csr.py:284-296."""
    if n_dense_cols > 64:
        return 32, 4
    if n_dense_cols > 32:
        return 32, 2
    if n_dense_cols > 16:
        return 32, 1
    if n_dense_cols > 8:
        return 16, 1
    if n_dense_cols > 4:
        return 8, 1
    return 4, 1


def _resolve_spmm_alg1_launch_config(n_dense_cols, max_row_nnz, block_n=None, block_nnz=None,
                                     max_segments=None):
    """spmm_csr.py:299-334 (ValueError when max_segments cannot cover the longest row)."""
    warp_size, factor = _select_spmm_alg1_warp_and_factor(n_dense_cols)
    if block_n is None:
        block_n = warp_size * factor
    if block_nnz is None:
        block_nnz = warp_size
    if block_n <= 0 or block_nnz <= 0:
        raise ValueError("block_n and block_nnz must be positive when provided")
    if max_segments is not None and max_segments <= 0:
        raise ValueError("max_segments must be positive when provided")
    required_segments = -(-max_row_nnz // block_nnz) if max_row_nnz > 0 else 0
    if max_segments is not None and required_segments > int(max_segments):
        raise ValueError(
            "row nnz requires more CSR segments than the explicit max_segments override allows: "
            f"required {required_segments}, provided {int(max_segments)}")
    return {
        "block_n": int(block_n),
        "block_nnz": int(block_nnz),
        "max_segments": (None if max_segments is None else int(max_segments)),
        "required_segments": int(required_segments),
        "warp_size": int(warp_size),
        "factor": int(factor),
        "max_row_nnz": int(max_row_nnz),
        "auto_max_segments": max_segments is None,
    }


def _next_pow2(v):
    p = 1
    while p < v:
        p <<= 1
    return p


def _spmm_lane_shape(n_dense_cols, dtype, B, C, tile_cols=None):
    """(lanes per B row G, elements per lane vec) for the gfx950 kernel.

    vec: 16-byte loads (4 fp32 / 2 fp64) when N and both base pointers allow it, else 2 or 1.
    G: enough lanes to cover min(N, tile_cols) columns, a power of two <= 64.  The kernel's
    column tile is G * vec, so with narrower lanes (odd N, unaligned B or C) a tile of more
    than 64 * vec columns is launched as tiles of 64 * vec.
    """
    vmax = 4 if dtype == torch.float32 else 2
    aligned = B.data_ptr() % 16 == 0 and C.data_ptr() % 16 == 0
    vec = 1
    for v in (vmax, 2):
        if aligned and n_dense_cols % v == 0:
            vec = v
            break
    width = n_dense_cols if tile_cols is None else max(1, min(n_dense_cols, int(tile_cols)))
    lanes = min(64, _next_pow2(max(1, -(-width // vec))))
    return lanes, vec


class _SpmmKernelCsr:
    """Kernel-facing CSR arrays (aligned, int32 offsets when they fit) and plans per G."""

    __slots__ = ("data", "cols", "rowptr", "rowptr_bits", "nnz", "n_rows", "_plans", "_args",
                 "_keep", "window_blocks", "_order")

    def __init__(self, data, cols, indptr64, window_blocks=None):
        # window_blocks: plan window in blocks' rows (SPMM_PLAN_WINDOW_BLOCKS when None); the
        # paths that plan on every call use 1, which plans fastest
        self.window_blocks = window_blocks
        self.data = _aligned(data)
        self.cols = _aligned(cols)
        self.nnz = int(data.numel())
        self.n_rows = int(indptr64.numel()) - 1
        if self.nnz <= _common.ROWPTR32_MAX_NNZ:
            self.rowptr, self.rowptr_bits = indptr64.to(torch.int32), 32
        else:
            self.rowptr, self.rowptr_bits = indptr64.to(torch.int64).contiguous(), 64
        self._plans = {}
        self._args = {}
        self._keep = [self.data, self.cols, self.rowptr]  # what a launch reads or writes
        self._order = StreamOrder(self.data.device)

    def kernel_name(self):
        return "spmm_rowblock_kernel"

    def describe(self):
        return {"layout": "rowblock", "plans": {g: {"descriptors": p.n_desc,
                                                    "split_rows": p.n_split_rows}
                                                for g, p in self._plans.items()}}

    def plan(self, lanes):
        p = self._plans.get(lanes)
        if p is None:
            ngrp = 256 // lanes
            cap = _abi.caps()["spmm_block_nnz"]
            threshold = min(_SPMM_ROW_SPLIT_THRESHOLD, cap)
            chunk = min(cap, max(threshold, 16 * ngrp))
            p = build_row_block_plan_device(self.rowptr, cap, ngrp, threshold, chunk,
                                            window_rows=(self.window_blocks
                                                         or SPMM_PLAN_WINDOW_BLOCKS) * ngrp)
            self._plans[lanes] = p
        return p


# A B of more than half this many bytes is read in column tiles: the widest power of two of
# columns narrower than B whose slice is at most this many bytes (the kernel walks the tiles in
# launch order, so one tile's rows of B are gathered at a time and stay in the 256 MiB MALL for
# longer).  Measured on MI355X, cfg5's matrix: fp32 N=256 (B of 1 GiB) 3.34 -> 2.86 ms with
# tiles of 128 columns (64: 3.01, 32: 2.92); fp64 N=256 6.69 -> 5.82 ms (64); B of 512 MiB:
# fp64 N=64 1437 -> 1372 us (32; 16: 1466), fp32 N=128 1416 -> 1350 us (64; 32: 1490); B of
# 256 MiB is fastest untiled (fp32 N=64 662 vs 710 us with 32; fp64 N=32 689 vs 770 with 16).
SPMM_B_TILE_BYTES = 512 << 20


def _auto_tile_cols(B):
    """Column tile for a large B (None: no tiling), by the rule above."""
    rows, n, v = int(B.shape[0]), int(B.shape[1]), B.element_size()
    if 2 * rows * n * v <= SPMM_B_TILE_BYTES:
        return None
    t = _next_pow2(n)
    while t > 4 and (t >= n or rows * t * v > SPMM_B_TILE_BYTES):
        t >>= 1
    return t if t < n else None


def _run_spmm(kc, B, C, acc_f64, tile_cols=None):
    """Launch fsp_spmm_csr: C[n_rows, N] = A @ B (B, C contiguous row-major).  Without an
    explicit tile (the reference's block_n), a B over SPMM_B_TILE_BYTES is tiled by columns."""
    n_dense_cols = int(B.shape[1])
    if kc.n_rows == 0 or n_dense_cols == 0:
        return C
    if tile_cols is None:
        tile_cols = _auto_tile_cols(B)
    dtype = B.dtype
    lanes, vec = _spmm_lane_shape(n_dense_cols, dtype, B, C, tile_cols)
    key = (lanes, vec, n_dense_cols, bool(acc_f64), dtype)
    args = kc._args.get(key)
    if args is None:  # the arguments that do not change between calls, converted once
        plan = kc.plan(lanes)
        partials = plan.workspace(n_dense_cols)
        groups, group_base, split_rows = plan.split_groups()
        p = lambda t: t.data_ptr() if t.numel() else None  # noqa: E731
        args = [_abi.dtype_code(dtype), 1 if acc_f64 else 0, p(kc.data), p(kc.cols),
                p(kc.rowptr), kc.rowptr_bits, kc.n_rows, kc.nnz, None, 0, n_dense_cols, None, 0,
                p(plan.desc), plan.n_desc, plan.chunk, lanes, vec, p(partials), p(groups),
                p(group_base), p(split_rows), int(groups.shape[0]), 0, None]
        kc._args[key] = args
        kc._keep.extend((partials, plan.desc, groups, group_base, split_rows))
    a = list(args)
    a[8], a[9], a[11], a[12] = B.data_ptr(), B.stride(0), C.data_ptr(), C.stride(0)
    a[23] = XCD_REMAP
    a[24] = kc._order.stream(C.device, kc._keep)
    _abi.check(_abi.lib().fsp_spmm_csr(*a), "fsp_spmm_csr")
    return C


def _out_ok_direct(out, inputs):
    if out is None or not out.is_contiguous() or out.data_ptr() % 16:
        return False
    base = out.untyped_storage().data_ptr()
    return all(t.untyped_storage().data_ptr() != base for t in inputs)


# ------------------------------------------------------------------------------------------
# Opt path: prepared object and entry point
# ------------------------------------------------------------------------------------------

_SPMM_OPT_BUCKET_SPECS = (
    {"max_row_nnz": 32, "kind": "batched", "batch_rows": 8, "block_nnz": 32},
    {"max_row_nnz": 128, "kind": "batched", "batch_rows": 4, "block_nnz": 64},
    {"max_row_nnz": 512, "kind": "vector", "batch_rows": 1, "block_nnz": 128},
    {"max_row_nnz": 2048, "kind": "vector", "batch_rows": 1, "block_nnz": 128},
    {"max_row_nnz": None, "kind": "split", "batch_rows": 1, "block_nnz": 256},
)
_SPMM_OPT_LONG_ROW_THRESHOLD = 2048


class PreparedCsrSpmmOpt:
    """Cached CSR metadata for repeated SpMM-opt calls (spmm_csr.py:337-392).

    ``row_buckets`` and the ``long_*`` split attributes reproduce the reference's metadata on
    first access (spmm_csr.py:417-477); the gfx950 kernel runs from its own descriptor plan.
    """

    __slots__ = (
        "data",
        "kernel_indices",
        "kernel_indptr",
        "shape",
        "n_rows",
        "n_cols",
        "row_lengths",
        "max_row_nnz",
        "supports_opt",
        "long_row_fallback_only",
        "_ref_meta",
        "_kernel",
    )

    def __init__(self, data, kernel_indices, kernel_indptr, shape, n_rows, n_cols, row_lengths,
                 max_row_nnz):
        self.data = data
        self.kernel_indices = kernel_indices
        self.kernel_indptr = kernel_indptr
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows = int(n_rows)
        self.n_cols = int(n_cols)
        self.row_lengths = row_lengths
        self.max_row_nnz = int(max_row_nnz)
        self.supports_opt = data.dtype in (torch.float32, torch.float64)
        self.long_row_fallback_only = False
        self._ref_meta = None
        self._kernel = None

    def _kernel_csr(self):
        if self._kernel is None:
            self._kernel = _SpmmKernelCsr(self.data, self.kernel_indices, self.kernel_indptr)
        return self._kernel

    def _reference_metadata(self):
        if self._ref_meta is None:
            device = self.data.device
            row_index_dtype = (torch.int32 if self.row_lengths.numel() - 1 <= _INDEX_LIMIT_INT32
                               else torch.int64)
            buckets = []
            lower = 0
            long_rows = torch.empty((0,), dtype=row_index_dtype, device=device)
            for spec in _SPMM_OPT_BUCKET_SPECS:
                upper = spec["max_row_nnz"]
                if upper is None:
                    mask = self.row_lengths > lower
                elif lower == 0:
                    mask = self.row_lengths <= upper
                else:
                    mask = (self.row_lengths > lower) & (self.row_lengths <= upper)
                rows = torch.nonzero(mask, as_tuple=False).flatten().to(row_index_dtype)
                if rows.numel():
                    buckets.append({"kind": spec["kind"], "rows": rows,
                                    "batch_rows": spec["batch_rows"],
                                    "block_nnz": spec["block_nnz"]})
                    if spec["kind"] == "split":
                        long_rows = rows
                if upper is not None:
                    lower = upper
            part_rows, starts, ends, ptr = [], [], [], [0]
            if long_rows.numel():
                ip = self.kernel_indptr.to(torch.int64).cpu().tolist()
                for r in long_rows.to(torch.int64).cpu().tolist():
                    cur, end = ip[r], ip[r + 1]
                    while cur < end:
                        part_rows.append(r)
                        starts.append(cur)
                        cur = min(cur + 256, end)
                        ends.append(cur)
                    ptr.append(len(part_rows))
            self._ref_meta = {
                "row_buckets": buckets,
                "long_row_ids": long_rows,
                "long_part_rows": torch.tensor(part_rows, dtype=long_rows.dtype, device=device),
                "long_part_starts": torch.tensor(starts, dtype=torch.int64, device=device),
                "long_part_ends": torch.tensor(ends, dtype=torch.int64, device=device),
                "long_row_part_ptr": torch.tensor(ptr, dtype=torch.int64, device=device),
            }
        return self._ref_meta

    @property
    def row_buckets(self):
        return self._reference_metadata()["row_buckets"]

    @property
    def long_row_ids(self):
        return self._reference_metadata()["long_row_ids"]

    @property
    def long_part_rows(self):
        return self._reference_metadata()["long_part_rows"]

    @property
    def long_part_starts(self):
        return self._reference_metadata()["long_part_starts"]

    @property
    def long_part_ends(self):
        return self._reference_metadata()["long_part_ends"]

    @property
    def long_row_part_ptr(self):
        return self._reference_metadata()["long_row_part_ptr"]


def prepare_spmm_csr_opt(data, indices, indptr, shape):
    """spmm_csr.py:480-522: validation plus the gfx950 row-block plan for common widths."""
    (data, kernel_indices, kernel_indptr, n_rows, n_cols, row_lengths,
     max_row_nnz) = _prepare_spmm_csr_matrix(data, indices, indptr, shape)
    prepared = PreparedCsrSpmmOpt(data, kernel_indices, kernel_indptr, shape, n_rows, n_cols,
                                  row_lengths, max_row_nnz)
    if prepared.supports_opt and n_rows > 0:
        prepared._kernel_csr()
    return prepared


def _triton_spmm_csr_impl_opt_prepared(prepared, B):
    """spmm_csr.py:1033-1055 checks, then one gfx950 launch (native-precision accumulation)."""
    if not prepared.supports_opt:
        raise TypeError("spmm opt only supports float32 and float64")
    if not B.is_cuda:
        raise ValueError("B must be a CUDA tensor")
    if B.device != prepared.data.device:
        raise ValueError("B must be on the same CUDA device as the sparse matrix")
    if B.dtype != prepared.data.dtype:
        raise TypeError("B dtype must match sparse matrix dtype")
    if B.shape[0] != prepared.n_cols:
        raise ValueError(f"B.shape[0] must be n_cols={prepared.n_cols}, got {B.shape[0]}")
    if B.ndim != 2:
        raise ValueError("B must be a 2D dense tensor")
    return B.contiguous()


def flagsparse_spmm_csr_opt(data=None, indices=None, indptr=None, B=None, shape=None,
                            prepared=None, out=None, return_time=False):
    """CSR SpMM-opt: native float32/float64 path for CSR @ dense (spmm_csr.py:1129-1183)."""
    if prepared is not None and not isinstance(prepared, PreparedCsrSpmmOpt):
        raise TypeError("prepared must be a PreparedCsrSpmmOpt instance")
    if prepared is None:
        if any(arg is None for arg in (data, indices, indptr, shape)):
            raise ValueError(
                "data, indices, indptr, and shape are required when prepared is not provided")
        prepared = prepare_spmm_csr_opt(data, indices, indptr, shape)
    elif shape is not None:
        resolved_shape = (int(shape[0]), int(shape[1]))
        if resolved_shape != prepared.shape:
            raise ValueError(
                f"shape {resolved_shape} does not match prepared.shape {prepared.shape}")
    if B is None:
        raise ValueError("B is required")
    if not prepared.supports_opt:
        raise TypeError("flagsparse_spmm_csr_opt only supports float32 and float64")
    if not B.is_cuda:
        raise ValueError("B must be a CUDA tensor")
    if B.device != prepared.data.device:
        raise ValueError("B must be on the same CUDA device as sparse matrix data")
    if out is not None:
        if not out.is_cuda:
            raise ValueError("out must be a CUDA tensor")
        if out.device != prepared.data.device:
            raise ValueError("out must be on the same CUDA device as sparse matrix data")
        if out.shape != (prepared.n_rows, int(B.shape[1])) or out.dtype != prepared.data.dtype:
            raise ValueError("out shape/dtype must match result")
    t0 = None
    if return_time:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
    B = _triton_spmm_csr_impl_opt_prepared(prepared, B)
    n_dense_cols = int(B.shape[1])
    direct = _out_ok_direct(out, (B, prepared.data))
    C = out if direct else torch.empty((prepared.n_rows, n_dense_cols), dtype=B.dtype,
                                       device=B.device)
    _run_spmm(prepared._kernel_csr(), B, C, acc_f64=B.dtype == torch.float64)
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


# ------------------------------------------------------------------------------------------
# Base (ALG1) path
# ------------------------------------------------------------------------------------------


def flagsparse_spmm_csr(data, indices, indptr, B, shape, block_n=None, block_nnz=None,
                        max_segments=None, out=None, return_time=False):
    """CSR SpMM C = A @ B (spmm_csr.py:1057-1126).

    float32 is accumulated in float64 and rounded once, as in the reference.  ``block_n``
    sets the column tile of a workgroup; ``block_nnz`` / ``max_segments`` are validated with
    the reference's ALG1 rules (ValueError when max_segments cannot cover the longest row).
    """
    if block_n is not None and block_n <= 0:
        raise ValueError("block_n must be positive when provided")
    if block_nnz is not None and block_nnz <= 0:
        raise ValueError("block_nnz must be positive when provided")
    if max_segments is not None and max_segments <= 0:
        raise ValueError("max_segments must be positive when provided")
    (data, kernel_indices, kernel_indptr, B, n_rows, _n_cols, n_dense_cols,
     max_row_nnz) = _prepare_spmm_csr_inputs(data, indices, indptr, B, shape)
    launch = _resolve_spmm_alg1_launch_config(n_dense_cols, max_row_nnz, block_n=block_n,
                                              block_nnz=block_nnz, max_segments=max_segments)
    if out is not None:
        if not out.is_cuda:
            raise ValueError("out must be a CUDA tensor")
        if out.device != data.device:
            raise ValueError("out must be on the same CUDA device as the inputs")
        if out.shape != (n_rows, n_dense_cols) or out.dtype != data.dtype:
            raise ValueError("out shape/dtype must match result")
    dtype = data.dtype
    t0 = None
    if return_time:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
    if n_rows == 0 or n_dense_cols == 0 or B.shape[0] == 0:
        C = torch.zeros((n_rows, n_dense_cols), dtype=dtype, device=data.device)
        direct = False
    else:
        _require_kernel_dtype(dtype, "flagsparse_spmm_csr")
        kc = _SpmmKernelCsr(data, kernel_indices, kernel_indptr, window_blocks=1)
        direct = _out_ok_direct(out, (B, data))
        C = out if direct else torch.empty((n_rows, n_dense_cols), dtype=dtype,
                                           device=data.device)
        tile = launch["block_n"] if block_n is not None else None
        _run_spmm(kc, B, C, acc_f64=True, tile_cols=tile)
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


# ------------------------------------------------------------------------------------------
# Benchmark cases (spmm_csr.py:1195-1562): same result dictionaries; the "triton_*" keys
# name the flagsparse kernel as in the reference, cuSPARSE/CuPy is reported unavailable.
# ------------------------------------------------------------------------------------------


def _torch_sparse_reference(data, indices, indptr, B, shape):
    indptr64 = indptr.to(torch.int64)
    indices64 = indices.to(torch.int64)
    ref_dtype = torch.float64 if data.dtype == torch.float32 else data.dtype
    csr_ref = torch.sparse_csr_tensor(indptr64, indices64, data.to(ref_dtype), size=shape,
                                      device=data.device)
    return torch.sparse.mm(csr_ref, B.to(ref_dtype)).to(data.dtype)


def benchmark_spmm_opt_case(n_rows=4096, n_cols=4096, nnz=65536, n_dense_cols=32,
                            value_dtype=torch.float32, index_dtype=torch.int32, warmup=20,
                            iters=200, run_cusparse=True, seed=0):
    """Base vs opt SpMM against one high-precision torch.sparse reference."""
    if value_dtype not in (torch.float32, torch.float64):
        raise TypeError("benchmark_spmm_opt_case only supports float32 and float64")
    device = torch.device("cuda")
    data, indices, indptr = build_random_csr(n_rows, n_cols, nnz, value_dtype, index_dtype,
                                             device, seed=seed)
    B = build_random_dense((n_cols, n_dense_cols), value_dtype, device, seed=seed)
    shape = (n_rows, n_cols)
    prepared = prepare_spmm_csr_opt(data, indices, indptr, shape)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    base_values = flagsparse_spmm_csr(data, indices, indptr, B, shape)
    torch.cuda.synchronize()
    base_first_call_ms = (time.perf_counter() - t0) * 1000.0
    base_values, base_ms = _benchmark_cuda_op(
        lambda: flagsparse_spmm_csr(data, indices, indptr, B, shape), warmup=warmup, iters=iters)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    opt_values = flagsparse_spmm_csr_opt(B=B, prepared=prepared)
    torch.cuda.synchronize()
    opt_first_call_ms = (time.perf_counter() - t0) * 1000.0
    opt_values, opt_ms = _benchmark_cuda_op(
        lambda: flagsparse_spmm_csr_opt(B=B, prepared=prepared), warmup=warmup, iters=iters)

    ref = _torch_sparse_reference(data, indices, indptr, B, shape)
    pt_ms = None
    try:
        pt_sparse = torch.sparse_csr_tensor(indptr.to(torch.int64), indices.to(torch.int64),
                                            data, size=shape, device=device)
        _, pt_ms = _benchmark_cuda_op(lambda: torch.sparse.mm(pt_sparse, B), warmup=warmup,
                                      iters=iters)
    except Exception:
        pt_ms = None
    err_base = _spmm_opt_reference_error(base_values, ref, value_dtype)
    err_opt = _spmm_opt_reference_error(opt_values, ref, value_dtype)
    return {
        "parameters": {"n_rows": n_rows, "n_cols": n_cols, "nnz": nnz,
                       "n_dense_cols": n_dense_cols, "value_dtype": str(value_dtype),
                       "index_dtype": str(index_dtype)},
        "performance": {
            "base_ms": base_ms, "base_first_call_ms": base_first_call_ms, "opt_ms": opt_ms,
            "opt_first_call_ms": opt_first_call_ms, "pt_ms": pt_ms, "cu_ms": None,
            "opt_vs_base": (base_ms / opt_ms if opt_ms and opt_ms > 0 else None),
            "opt_vs_pt": (pt_ms / opt_ms if pt_ms is not None and opt_ms > 0 else None),
            "opt_vs_cu": None,
        },
        "verification": {"err_base": err_base, "err_opt": err_opt, "base_ok": err_base <= 1.0,
                         "opt_ok": err_opt <= 1.0,
                         "status": ("PASS" if err_opt <= 1.0 else "FAIL")},
        "backend_status": {"long_row_fallback_used": bool(prepared.long_row_fallback_only),
                           "flagsparse_internal_route": "gfx950-rowblock"},
        "samples": {"base": base_values, "opt": opt_values, "reference": ref},
    }


def benchmark_spmm_case(n_rows=4096, n_cols=4096, nnz=65536, n_dense_cols=32,
                        value_dtype=torch.float32, index_dtype=torch.int32, warmup=20, iters=200,
                        block_n=None, block_nnz=None, max_segments=None, run_cusparse=True,
                        seed=0):
    """flagsparse SpMM vs torch.sparse.mm (CuPy/cuSPARSE is not part of this build)."""
    device = torch.device("cuda")
    data, indices, indptr = build_random_csr(n_rows, n_cols, nnz, value_dtype, index_dtype,
                                             device, seed=seed)
    B = build_random_dense((n_cols, n_dense_cols), value_dtype, device, seed=seed)
    shape = (n_rows, n_cols)
    max_row_nnz = int(torch.max(indptr[1:] - indptr[:-1]).item()) if n_rows > 0 else 0
    launch = _resolve_spmm_alg1_launch_config(n_dense_cols, max_row_nnz, block_n=block_n,
                                              block_nnz=block_nnz, max_segments=max_segments)
    kwargs = {"data": data, "indices": indices, "indptr": indptr, "B": B, "shape": shape,
              "block_n": launch["block_n"], "block_nnz": launch["block_nnz"],
              "max_segments": launch["max_segments"], "return_time": False}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    _ = flagsparse_spmm_csr(**kwargs)
    torch.cuda.synchronize()
    first_call_ms = (time.perf_counter() - t0) * 1000.0
    triton_C, triton_ms = _benchmark_cuda_op(lambda: flagsparse_spmm_csr(**kwargs),
                                             warmup=warmup, iters=iters)
    pytorch_reason = None
    pytorch_ms = None
    expected = _torch_sparse_reference(data, indices, indptr, B, shape)
    pytorch_values = expected
    try:
        csr_pt = torch.sparse_csr_tensor(indptr.to(torch.int64), indices.to(torch.int64), data,
                                         size=shape, device=device)
        pytorch_values, pytorch_ms = _benchmark_cuda_op(lambda: torch.sparse.mm(csr_pt, B),
                                                        warmup=warmup, iters=iters)
    except Exception as exc:
        pytorch_reason = str(exc)
    metrics = _spmm_validation_metrics(triton_C, expected)
    threshold = _spmm_relative_threshold(value_dtype)
    return {
        "parameters": {
            "format": "csr", "n_rows": n_rows, "n_cols": n_cols, "nnz": nnz,
            "n_dense_cols": n_dense_cols, "value_dtype": str(value_dtype),
            "index_dtype": str(index_dtype), "warmup": warmup, "iters": iters,
            "block_n": launch["block_n"], "block_nnz": launch["block_nnz"],
            "max_segments": launch["max_segments"],
            "required_segments": launch["required_segments"],
            "alg1_warp_size": launch["warp_size"], "alg1_factor": launch["factor"],
            "auto_max_segments": launch["auto_max_segments"], "run_cusparse": run_cusparse,
        },
        "performance": {
            "pytorch_ms": pytorch_ms, "triton_ms": triton_ms,
            "triton_first_call_ms": first_call_ms, "cusparse_ms": None,
            "triton_speedup_vs_pytorch": (pytorch_ms / triton_ms
                                          if pytorch_ms is not None and triton_ms > 0 else None),
            "triton_speedup_vs_cusparse": None,
        },
        "verification": {
            "triton_match_reference": metrics["strict_allclose_match"],
            "triton_match_pytorch": metrics["strict_allclose_match"],
            "triton_max_error": metrics["max_abs_error"],
            "triton_max_abs_error": metrics["max_abs_error"],
            "triton_max_relative_error": metrics["max_relative_error"],
            "triton_sum_relative_error": metrics["sum_relative_error"],
            "triton_relative_threshold": metrics["relative_threshold"],
            "triton_strict_allclose_match": metrics["strict_allclose_match"],
            "pytorch_match_reference": True, "pytorch_max_error": 0.0,
            "pytorch_max_abs_error": 0.0, "pytorch_max_relative_error": 0.0,
            "pytorch_sum_relative_error": 0.0, "pytorch_relative_threshold": threshold,
            "cusparse_match_reference": None, "cusparse_match_pytorch": None,
            "cusparse_max_error": None, "cusparse_max_abs_error": None,
            "cusparse_max_relative_error": None, "cusparse_sum_relative_error": None,
            "cusparse_relative_threshold": threshold, "cusparse_strict_allclose_match": None,
        },
        "backend_status": {
            "pytorch_unavailable_reason": pytorch_reason, "pytorch_sparse_format": "CSR",
            "cusparse_unavailable_reason": "CuPy/cuSPARSE is not part of the MI355X build",
            "flagsparse_internal_route": "gfx950-rowblock",
        },
        "samples": {"pytorch": pytorch_values, "triton": triton_C, "reference": expected,
                    "cusparse": None},
    }


def comprehensive_spmm_test(n_rows=4096, n_cols=4096, nnz=65536, n_dense_cols=32,
                            dtype=torch.float32, index_dtype=torch.int32, warmup=20, iters=200,
                            block_n=None, block_nnz=None, max_segments=None, run_cusparse=True):
    """Full SpMM benchmark entry for one configuration (spmm_csr.py:1534-1562)."""
    return benchmark_spmm_case(n_rows=n_rows, n_cols=n_cols, nnz=nnz, n_dense_cols=n_dense_cols,
                               value_dtype=dtype, index_dtype=index_dtype, warmup=warmup,
                               iters=iters, block_n=block_n, block_nnz=block_nnz,
                               max_segments=max_segments, run_cusparse=run_cusparse)
