"""CSR SpMV y = A @ x on gfx950, behind the reference's entry points.

Public API and error behaviour mirror ``src/flagsparse/sparse_operations/spmv_csr.py``:
``prepare_spmv_csr`` (:455-495), ``flagsparse_spmv_csr`` (:557-610),
``coo_to_csr_for_spmv`` (:623-647), ``prepare_spmv_coo_tocsr`` (:650-684) and
``flagsparse_spmv_coo_tocsr`` (:687-758).

Numerics: the default path (``use_opt=False``) returns fp32(fp64 row sum) for float32 input,
as the reference's base path does (:498-536); ``use_opt=True`` accumulates in the input type
(:161-279).  float64 always accumulates in float64.  A caller's ``max_segments`` truncates
rows exactly where the reference's static tile loop stops (:111-118 base, :308-314 opt).

The kernel is one launch over a layout built once per matrix (flagsparse_amd/_spmv_layouts.py):
row blocks (csrc/spmv.hip) or, when x gathers would miss L2, the XCD column split
(csrc/spmv_xcs.hip).
"""

import time

import torch

from ._common import (
    SUPPORTED_INDEX_DTYPES,
    SUPPORTED_VALUE_DTYPES,
    _INDEX_LIMIT_INT32,
    _require_kernel_dtype,
)
from ._plan import truncate_rows
from ._spmv_layouts import build_layout

# Opt-path buckets of the reference (max_row_nnz, block_size, num_warps, num_stages,
# batch_rows) - spmv_csr.py:64-89.  Only their truncation effect under a caller's
# max_segments, and the ``opt_buckets`` attribute, depend on them here.
_SPMV_OPT_BUCKET_CONFIGS = (
    (64, 32, 1, 2, 16),
    (512, 256, 8, 2, 1),
    (4096, 512, 16, 2, 1),
    (None, 1024, 32, 3, 1),
)
_SPMV_OPT_BUCKET_CONFIGS_FP64 = (
    (64, 32, 1, 2, 4),
    (256, 64, 2, 2, 1),
    (2048, 128, 4, 2, 1),
    (8192, 256, 8, 2, 1),
    (None, 512, 16, 1, 1),
)


def _opt_bucket_block_sizes(row_lengths, fp64):
    """Per-row block_size of the reference's opt bucket (spmv_csr.py:291-302)."""
    configs = _SPMV_OPT_BUCKET_CONFIGS_FP64 if fp64 else _SPMV_OPT_BUCKET_CONFIGS
    bs = torch.empty_like(row_lengths)
    lower = 0
    for upper, block_size, _w, _s, _b in configs:
        if upper is None:
            mask = row_lengths > lower
        elif lower == 0:
            mask = row_lengths <= upper
        else:
            mask = (row_lengths > lower) & (row_lengths <= upper)
        bs[mask] = block_size
        if upper is not None:
            lower = upper
    return bs


class PreparedCsrSpmv:
    """Cached CSR metadata for repeated SpMV calls on the same sparse matrix
    (reference: spmv_csr.py:9-58)."""

    __slots__ = (
        "data",
        "kernel_indices",
        "kernel_indptr",
        "shape",
        "n_rows",
        "n_cols",
        "block_nnz",
        "max_segments",
        "max_row_nnz",
        "supports_opt",
        "_user_max_segments",
        "_row_lengths",
        "_opt_buckets",
        "_kernels",
        "_baseline_compute_dtype",
        "_baseline_data",
        "_one_shot",
    )

    def __init__(self, data, kernel_indices, kernel_indptr, shape, n_rows, n_cols, block_nnz,
                 max_segments, max_row_nnz, row_lengths, user_max_segments):
        self.data = data
        self.kernel_indices = kernel_indices
        self.kernel_indptr = kernel_indptr
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows = n_rows
        self.n_cols = n_cols
        self.block_nnz = block_nnz
        self.max_segments = max_segments
        self.max_row_nnz = max_row_nnz
        self._one_shot = False
        self.supports_opt = data.dtype in (torch.float32, torch.float64)
        if data.dtype in (torch.float16, torch.bfloat16):
            self._baseline_compute_dtype = torch.float32
        elif data.dtype == torch.float32:
            self._baseline_compute_dtype = torch.float64
        else:
            self._baseline_compute_dtype = data.dtype
        self._baseline_data = None
        self._user_max_segments = user_max_segments
        self._row_lengths = row_lengths
        self._opt_buckets = None
        self._kernels = {}

    @property
    def opt_buckets(self):
        """The reference's opt-path row buckets (spmv_csr.py:281-327), built on first access.

        The gfx950 kernel does not use them (one descriptor table covers every row); they are
        kept for callers that inspect the prepared object.
        """
        if self._opt_buckets is None:
            fp64 = self.data.dtype == torch.float64
            configs = _SPMV_OPT_BUCKET_CONFIGS_FP64 if fp64 else _SPMV_OPT_BUCKET_CONFIGS
            row_index_dtype = torch.int32 if self.n_rows <= _INDEX_LIMIT_INT32 else torch.int64
            lengths = self._row_lengths
            buckets = []
            lower = 0
            for upper, bs, warps, stages, batch in configs:
                if upper is None:
                    mask = lengths > lower
                    bucket_max = self.max_row_nnz
                elif lower == 0:
                    mask = lengths <= upper
                    bucket_max = upper
                else:
                    mask = (lengths > lower) & (lengths <= upper)
                    bucket_max = upper
                rows = torch.nonzero(mask, as_tuple=False).flatten()
                if rows.numel():
                    segs = (max((bucket_max + bs - 1) // bs, 1)
                            if self._user_max_segments is None else self._user_max_segments)
                    buckets.append({"rows": rows.to(row_index_dtype), "block_size": bs,
                                    "max_segs": segs, "num_warps": warps, "num_stages": stages,
                                    "batch_rows": batch})
                if upper is not None:
                    lower = upper
            self._opt_buckets = buckets
        return self._opt_buckets

    def _row_caps(self, opt):
        """Entries of each row the reference visits, or None when every row is complete."""
        lengths = self._row_lengths.to(torch.int64)
        if not opt:
            limit = max(0, int(self.max_segments)) * int(self.block_nnz)
            if self.max_row_nnz <= limit:
                return None
            return torch.clamp(lengths, max=limit)
        if self._user_max_segments is None:
            return None
        bs = _opt_bucket_block_sizes(lengths, self.data.dtype == torch.float64)
        caps = torch.minimum(lengths, bs * max(0, int(self._user_max_segments)))
        if bool(torch.equal(caps, lengths)):
            return None
        return caps

    def _kernel(self, opt):
        """The kernel layout (flagsparse_amd/_spmv_layouts.py) for the base or opt path."""
        key = "opt" if opt else "base"
        kc = self._kernels.get(key)
        if kc is not None:
            return kc
        caps = self._row_caps(opt) if self.n_rows > 0 else None
        if caps is None:
            kc = self._kernels.get("full")
            if kc is None:
                kc = build_layout(self.data, self.kernel_indices, self.kernel_indptr,
                                  self.n_cols, one_shot=self._one_shot)
                self._kernels["full"] = kc
        else:
            d, c, ip = truncate_rows(self.data, self.kernel_indices, self.kernel_indptr, caps)
            kc = build_layout(d, c, ip, self.n_cols, one_shot=self._one_shot)
        self._kernels[key] = kc
        return kc


def _prepare_spmv_csr_matrix(data, indices, indptr, shape):
    """Validation and narrowing - spmv_csr.py:379-436 (same checks, order and exceptions;
    the device-side checks are gathered into one host synchronisation)."""
    if not all(torch.is_tensor(t) for t in (data, indices, indptr)):
        raise TypeError("data, indices, indptr must all be torch.Tensor")
    if data.ndim != 1 or indices.ndim != 1 or indptr.ndim != 1:
        raise ValueError("data, indices, indptr must be 1D tensors")
    n_rows, n_cols = int(shape[0]), int(shape[1])
    if indptr.numel() != n_rows + 1:
        raise ValueError(f"indptr length must be n_rows+1={n_rows + 1}, got {indptr.numel()}")
    if data.numel() != indices.numel():
        raise ValueError("data and indices must have the same length (nnz)")
    if not all(t.is_cuda for t in (data, indices, indptr)):
        raise ValueError("data, indices, indptr must be CUDA tensors")
    if data.dtype not in SUPPORTED_VALUE_DTYPES:
        raise TypeError(
            "data dtype must be one of: float16, bfloat16, float32, float64, complex64, complex128"
        )
    if indices.dtype not in SUPPORTED_INDEX_DTYPES:
        raise TypeError("indices dtype must be torch.int32 or torch.int64")

    data = data.contiguous()
    indices = indices.contiguous()
    indptr = indptr.contiguous()
    nnz = data.numel()

    probes = []
    if indptr.numel() > 0:
        probes += [indptr[0].to(torch.int64), indptr[-1].to(torch.int64)]
        if indptr.numel() > 1:
            probes.append(torch.any(indptr[1:] < indptr[:-1]).to(torch.int64))
    if nnz > 0:
        probes += [indices.min().to(torch.int64), indices.max().to(torch.int64)]
    vals = torch.stack(probes).tolist() if probes else []
    pos = 0
    if indptr.numel() > 0:
        first, last = vals[0], vals[1]
        pos = 2
        if first != 0:
            raise ValueError("indptr must start at zero")
        if last != nnz:
            raise ValueError("indptr[-1] must equal nnz")
        if indptr.numel() > 1:
            if vals[2]:
                raise ValueError("indptr must be non-decreasing")
            pos = 3
    if nnz > 0:
        min_index, max_index = vals[pos], vals[pos + 1]
        if min_index < 0 or max_index >= n_cols:
            raise IndexError("indices out of range for n_cols")
        if max_index > _INDEX_LIMIT_INT32:
            raise ValueError(f"int64 column index {max_index} exceeds Triton int32 kernel range")
    kernel_indices = indices.to(torch.int32) if indices.dtype == torch.int64 else indices
    kernel_indptr = indptr.to(torch.int32) if nnz <= _INDEX_LIMIT_INT32 else indptr.to(torch.int64)
    row_lengths = kernel_indptr[1:] - kernel_indptr[:-1]
    max_row_nnz = int(row_lengths.max().item()) if n_rows > 0 else 0
    return data, kernel_indices, kernel_indptr, n_rows, n_cols, row_lengths, max_row_nnz


def _validate_spmv_x(x, prepared):
    """spmv_csr.py:439-452."""
    if x is None or not torch.is_tensor(x):
        raise TypeError("x must be a torch.Tensor")
    if x.ndim != 1:
        raise ValueError("x must be a 1D tensor")
    if not x.is_cuda:
        raise ValueError("x must be a CUDA tensor")
    if x.dtype != prepared.data.dtype:
        raise TypeError("x dtype must match sparse matrix dtype")
    if x.numel() != prepared.n_cols:
        raise ValueError(f"x length must be n_cols={prepared.n_cols}, got {x.numel()}")
    if x.device != prepared.data.device:
        raise ValueError("x must be on the same device as sparse matrix data")
    return x.contiguous()


def prepare_spmv_csr(data, indices, indptr, shape, block_nnz=256, max_segments=None):
    """One-time validation, narrowing and planning - spmv_csr.py:455-495."""
    return _prepare_spmv_csr(data, indices, indptr, shape, block_nnz, max_segments, False)


def _prepare_spmv_csr(data, indices, indptr, shape, block_nnz, max_segments, one_shot):
    """prepare_spmv_csr; one_shot marks a prepared object made for a single call (the layout
    that builds fastest)."""
    (data, kernel_indices, kernel_indptr, n_rows, n_cols, row_lengths,
     max_row_nnz) = _prepare_spmv_csr_matrix(data, indices, indptr, shape)
    block_nnz_use = block_nnz
    if max_segments is None:
        max_segments_use = max((max_row_nnz + block_nnz_use - 1) // block_nnz_use, 1)
        while max_segments_use > 2048 and block_nnz_use < 65536:
            block_nnz_use *= 2
            max_segments_use = max((max_row_nnz + block_nnz_use - 1) // block_nnz_use, 1)
    else:
        max_segments_use = max_segments
    prepared = PreparedCsrSpmv(data, kernel_indices, kernel_indptr, shape, n_rows, n_cols,
                               block_nnz_use, max_segments_use, max_row_nnz, row_lengths,
                               max_segments)
    prepared._one_shot = bool(one_shot)
    if prepared.supports_opt and n_rows > 0:
        prepared._kernel(False)  # build the descriptor table now, outside the timed calls
    return prepared


def _out_is_direct(out, shape, dtype, device, inputs):
    """True when the kernel may write straight into ``out``."""
    if out is None or not out.is_cuda or out.device != device or not out.is_contiguous():
        return False
    if out.data_ptr() % 16:
        return False
    base = out.untyped_storage().data_ptr()
    return all(t is None or t.untyped_storage().data_ptr() != base for t in inputs)


def _run_spmv_csr(prepared, x, opt, y):
    dtype = prepared.data.dtype
    _require_kernel_dtype(dtype, "flagsparse_spmv_csr")
    if prepared.n_rows == 0:
        return y
    acc_f64 = dtype == torch.float64 or not opt
    return prepared._kernel(opt).launch(x, y, acc_f64)


def flagsparse_spmv_csr(
    data=None,
    indices=None,
    indptr=None,
    x=None,
    shape=None,
    block_nnz=256,
    max_segments=None,
    out=None,
    return_time=False,
    use_opt=False,
    prepared=None,
):
    """CSR SpMV y = A @ x (reference signature: spmv_csr.py:557-610).

    prepared: from prepare_spmv_csr for steady-state calls.  use_opt: native-precision
    accumulation (float32 stays float32); the default sums float32 in float64.
    """
    if prepared is None:
        if any(arg is None for arg in (data, indices, indptr, shape)):
            raise ValueError(
                "data, indices, indptr, and shape are required when prepared is not provided"
            )
        prepared = _prepare_spmv_csr(data, indices, indptr, shape, block_nnz, max_segments,
                                     True)
    x = _validate_spmv_x(x, prepared)
    dtype = prepared.data.dtype
    if out is not None and (tuple(out.shape) != (prepared.n_rows,) or out.dtype != dtype):
        raise ValueError("out shape/dtype must match result")
    _require_kernel_dtype(dtype, "flagsparse_spmv_csr")
    direct = _out_is_direct(out, (prepared.n_rows,), dtype, x.device, (x, prepared.data))
    y = out if direct else torch.empty(prepared.n_rows, dtype=dtype, device=x.device)
    t0 = None
    if return_time:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
    _run_spmv_csr(prepared, x, bool(use_opt and prepared.supports_opt), y)
    elapsed_ms = None
    if return_time:
        torch.cuda.synchronize()
        elapsed_ms = (time.perf_counter() - t0) * 1000.0
    if out is not None and not direct:
        out.copy_(y)
        y = out
    if return_time:
        return y, elapsed_ms
    return y


def _coo_is_sorted_lex(row_i64, col_i64, n_cols):
    """spmv_csr.py:613-620."""
    n = row_i64.numel()
    if n <= 1:
        return True
    key = row_i64 * max(1, int(n_cols)) + col_i64
    return bool((key[1:] >= key[:-1]).all().item())


def coo_to_csr_for_spmv(data, row, col, shape, assume_sorted=False):
    """COO -> CSR (data, int32 column indices, int64 indptr) - spmv_csr.py:623-647.

    Unsorted input is sorted by (row, col) with a stable sort, which fixes the order of
    repeated (row, col) entries.
    """
    n_rows, n_cols = int(shape[0]), int(shape[1])
    row64 = row.to(torch.int64)
    col64 = col.to(torch.int64)
    if row64.numel() == 0:
        indptr = torch.zeros(n_rows + 1, dtype=torch.int64, device=data.device)
        return data, col64.to(torch.int32), indptr
    if assume_sorted or _coo_is_sorted_lex(row64, col64, n_cols):
        row_s, col_s, data_s = row64, col64, data
    else:
        key = row64 * max(1, n_cols) + col64
        order = torch.argsort(key, stable=True)
        row_s = row64[order]
        col_s = col64[order]
        data_s = data[order].to(data.dtype)
    indptr = torch.zeros(n_rows + 1, dtype=torch.int64, device=data.device)
    if data_s.numel() > 0:
        indptr[1:] = torch.cumsum(torch.bincount(row_s, minlength=n_rows), dim=0)
    return data_s, col_s.to(torch.int32), indptr


def prepare_spmv_coo_tocsr(data, row, col, shape, block_nnz=256, max_segments=None,
                           assume_sorted=False):
    """One-time COO -> CSR + plan - spmv_csr.py:650-684."""
    if not all(torch.is_tensor(t) for t in (data, row, col)):
        raise TypeError("data, row, col must all be torch.Tensor")
    if not all(t.is_cuda for t in (data, row, col)):
        raise ValueError("data, row, col must all be CUDA tensors")
    if data.ndim != 1 or row.ndim != 1 or col.ndim != 1:
        raise ValueError("data, row, col must all be 1D tensors")
    if data.dtype not in SUPPORTED_VALUE_DTYPES:
        raise TypeError(
            "data dtype must be one of: float16, bfloat16, float32, float64, complex64, complex128"
        )
    if row.numel() != col.numel() or data.numel() != row.numel():
        raise ValueError("data, row, col must have the same length")
    data_s, indices, indptr = coo_to_csr_for_spmv(data, row, col, shape,
                                                  assume_sorted=assume_sorted)
    return prepare_spmv_csr(data_s, indices, indptr, shape, block_nnz=block_nnz,
                            max_segments=max_segments)


def flagsparse_spmv_coo_tocsr(
    data=None,
    row=None,
    col=None,
    x=None,
    shape=None,
    block_nnz=256,
    max_segments=None,
    out=None,
    return_time=False,
    use_opt=True,
    prepared=None,
    assume_sorted=False,
):
    """COO SpMV through CSR conversion - spmv_csr.py:687-758 (default use_opt=True)."""
    if prepared is not None:
        if x is None:
            raise TypeError("x is required")
        if shape is None:
            shape = prepared.shape
        sh = (int(shape[0]), int(shape[1]))
        if sh != prepared.shape:
            raise ValueError(f"shape {sh} does not match prepared.shape {prepared.shape}")
        return flagsparse_spmv_csr(x=x, shape=shape, block_nnz=block_nnz,
                                   max_segments=max_segments, out=out, return_time=return_time,
                                   use_opt=use_opt, prepared=prepared)

    if not all(torch.is_tensor(t) for t in (data, row, col, x)):
        raise TypeError("data, row, col, x must all be torch.Tensor")
    if not all(t.is_cuda for t in (data, row, col, x)):
        raise ValueError("data, row, col, x must all be CUDA tensors")
    if data.ndim != 1 or row.ndim != 1 or col.ndim != 1 or x.ndim != 1:
        raise ValueError("data, row, col, x must all be 1D tensors")
    if data.dtype not in SUPPORTED_VALUE_DTYPES:
        raise TypeError(
            "data dtype must be one of: float16, bfloat16, float32, float64, complex64, complex128"
        )
    if x.dtype != data.dtype:
        raise TypeError("x dtype must match data dtype")
    data_s, indices, indptr = coo_to_csr_for_spmv(data, row, col, shape,
                                                  assume_sorted=assume_sorted)
    return flagsparse_spmv_csr(data_s, indices, indptr, x, shape, block_nnz=block_nnz,
                               max_segments=max_segments, out=out, return_time=return_time,
                               use_opt=use_opt)
