"""COO SpMV y = A @ x on gfx950 without an indptr over all rows.

Public API mirrors ``src/flagsparse/sparse_operations/spmv_coo.py``: ``PreparedCoo``
(:19-48), ``prepare_spmv_coo`` (:220-225) and ``flagsparse_spmv_coo`` (:284-348).

* ``sort_by_row=True``: entries sorted by (row, col) (skipped when already sorted), constant-row
  runs ``seg_starts`` (:167-179); one sum per run, rows without a run are 0.  The runs are fed
  to the same row-block kernel as CSR SpMV with a run -> row map (identity, and then omitted,
  when every row has entries).
* ``sort_by_row=False``: one atomic add per entry into a zeroed y (:111-150); the summation
  order, and so the last bits of y, vary from call to call, as in the reference.
"""

import time

import torch

from . import _abi
from ._common import _INDEX_LIMIT_INT32
from ._spmv_layouts import build_layout


class PreparedCoo:
    """Sorted COO + optional row-run bounds ``seg_starts``; no CSR indptr (spmv_coo.py:19-48)."""

    __slots__ = (
        "data",
        "row",
        "col",
        "shape",
        "n_rows",
        "n_cols",
        "nnz",
        "seg_starts",
        "n_segs",
        "use_seg_kernel",
        "_run_rows",
        "_layout",
        "_one_shot",
    )

    def __init__(self, data, row, col, shape, seg_starts=None):
        self.data = data
        self.row = row
        self.col = col
        self.shape = (int(shape[0]), int(shape[1]))
        self.n_rows, self.n_cols = self.shape
        self.nnz = int(data.numel())
        self.seg_starts = seg_starts
        if seg_starts is None:
            self.n_segs = 0
            self.use_seg_kernel = False
        else:
            self.n_segs = int(seg_starts.numel()) - 1
            self.use_seg_kernel = self.n_segs > 0
        self._run_rows = None
        self._layout = None
        self._one_shot = False

    def _run_layout(self):
        """Kernel layout over the row runs (flagsparse_amd/_spmv_layouts.py) and the
        run -> row map, omitted when it is the identity."""
        if self._layout is None:
            self._layout = build_layout(self.data, self.col, self.seg_starts, self.n_cols,
                                        one_shot=self._one_shot)
            if self.n_segs == self.n_rows:
                self._run_rows = None  # sorted and every row present: run k is row k
            else:
                self._run_rows = self.row[self.seg_starts[:-1].to(torch.int64)].to(torch.int32)
        return self._layout

    def _kernel_name(self):
        if self.use_seg_kernel:
            return self._run_layout().kernel_name()
        return "spmv_coo_atomic_kernel"

    def _kernel_plan_description(self):
        if self.use_seg_kernel:
            return self._run_layout().describe()
        return {"layout": "atomic"}


def _sort_coo_lex_inplace(data, row, col, n_cols):
    """Lexicographic (row, col) order - spmv_coo.py:153-164.  Already-sorted input is kept
    as is (one O(nnz) check instead of a sort); otherwise a stable argsort."""
    row64 = row.to(torch.int64)
    col64 = col.to(torch.int64)
    if data.numel() == 0:
        return data.contiguous(), row64, col64
    key = row64 * max(1, int(n_cols)) + col64
    if data.numel() > 1 and bool((key[1:] >= key[:-1]).all().item()):
        return data.contiguous(), row64.contiguous(), col64.contiguous()
    order = torch.argsort(key, stable=True)
    return data[order].contiguous(), row64[order].contiguous(), col64[order].contiguous()


def _seg_starts_from_sorted_rows(row_sorted, nnz, device):
    """Boundaries of constant-row runs in sorted COO - spmv_coo.py:167-179 (int32, or int64
    past the int32 range)."""
    if nnz == 0:
        return None
    idx_dtype = torch.int32 if nnz <= _INDEX_LIMIT_INT32 else torch.int64
    diff = row_sorted[1:] != row_sorted[:-1]
    breaks = torch.nonzero(diff, as_tuple=False).flatten().to(idx_dtype) + 1
    return torch.cat([
        torch.zeros(1, dtype=idx_dtype, device=device),
        breaks,
        torch.tensor([nnz], dtype=idx_dtype, device=device),
    ])


def _prepare_coo_tensors(data, row, col, shape, sort_by_row):
    """spmv_coo.py:182-217 (same checks, order and exceptions)."""
    if not all(torch.is_tensor(t) for t in (data, row, col)):
        raise TypeError("data, row, col must all be torch.Tensor")
    if data.ndim != 1 or row.ndim != 1 or col.ndim != 1:
        raise ValueError("data, row, col must be 1D")
    if not all(t.is_cuda for t in (data, row, col)):
        raise ValueError("data, row, col must be CUDA tensors")
    n_rows, n_cols = int(shape[0]), int(shape[1])
    if data.numel() != row.numel() or data.numel() != col.numel():
        raise ValueError("data, row, col must have the same length")
    if data.dtype not in (torch.float32, torch.float64):
        raise TypeError(
            "this COO SpMV path supports float32/float64 only (use CSR for other dtypes)"
        )
    if sort_by_row:
        data, row64, col64 = _sort_coo_lex_inplace(data, row, col, n_cols)
        seg = _seg_starts_from_sorted_rows(row64, data.numel(), data.device)
    else:
        data = data.contiguous()
        row64 = row.to(torch.int64).contiguous()
        col64 = col.to(torch.int64).contiguous()
        seg = None
    if data.numel() > 0:
        rmin, rmax, cmin, cmax = torch.stack(
            [row64.min(), row64.max(), col64.min(), col64.max()]).tolist()
        if rmin < 0 or rmax >= n_rows:
            raise IndexError("row indices out of range")
        if cmin < 0 or cmax >= n_cols:
            raise IndexError("col indices out of range")
        if rmax > _INDEX_LIMIT_INT32 or cmax > _INDEX_LIMIT_INT32:
            raise ValueError("indices exceed int32 Triton kernel range")
    return data, row64.to(torch.int32), col64.to(torch.int32), seg


def prepare_spmv_coo(data, row, col, shape, sort_by_row=True):
    """Cache sorted COO + row-run ``seg_starts`` when ``sort_by_row`` (spmv_coo.py:220-225)."""
    return _prepare_spmv_coo(data, row, col, shape, sort_by_row, False)


def _prepare_spmv_coo(data, row, col, shape, sort_by_row, one_shot):
    """prepare_spmv_coo; one_shot: for a single call (the layout that builds fastest)."""
    d, kr, kc, seg = _prepare_coo_tensors(data, row, col, shape, sort_by_row)
    prepared = PreparedCoo(d, kr, kc, shape, seg_starts=seg)
    prepared._one_shot = bool(one_shot)
    if prepared.use_seg_kernel:
        prepared._run_layout()
    return prepared


def _validate_x_coo(x, prepared):
    """spmv_coo.py:228-243."""
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


def _run_spmv_coo(prepared, x, y, block_size):
    dtype = prepared.data.dtype
    L = _abi.lib()
    stream = _abi.stream_handle(y.device)
    if prepared.nnz == 0:
        y.zero_()
        return y
    if prepared.use_seg_kernel:
        layout = prepared._run_layout()
        acc_f64 = dtype == torch.float64
        return layout.launch(x, y, acc_f64, row_map=prepared._run_rows, n_out=prepared.n_rows)
    _abi.check(
        L.fsp_spmv_coo_atomic(_abi.dtype_code(dtype), _abi.ptr(prepared.data),
                              _abi.ptr(prepared.row), _abi.ptr(prepared.col), prepared.nnz,
                              _abi.ptr(x), _abi.ptr(y), prepared.n_rows, int(block_size), stream),
        "fsp_spmv_coo_atomic")
    return y


def flagsparse_spmv_coo(
    data=None,
    row=None,
    col=None,
    x=None,
    shape=None,
    out=None,
    return_time=False,
    prepared=None,
    sort_by_row=True,
    block_size=256,
    num_warps=4,
    block_inner=128,
):
    """COO SpMV with no CSR indptr (spmv_coo.py:284-348).

    ``block_inner`` (row-run tile) and ``num_warps`` are validated as in the reference; the
    gfx950 kernels choose their own tiling.  ``block_size``: entries per workgroup of the
    atomic route (``sort_by_row=False``).
    """
    if prepared is None:
        if any(a is None for a in (data, row, col, x, shape)):
            raise ValueError("data, row, col, x, shape required when prepared is None")
        prepared = _prepare_spmv_coo(data, row, col, shape, sort_by_row, True)
    else:
        if x is None:
            raise TypeError("x is required when prepared is set")
        if shape is None:
            shape = prepared.shape
        sh = (int(shape[0]), int(shape[1]))
        if sh != prepared.shape:
            raise ValueError(f"shape {sh} does not match prepared.shape {prepared.shape}")
    x = _validate_x_coo(x, prepared)
    if num_warps not in (1, 2, 4, 8, 16, 32):
        raise ValueError("num_warps must be a power of 2 in [1, 32]")
    if block_inner <= 0 or (block_inner & (block_inner - 1)) != 0:
        raise ValueError("block_inner must be a positive power of 2")
    if not prepared.use_seg_kernel and prepared.nnz > 0 and int(block_size) <= 0:
        raise ValueError("block_size must be positive")
    dtype = prepared.data.dtype
    if out is not None and (tuple(out.shape) != (prepared.n_rows,) or out.dtype != dtype):
        raise ValueError("out shape/dtype must match result")
    direct = (out is not None and out.is_cuda and out.device == x.device and out.is_contiguous()
              and out.untyped_storage().data_ptr() not in (
                  x.untyped_storage().data_ptr(), prepared.data.untyped_storage().data_ptr()))
    y = out if direct else torch.empty(prepared.n_rows, dtype=dtype, device=x.device)
    t0 = None
    if return_time:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
    _run_spmv_coo(prepared, x, y, block_size)
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
