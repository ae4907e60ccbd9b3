"""ctypes binding of the C ABI in include/flagsparse_hip.h.

The library is loaded after ``import torch`` so that its libamdhip64.so.7 dependency
resolves to the HIP runtime torch already loaded (same SONAME): device pointers and
``hipStream_t`` handles from torch are then valid in the library.  A missing library is an
error - there is no fallback compute path.
"""

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime first; see module docstring)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libflagsparse_hip.so")

FSP_F32 = 0
FSP_F64 = 1
ABI_VERSION = 17

_lib = None

_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f64 = ctypes.c_double

# name -> (restype, argtypes); kept in the order of include/flagsparse_hip.h.
SIGNATURES = {
    "fsp_last_error": (ctypes.c_char_p, []),
    "fsp_abi_version": (_i32, []),
    "fsp_spmv_stream_nnz_cap": (_i64, []),
    "fsp_spmv_stream_rows_cap": (_i64, []),
    "fsp_spmv_chunk_nnz_cap": (_i64, []),
    "fsp_spmm_block_nnz_cap": (_i64, []),
    "fsp_xcs_item_cap": (_i64, []),
    "fsp_xcs_rows_cap": (_i64, []),
    "fsp_xcs_window_slots_cap": (_i64, []),
    "fsp_xcs_window_rows_cap": (_i64, []),
    "fsp_xcs_item_runs_cap": (_i64, []),
    "fsp_xcs_sorted_item_cap": (_i64, []),
    "fsp_xcs_sorted_col_bits": (_i64, []),
    "fsp_panel_bytes_cap": (_i64, []),
    "fsp_panel_chunk": (_i64, []),
    "fsp_panel_chunk_runs_cap": (_i64, []),
    "fsp_stage_window_cap": (_i64, []),
    "fsp_stage_window_rows_cap": (_i64, []),
    "fsp_stage_chunk": (_i64, []),
    "fsp_plan_panel_chunks": (_i32, [_p, _i64, _p, _i64, _i64, _p, _p]),
    "fsp_plan_panel_chunks_device": (_i32, [_p, _i64, _p, _i64, _i64, _p, _p, _p]),
    "fsp_plan_row_blocks": (_i32, [_p, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p]),
    "fsp_spmv_csr": (_i32, [_i32, _i32, _p, _p, _p, _i32, _i64, _i64, _p, _p, _p, _i64, _p, _p,
                            _i64, _i64, _p, _p, _p, _p, _i64, _i32, _p]),
    "fsp_spmv_scratch_slots": (_i64, []),
    "fsp_spmv_csr_static": (_i32, [_i32, _i32, _p, _p, _p, _i32, _i64, _i64, _p, _p, _p, _i64, _p,
                                   _p, _i64, _i64, _i64, _p, _p, _p, _i64, _i32, _p]),
    "fsp_spmv_xcs": (_i32, [_i32, _i32, _p, _p, _i64, _i32, _p, _p, _p, _i64, _p, _i64, _p, _p,
                            _p, _i64, _i64, _p, _p, _i32, _p]),
    "fsp_spmv_panels": (_i32, [_i32, _i32, _p, _p, _i64, _i32, _p, _i64, _p, _p, _p, _p, _i64,
                               _p, _p, _i64, _p, _p, _p, _i64, _p, _i64, _p, _p, _p, _p, _i64,
                               _p]),
    "fsp_spmv_stage_combine": (_i32, [_i32, _i32, _p, _p, _i64, _p, _i64, _i64, _p, _p, _p,
                                      _i64, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "fsp_spmv_hybrid_combine": (_i32, [_i32, _i32, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p,
                                       _p, _p, _i64, _p]),
    "fsp_spmv_coo_atomic": (_i32, [_i32, _p, _p, _p, _i64, _p, _p, _i64, _i64, _p]),
    "fsp_spmm_csr": (_i32, [_i32, _i32, _p, _p, _p, _i32, _i64, _i64, _p, _i64, _i64, _p, _i64, _p,
                            _i64, _i64, _i32, _i32, _p, _p, _p, _p, _i64, _i32, _p]),
    "fsp_index_stats": (_i32, [_p, _i32, _p, _i32, _i64, _p, _p, _p]),
    "fsp_index_stats_partial_len": (_i64, []),
    "fsp_spmm_coo_atomic": (_i32, [_i32, _i32, _p, _p, _p, _i64, _p, _i64, _i64, _p, _i64, _i64,
                                   _p]),
    "fsp_plan_windows_count": (_i32, [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p]),
    "fsp_plan_windows_emit": (_i32, [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p,
                                     _p, _p, _p]),
    "fsp_mtx_read": (_i32, [ctypes.c_char_p, _p, _p, _p, _p, _i64]),
    "fsp_sddmm_csr": (_i32, [_i32, _i32, _i32, _p, _p, _p, _i32, _i64, _p, _i64, _p, _i64, _i64,
                             _p, _f64, _f64, _p, _p, _p, _i64, _i32, _i32, _p]),
    "fsp_probe_gather_blocks": (_i64, [_i64]),
    "fsp_probe_gather": (_i32, [_p, _i64, _p, _i64, _p, _p]),
    "fsp_probe_rows_blocks": (_i64, [_i64]),
    "fsp_probe_rows": (_i32, [_p, _i64, _i64, _p, _i64, _p, _p]),
    "fsp_probe_stream_blocks": (_i64, [_i64]),
    "fsp_probe_stream": (_i32, [_p, _i64, _p, _p]),
}


class HipLibraryError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def lib():
    """The loaded library (loaded on first use)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"flagsparse_amd HIP library not found at {LIB_PATH}; build it with "
                "`python -m flagsparse_amd._build` (there is no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        version = handle.fsp_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libflagsparse_hip.so ABI {version}, expected {ABI_VERSION}; rebuild")
        _lib = handle
    return _lib


def check(status, what):
    if status != 0:
        msg = lib().fsp_last_error().decode(errors="replace")
        raise HipLibraryError(f"{what} failed (status {status}): {msg}")


def dtype_code(dtype):
    if dtype == torch.float32:
        return FSP_F32
    if dtype == torch.float64:
        return FSP_F64
    raise TypeError(f"no gfx950 kernel for value dtype {dtype}")


def ptr(t):
    """Device (or host) address of a tensor's first element; None for absent tensors."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device):
    """hipStream_t of torch's current stream on ``device``."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_current_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def raw_stream(device):
    """The same handle as an int, through torch's C accessor when it exists (a few hundred ns
    instead of building a Stream object) - for per-call launch paths."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _current_raw_stream is not None:
        return _current_raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


def caps():
    """Kernel capacities compiled into the library."""
    L = lib()
    return {
        "spmv_stream_nnz": int(L.fsp_spmv_stream_nnz_cap()),
        "spmv_stream_rows": int(L.fsp_spmv_stream_rows_cap()),
        "spmv_chunk_nnz": int(L.fsp_spmv_chunk_nnz_cap()),
        "spmm_block_nnz": int(L.fsp_spmm_block_nnz_cap()),
        "xcs_item": int(L.fsp_xcs_item_cap()),
        "xcs_rows": int(L.fsp_xcs_rows_cap()),
        "xcs_window_slots": int(L.fsp_xcs_window_slots_cap()),
        "xcs_window_rows": int(L.fsp_xcs_window_rows_cap()),
        "xcs_item_runs": int(L.fsp_xcs_item_runs_cap()),
        "xcs_sorted_item": int(L.fsp_xcs_sorted_item_cap()),
        "xcs_sorted_col_bits": int(L.fsp_xcs_sorted_col_bits()),
        "panel_bytes": int(L.fsp_panel_bytes_cap()),
        "panel_chunk": int(L.fsp_panel_chunk()),
        "panel_chunk_runs": int(L.fsp_panel_chunk_runs_cap()),
        "stage_window": int(L.fsp_stage_window_cap()),
        "stage_window_rows": int(L.fsp_stage_window_rows_cap()),
        "stage_chunk": int(L.fsp_stage_chunk()),
    }
