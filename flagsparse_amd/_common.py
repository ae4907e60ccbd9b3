"""Shared dtypes, tolerances and helpers (mirrors sparse_operations/_common.py)."""

import time

import torch

# Same tables as _common.py:22-31 of the reference.  The gfx950 kernels cover float32 and
# float64; the other value dtypes pass validation like in the reference and then raise
# NotImplementedError at the kernel boundary.
SUPPORTED_VALUE_DTYPES = (
    torch.float16,
    torch.bfloat16,
    torch.float32,
    torch.float64,
    torch.complex64,
    torch.complex128,
)
SUPPORTED_INDEX_DTYPES = (torch.int32, torch.int64)
KERNEL_VALUE_DTYPES = (torch.float32, torch.float64)
_INDEX_LIMIT_INT32 = 2**31 - 1
# The largest entry count for which the kernels read 32-bit row pointers (above it, 64-bit);
# read at prepare time, so tests can lower it to run the 64-bit row-pointer kernels on small
# matrices.
ROWPTR32_MAX_NNZ = _INDEX_LIMIT_INT32


# CuPy / cuSPARSE: the reference compares against them when they import (_common.py:14-19),
# and its scripts skip those comparisons when ``cp`` is None.  This build has no CuPy: the
# module handles exist for those scripts, and the converters say so.
cp = None
cpx_sparse = None


def _require_cupy():
    raise RuntimeError("CuPy is not available in the flagsparse_amd build (the cuSPARSE "
                       "comparison is skipped when cp is None)")


def _cupy_from_torch(tensor):
    _require_cupy()


def _torch_from_cupy(array):
    _require_cupy()


def _is_complex_dtype(value_dtype):
    return value_dtype in (torch.complex64, torch.complex128)


def _tolerance_for_dtype(value_dtype):
    """(atol, rtol) - _common.py:76-85."""
    if value_dtype == torch.float16:
        return 2e-3, 2e-3
    if value_dtype == torch.bfloat16:
        return 1e-1, 1e-1
    if value_dtype in (torch.float32, torch.complex64):
        return 1e-6, 1e-5
    if value_dtype in (torch.float64, torch.complex128):
        return 1e-10, 1e-8
    return 1e-6, 1e-5


def _require_kernel_dtype(dtype, what):
    if dtype not in KERNEL_VALUE_DTYPES:
        raise NotImplementedError(
            f"{what}: value dtype {dtype} is accepted by the reference but has no gfx950 kernel "
            "in flagsparse_amd (float32 and float64 are supported)")


def _aligned(t, align=16):
    """``t`` itself when its data pointer is ``align``-byte aligned, else an aligned copy."""
    if t.numel() == 0 or t.data_ptr() % align == 0:
        return t
    out = torch.empty_like(t, memory_format=torch.contiguous_format)
    out.copy_(t)
    return out


def _benchmark_cuda_op(op, warmup, iters):
    """Host-timed loop with device syncs - _common.py:286-304."""
    warmup = max(0, int(warmup))
    iters = max(1, int(iters))
    output = None
    for _ in range(warmup):
        output = op()
    torch.cuda.synchronize()
    start_time = time.perf_counter()
    for _ in range(iters):
        output = op()
    torch.cuda.synchronize()
    elapsed_ms = (time.perf_counter() - start_time) * 1000.0 / iters
    return output, elapsed_ms
