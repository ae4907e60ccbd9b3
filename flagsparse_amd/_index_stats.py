"""Index checks of the per-call COO paths in one device pass (fsp_index_stats in
csrc/index_stats.hip): the bounds of two index arrays and whether the first is in order."""

import torch

from . import _abi


def index_stats(a, b):
    """[min a, max a, min b, max b, number of i with a[i] < a[i-1]] as Python ints, for two
    contiguous 1-D int32/int64 device tensors of the same length (one host synchronisation)."""
    return index_stats_device(a, b).tolist()


def index_stats_device(a, b):
    """The same five values as an int64 device tensor, without synchronising."""
    L = _abi.lib()
    dev = a.device
    partial = torch.empty(int(L.fsp_index_stats_partial_len()), dtype=torch.int64, device=dev)
    out = torch.empty(5, dtype=torch.int64, device=dev)
    _abi.check(L.fsp_index_stats(_abi.ptr(a), 32 if a.dtype == torch.int32 else 64, _abi.ptr(b),
                                 32 if b.dtype == torch.int32 else 64, int(a.numel()),
                                 _abi.ptr(partial), _abi.ptr(out), _abi.stream_handle(dev)),
               "fsp_index_stats")
    return out
