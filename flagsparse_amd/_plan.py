"""Row-block descriptor tables for the gfx950 kernels (host planner in the C library).

One table of int32 quadruples drives a single kernel launch; it replaces the reference's
per-bucket row lists (spmv_csr.py:281-327, spmm_csr.py:444-477) and its host loop over long
rows (spmm_csr.py:417-441):

  {r0, r1, 0, 0}          short-row block: rows [r0, r1)
  {row, k, nch, part}     chunk k of a row split into nch chunks; chunk sums of rows with
                          nch > 1 go to partial slots part .. part+nch-1
"""

import ctypes

import numpy as np
import torch

from . import _abi


class RowBlockPlan:
    """A descriptor table on the device plus the zeroed workspace its split rows need."""

    __slots__ = ("desc", "n_desc", "n_parts", "n_split_rows", "chunk", "rows_cap", "nnz_cap",
                 "long_threshold", "_workspaces")

    def __init__(self, desc, n_parts, n_split_rows, chunk, rows_cap, nnz_cap, long_threshold):
        self.desc = desc
        self.n_desc = int(desc.shape[0])
        self.n_parts = int(n_parts)
        self.n_split_rows = int(n_split_rows)
        self.chunk = int(chunk)
        self.rows_cap = int(rows_cap)
        self.nnz_cap = int(nnz_cap)
        self.long_threshold = int(long_threshold)
        self._workspaces = {}

    def workspace(self, width=1, tiles=1):
        """(partials, tickets) for ``width`` values per part and ``tiles`` tickets per part.

        Kept on the plan and reused by every call: the kernels leave the tickets at zero.
        Calls that share a plan must therefore not run concurrently on different streams.
        """
        key = (int(width), int(tiles))
        ws = self._workspaces.get(key)
        if ws is None:
            device = self.desc.device
            n = max(self.n_parts, 1)
            partials = torch.empty(n * max(int(width), 1), dtype=torch.float64, device=device)
            tickets = torch.zeros(n * max(int(tiles), 1), dtype=torch.int32, device=device)
            ws = (partials, tickets)
            self._workspaces[key] = ws
        return ws


def rowptr_to_host(rowptr):
    """int64 numpy copy of a (device) offsets tensor."""
    return np.ascontiguousarray(rowptr.detach().to("cpu", torch.int64).numpy())


def build_row_block_plan(rowptr_host, device, nnz_cap, rows_cap, long_threshold, chunk):
    """Run the greedy planner (fsp_plan_row_blocks) and upload the table to ``device``."""
    L = _abi.lib()
    rp = np.ascontiguousarray(rowptr_host, dtype=np.int64)
    n_rows = rp.size - 1
    nd, npart, nsplit = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    args = (rp.ctypes.data_as(ctypes.c_void_p), n_rows, int(nnz_cap), int(rows_cap),
            int(long_threshold), int(chunk))
    _abi.check(L.fsp_plan_row_blocks(*args, None, ctypes.byref(nd), ctypes.byref(npart),
                                     ctypes.byref(nsplit)), "fsp_plan_row_blocks (count)")
    desc = np.empty((nd.value, 4), dtype=np.int32)
    _abi.check(L.fsp_plan_row_blocks(*args, desc.ctypes.data_as(ctypes.c_void_p), ctypes.byref(nd),
                                     ctypes.byref(npart), ctypes.byref(nsplit)),
               "fsp_plan_row_blocks")
    desc_t = torch.from_numpy(desc)
    if device is not None and torch.device(device).type != "cpu":
        desc_t = desc_t.to(device)
    return RowBlockPlan(desc_t, npart.value, nsplit.value, chunk, rows_cap, nnz_cap,
                        long_threshold)


def truncate_rows(data, indices, indptr, caps):
    """Keep the first caps[r] entries of every row r (device-side).  Returns new CSR arrays
    with indptr int64.  Used for the reference's max_segments truncation."""
    n_rows = indptr.numel() - 1
    ip = indptr.to(torch.int64)
    lengths = ip[1:] - ip[:-1]
    caps = torch.minimum(lengths, caps.to(torch.int64).clamp(min=0))
    row_of = torch.repeat_interleave(torch.arange(n_rows, device=ip.device), lengths)
    pos = torch.arange(data.numel(), device=ip.device, dtype=torch.int64) - ip[row_of]
    keep = pos < caps[row_of]
    new_ip = torch.zeros(n_rows + 1, dtype=torch.int64, device=ip.device)
    new_ip[1:] = torch.cumsum(caps, 0)
    return data[keep].contiguous(), indices[keep].contiguous(), new_ip
