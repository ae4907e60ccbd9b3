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
    """A descriptor table on the device plus the partial-sum workspace its split rows need."""

    __slots__ = ("desc", "desc_host", "ranges", "n_desc", "n_parts", "n_split_rows", "chunk",
                 "rows_cap", "nnz_cap", "long_threshold", "_workspaces", "_groups")

    def __init__(self, desc, n_parts, n_split_rows, chunk, rows_cap, nnz_cap, long_threshold,
                 desc_host=None, ranges=None, groups=None):
        self.desc = desc
        self.desc_host = desc_host
        self.ranges = ranges
        self.n_desc = int(desc.shape[0])
        self.n_parts = int(n_parts)
        self.n_split_rows = int(n_split_rows)
        self.chunk = int(chunk)
        self.rows_cap = int(rows_cap)
        self.nnz_cap = int(nnz_cap)
        self.long_threshold = int(long_threshold)
        self._workspaces = {}
        self._groups = groups

    def workspace(self, width=1):
        """Partial-sum buffer for ``width`` values per row part, kept on the plan and reused by
        every call; the layouts that launch with it order calls from different streams
        (StreamOrder)."""
        ws = self._workspaces.get(int(width))
        if ws is None:
            n = max(self.n_parts, 1)
            ws = torch.empty(n * max(int(width), 1), dtype=torch.float64, device=self.desc.device)
            self._workspaces[int(width)] = ws
        return ws

    def split_groups(self):
        """(groups int32[g, 4], group_base int64[g], split_rows int32[g]) on the device for the
        second-pass combine of rows cut into several chunks: group {g, 1, nch, 0} adds
        partials[part .. part + nch) into that row."""
        if self._groups is None:
            d = self.desc_host
            first = (d[:, 2] > 1) & (d[:, 1] == 0)
            rows = np.ascontiguousarray(d[first, 0], dtype=np.int32)
            base = np.ascontiguousarray(d[first, 3], dtype=np.int64)
            g = rows.size
            groups = np.zeros((g, 4), dtype=np.int32)
            groups[:, 0] = np.arange(g, dtype=np.int32)
            groups[:, 1] = 1
            groups[:, 2] = d[first, 2]
            device = self.desc.device
            self._groups = (torch.from_numpy(groups).to(device), torch.from_numpy(base).to(device),
                            torch.from_numpy(rows).to(device))
        return self._groups


class StreamOrder:
    """Orders the calls that share one workspace (partial sums) across streams.

    Calls made on one stream are ordered by the stream itself.  When a call comes from a
    different stream than the previous one (or than the one the object was built on), the new
    stream first waits for everything already queued on the previous stream - an event recorded
    there at that moment - so two streams never interleave their use of the workspace.  The
    reference allocates its workspace per call (spmm_csr.py:979-983) and has no such hazard;
    here the steady state on one stream costs one comparison and allocates nothing.  The
    tensors passed are also marked as used on the new stream, so the caching allocator does
    not reuse their memory while that stream may still read them."""

    __slots__ = ("_last",)

    def __init__(self, device=None):
        self._last = _abi.raw_stream(device) if device is not None and \
            torch.device(device).type == "cuda" else None

    def stream(self, device, tensors=()):
        """The raw handle of torch's current stream on ``device``, ordered after the previous
        user's work when it differs."""
        s = _abi.raw_stream(device)
        if torch.cuda.is_current_stream_capturing():
            # A graph being captured: nothing runs now, and a wait on an event recorded
            # outside the capture cannot be recorded into it.  Replays run in the order of
            # the stream they are replayed on; ordering them against eager calls of the
            # same object on other streams is the caller's (as for the graph's inputs).
            return s
        last = self._last
        if last is not None and s != last:
            old = torch.cuda.ExternalStream(last, device=device)
            new = torch.cuda.ExternalStream(s, device=device)
            ev = torch.cuda.Event()
            ev.record(old)
            new.wait_event(ev)
            for t in tensors:
                if t is not None and t.is_cuda:
                    t.record_stream(new)
        self._last = s
        return s


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
    # entry range [lo, hi) of every descriptor, so kernels need not read row pointers first
    d = desc.astype(np.int64)
    short = d[:, 2] == 0
    lo = np.where(short, rp[d[:, 0]], rp[d[:, 0]] + d[:, 1] * int(chunk))
    hi = np.where(short, rp[np.where(short, d[:, 1], d[:, 0])],
                  np.minimum(lo + int(chunk), rp[np.minimum(d[:, 0] + 1, n_rows)]))
    ranges = np.ascontiguousarray(np.stack([lo, hi], 1), dtype=np.int64)
    desc_t = torch.from_numpy(desc)
    ranges_t = torch.from_numpy(ranges)
    if device is not None and torch.device(device).type != "cpu":
        desc_t = desc_t.to(device)
        ranges_t = ranges_t.to(device)
    return RowBlockPlan(desc_t, npart.value, nsplit.value, chunk, rows_cap, nnz_cap,
                        long_threshold, desc_host=desc, ranges=ranges_t)


def build_row_block_plan_device(rowptr, nnz_cap, rows_cap, long_threshold, chunk,
                                window_rows=None):
    """The row-block plan built on the device (fsp_plan_windows_count / _emit): rows cut into
    windows of ``window_rows`` rows (default ``rows_cap``), each planned like the host
    planner; one small device-to-host copy (the three totals) between the passes.  ``rowptr``
    is an int32 or int64 device tensor."""
    L = _abi.lib()
    dev = rowptr.device
    bits = 32 if rowptr.dtype == torch.int32 else 64
    rp = rowptr if bits == 32 else rowptr.to(torch.int64)
    rp = rp.contiguous()
    n_rows = int(rp.numel()) - 1
    window = int(rows_cap if window_rows is None else window_rows)
    args = (_abi.ptr(rp), bits, n_rows, window, int(nnz_cap), int(rows_cap), int(long_threshold),
            int(chunk))
    n_win = -(-max(n_rows, 0) // max(window, 1))
    stream = _abi.stream_handle(dev)
    counts = torch.empty((3, max(n_win, 1)), dtype=torch.int64, device=dev)
    if n_win == 0:
        counts.zero_()
    _abi.check(L.fsp_plan_windows_count(*args, _abi.ptr(counts), stream), "fsp_plan_windows_count")
    # exclusive prefix sums, one contiguous 1-D scan per counter
    incl = torch.stack([torch.cumsum(counts[k], 0) for k in range(3)])
    offsets = (incl - counts).contiguous()
    nd, n_parts, n_split = (int(v) for v in incl[:, -1].tolist())
    if max(nd, n_parts) > 0x7FFFFFFF:
        raise ValueError("row-block plan: more than 2^31-1 descriptors or partial slots")
    desc = torch.empty((nd, 4), dtype=torch.int32, device=dev)
    ranges = torch.empty((nd, 2), dtype=torch.int64, device=dev)
    groups = torch.empty((n_split, 4), dtype=torch.int32, device=dev)
    group_base = torch.empty(n_split, dtype=torch.int64, device=dev)
    split_rows = torch.empty(n_split, dtype=torch.int32, device=dev)
    _abi.check(L.fsp_plan_windows_emit(*args, _abi.ptr(offsets), _abi.ptr(desc), _abi.ptr(ranges),
                                       _abi.ptr(groups), _abi.ptr(group_base),
                                       _abi.ptr(split_rows), stream), "fsp_plan_windows_emit")
    return RowBlockPlan(desc, n_parts, n_split, chunk, rows_cap, nnz_cap, long_threshold,
                        ranges=ranges, groups=(groups, group_base, split_rows))


def build_row_block_plan_windows(rowptr, nnz_cap, rows_cap, long_threshold, chunk,
                                 window_rows):
    """The windowed row-block plan for ``rowptr`` wherever it lives: on a GPU tensor the device
    planner; on a CPU tensor the host planner run window by window (the same table - the
    device planner's contract - for host-side tests of the layouts built on it)."""
    if rowptr.is_cuda:
        return build_row_block_plan_device(rowptr, nnz_cap, rows_cap, long_threshold, chunk,
                                           window_rows)
    rp = rowptr_to_host(rowptr)
    n_rows = rp.size - 1
    window = max(int(window_rows), 1)
    tables, ranges, parts, splits = [], [], 0, 0
    for w0 in range(0, n_rows, window):
        w1 = min(w0 + window, n_rows)
        p = build_row_block_plan(rp[w0:w1 + 1] - rp[w0], None, nnz_cap, rows_cap,
                                 long_threshold, chunk)
        d = p.desc_host.astype(np.int64)
        short = d[:, 2] == 0
        d[:, 0] += w0
        d[short, 1] += w0
        d[(~short) & (d[:, 3] >= 0), 3] += parts
        tables.append(d)
        ranges.append(p.ranges.numpy() + rp[w0])
        parts += p.n_parts
        splits += p.n_split_rows
    desc = np.concatenate(tables) if tables else np.zeros((0, 4), dtype=np.int64)
    rng = np.concatenate(ranges) if ranges else np.zeros((0, 2), dtype=np.int64)
    desc32 = np.ascontiguousarray(desc, dtype=np.int32)
    return RowBlockPlan(torch.from_numpy(desc32), parts, splits, chunk, rows_cap, nnz_cap,
                        long_threshold, desc_host=desc32,
                        ranges=torch.from_numpy(np.ascontiguousarray(rng)))


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
