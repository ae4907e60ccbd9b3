"""Kernel-facing layouts of a CSR matrix for SpMV (CSR SpMV and COO row runs).

The layouts below, chosen once per matrix at prepare time:

``RowBlockLayout`` (csrc/spmv.hip, ``spmv_rowblock_kernel``)
    The CSR arrays as given plus a descriptor table: short-row blocks of <= 1021 entries and
    <= 1024 rows, and long rows cut into chunks of <= 4093 entries whose sums are added in
    chunk order.  Right when the x entries a block gathers lie close together (banded,
    stencil, locally clustered columns) or x fits in one XCD's L2.

``XcsLayout`` (csrc/spmv_xcs.hip, ``spmv_xcs_kernel``, ``xcs_window_combine_kernel``)
    Columns split into panels of about equal nnz (P of them, P / 8 per XCD in turn, or shared
    by two XCDs when P = 4); entries regrouped by (row tile, panel) so that every workgroup
    gathers from one panel only, and that panel is resident in its XCD's L2.  Right when
    columns are spread over an x larger than an L2 (uniform random columns, power-law graphs).
    Each row's partial sums (one per workgroup holding entries of it) are added by a second
    launch over windows of consecutive rows, in a fixed order (deterministic).

``PanelLayout`` (csrc/spmv_xcs.hip, ``spmv_panel_kernel``)
    The long rows of a power-law matrix: x cut into panels of 128 KiB, the rows' entries ordered
    by (panel, row); a workgroup copies one panel into LDS and its waves gather from there, so
    these gathers run at LDS speed instead of the L2 request rate.  One partial per (row,
    chunk of 512 entries; a chunk holds at most 64 rows), added per row in a fixed order.

``XcsHybridLayout``
    ``PanelLayout`` for the rows long enough to put several entries in every panel,
    ``XcsLayout`` for the others; both parts run one after the other on the caller's stream.

``XstageLayout`` (csrc/spmv_xcs.hip: ``spmv_panel_kernel`` + ``stage_combine_kernel``)
    The default where columns are spread over an x larger than an L2: the long rows as in
    ``PanelLayout``, and for the other rows the panel jobs also *stage* x - entry e of panel p
    gets xs[e] = x[its column], read from the same LDS copy of the panel - so no entry gathers
    from L2.  A second launch takes windows of consecutive rows: each entry's value times its
    staged x, placed in LDS in (row, panel) order, and each row's products summed in that
    fixed order (deterministic), beside the long rows' partial sums.

Both replace the reference's per-bucket launches (spmv_csr.py:281-376) and produce the same
row sums up to floating-point summation order.
"""

import numpy as np
import torch

from . import _abi
from . import _common
from ._common import _INDEX_LIMIT_INT32, _aligned
from ._plan import StreamOrder, build_row_block_plan_windows

XCD_COUNT = 8
L2_BYTES = 4 << 20
# Bytes of x one panel may span: leaves room in the 4 MiB L2 for the entry stream.  More
# panels also split more rows (more partial slots), so this is a balance measured on MI355X:
# 8.4 MB of x (2M fp32 columns, cfg4) runs best as 4 panels each shared by 2 XCDs (231 us vs
# 243 us as 8), 33.5 MB (8M columns) as 16.
PANEL_BYTES = 3 << 20
MIN_PANELS = 4
# A column counts as "near" its row when within this many columns of the row's position on
# the diagonal; the row-block layout is kept when most entries are near (x reuse in L2).
NEAR_COLUMNS = 1 << 16
SAMPLE = 1 << 20

# Test hooks: layout (None: choose per matrix, "rowblock", "xstage", "xcs" - hybrid when the
# long rows qualify -, "xcs-l2" - never hybrid - or "xcs-hybrid" - hybrid whenever there is a
# long row); panels per XCD (None: from the size of x).
FORCE = None
# Matrices whose columns are spread over an x larger than an L2 take the staged-x layout
# (False: the XCS layouts).  Measured on MI355X, cfg3's short rows (26.4M entries, both passes):
# 123 us staged against 161 us as XCS items and their combine.
STAGED = True
# Jobs the staged entries of a matrix are cut into, about (one per CU of the MI355X: a job
# copies its x panel into LDS once, so more jobs copy more), of at least STAGE_JOB_MIN entries
# (whose columns and staged values are about as many bytes as the panel copy).  Measured on
# MI355X, cfg4 (64 panels, staged entries only) with about 192 / 256 / 384 / 512 jobs: panel
# pass 75.7 / 59.4 / 77.3 / 66.6 us - the jobs, one workgroup per CU, run in whole rounds.
STAGE_JOBS = 256
STAGE_JOB_MIN = 16384
# Segments of a window in the order of the XCDs whose jobs stage them (test hook: False = panel
# order): measured on MI355X, cfg3's panel kernel 128.4 against 135.6 us in panel order.
STAGE_XCD_ORDER = True
STAGE_SEGMENT_MIN = 32
FORCE_STAGE_WINDOW = None  # test hook: the staged-x window size
# Row-block SpMV launches in hardware order (workgroup i on XCD i % 8): on MI355X this streamed
# faster than one contiguous descriptor range per XCD (cfg2 60.5 vs 64.7 us, cfg1 9.7 vs 12.0
# us; banded and power-law matrices within 1%).
XCD_REMAP_ROWBLOCK = 0
FORCE_PANELS_PER_XCD = None
# Plans are built on the device in windows of this many times the block row cap (one thread
# per window; a block never crosses a window end, so this bounds the blocks cut short to one
# per window - about 2.5 % more blocks on a 5-point stencil - while keeping thousands of
# threads busy on large matrices).
PLAN_WINDOW_BLOCKS = 16
# Launch order for banded / stencil matrices (band_launch_order): on for row blocks; chain
# segments of BAND_SEGMENT blocks share an XCD.  Measured on MI355X, cfg2 (5-point stencil,
# far diagonals 5 blocks away): 58.9 us in hardware order, 57.0 us with segments of 3-4
# (57.7 with 2, 57.3 with 6), L2 fill traffic 379 -> 333 MB per launch.
BAND_ORDER = True
BAND_SEGMENT = 4
BAND_MIN_SHARE = 0.2
# Panel layout: chunks per job at most (a job copies its panel of x into LDS once), and the
# long-row rule of the hybrid - rows with at least PANEL_RUNS entries per x panel go to the
# panel layout when they hold at least PANEL_MIN_SHARE of the entries.  Measured on MI355X
# for cfg3 with 128 KiB panels (256 of them; whole path): PANEL_RUNS 1 / 2 / 3 / 4 / 8 (rows
# >= 256 / 512 / 768 / 1024 / 2048 entries) 0.302 / 0.289 / 0.289 / 0.290 / 0.309 ms with
# 1024 chunks per job, 4 with 256 / 512 chunks per job 0.294 / 0.293 ms; with the current
# kernels (both second passes in one launch) rows >= 512 / 640 / 768 / 1024 entries 267.6 /
# 266.7 / 267.5 / 268.1 us: each row moved to the panels saves its gathers (the XCS kernel
# 139.5 -> 128.1 us at 640) and adds a partial sum per panel (the panel kernel 88.7 -> 94.7
# us, the combine +1.6 us).
PANEL_JOB_CHUNKS = 1024
# The XCS + panel hybrid launches the panel part's first pass before the XCS part's (False:
# after it); both second passes then run in one launch.
HYBRID_PANEL_FIRST = False
PANEL_RUNS = 2.5
PANEL_MIN_SHARE = 0.25
FORCE_PANEL_ROW_MIN = None
# Combine windows of the XCS layout: consecutive rows with at most this many partial slots
# (32 KiB of fp64 sums in LDS) and rows.
WINDOW_SLOTS = 4096
WINDOW_ROWS = 2048
# Sums of one row in a combine window at most (the combine reads one byte per row); a row
# with more is a window of its own.  The byte value ROW_SKIP marks a row the window leaves
# alone (the hybrid's long rows, written by the panel rows of the same launch).
ROW_COUNT_MAX = 254
ROW_SKIP = 255
# Stored runs of partial sums (one item's sums in one window) start on a multiple of this many
# slots: 128 bytes of fp64 sums, a cache line.
RUN_ALIGN = 16
# Every combine window's stored range starts on a multiple of this many slots (a line).
WINDOW_ALIGN = 16
# XCS items with sorted gathers (item format 1, spmv_xcs_sorted_kernel): up to 4096 entries
# per item, the gathers issued in column order so that the lanes of one instruction reach
# neighbouring lines; used when the panels need at most 19 column bits.  Tiles of up to
# SORTED_TILE_ROWS rows (rows are not packed into the entries).
SORTED_ITEMS = True
SORTED_TILE_ROWS = 16384
# A tile holds up to this many items' worth of entries per panel, so that its pieces split
# into nearly full items (tiles of one item per panel left pieces just over 4096 entries as
# two half items: cfg4 items of 2771 entries on average, 3856 here; 203.9 -> 199.4 us a call,
# 2 and 4 in between).
SORTED_TILE_ITEMS = 8
# ... for matrices whose rows put at least this many entries, on average, into each panel they
# reach.  Measured on MI355X: cfg4 (rows of 21 entries over 4 panels, 5.3 per panel) 193 ->
# 186 us in the XCS kernel; cfg3's short rows (2.0 per panel: most rows put one entry into
# each panel they reach, so most entries are row runs of their own) 142 us with row-order
# items, 144-155 us with sorted ones for tiles of 6144 to 16384 rows; with sorted items of
# 2048 entries in workgroups of 256 (the row-order items' tiles and sizes, results
# bit-identical) 130.5 us against 126.7 us - the LDS permutation back to row order costs more
# than the sorted gathers save.
SORTED_MIN_RUN = 3.0


class RowBlockLayout:
    """CSR arrays (16-byte aligned) and the row-block descriptor plan."""

    kind = "rowblock"

    def __init__(self, data, cols, rowptr, window_rows=None):
        self.data = _aligned(data)
        self.cols = _aligned(cols)
        nnz = int(data.numel())
        if nnz <= _common.ROWPTR32_MAX_NNZ:
            self.rowptr, self.rowptr_bits = rowptr.to(torch.int32).contiguous(), 32
        else:
            self.rowptr, self.rowptr_bits = rowptr.to(torch.int64).contiguous(), 64
        self.nnz = nnz
        self.n_rows = int(rowptr.numel()) - 1
        caps = _abi.caps()
        rows_cap = caps["spmv_stream_rows"]
        window = PLAN_WINDOW_BLOCKS * rows_cap if window_rows is None else int(window_rows)
        self.plan = build_row_block_plan_windows(self.rowptr, caps["spmv_stream_nnz"], rows_cap,
                                                 caps["spmv_stream_nnz"], caps["spmv_chunk_nnz"],
                                                 window)
        self.band_offset = None
        if BAND_ORDER and self.plan.desc.is_cuda and self.plan.n_desc >= 8 * BAND_SEGMENT * 4:
            off = band_block_offset(self.cols, self.rowptr, self.plan.n_desc)
            if off is not None:
                order = band_launch_order(self.plan.n_desc, off, self.plan.desc.device)
                self.plan.desc = self.plan.desc[order].contiguous()
                self.plan.ranges = self.plan.ranges[order].contiguous()
                self.band_offset = off
        self._args = {}
        self._keep = None
        self._order = StreamOrder(self.data.device)

    def kernel_name(self):
        return "spmv_rowblock_kernel"

    def held_bytes(self, caller=()):
        """Device bytes this layout holds beyond the caller's arrays ``caller``."""
        plan = self.plan
        mine = [plan.desc, plan.ranges, plan.workspace(), *plan.split_groups(), self.data,
                self.cols, self.rowptr]
        theirs = {t.untyped_storage().data_ptr() for t in caller if isinstance(t, torch.Tensor)}
        return tensor_bytes(*[t for t in mine if t.untyped_storage().data_ptr() not in theirs])

    def describe(self):
        return {"layout": self.kind, "descriptors": self.plan.n_desc,
                "split_rows": self.plan.n_split_rows, "partials": self.plan.n_parts,
                "band_block_offset": self.band_offset}

    def launch(self, x, y, acc_f64, row_map=None, n_out=0):
        # The arguments that do not change between calls are converted once (per accumulation
        # mode); a call fills in x, y, the row map and the stream.
        args = self._args.get(bool(acc_f64))
        if args is None:
            plan = self.plan
            groups, group_base, split_rows = plan.split_groups()
            keep = (plan.workspace(), groups, group_base, split_rows, plan.desc, plan.ranges,
                    self.data, self.cols, self.rowptr)
            args = [_abi.dtype_code(self.data.dtype), int(acc_f64), self.data.data_ptr(),
                    self.cols.data_ptr(), self.rowptr.data_ptr(), self.rowptr_bits,
                    self.n_rows, self.nnz, None, None, None, 0, plan.desc.data_ptr(),
                    plan.ranges.data_ptr(), plan.n_desc, plan.chunk, keep[0].data_ptr(),
                    groups.data_ptr() if groups.numel() else None,
                    group_base.data_ptr() if group_base.numel() else None,
                    split_rows.data_ptr() if split_rows.numel() else None,
                    int(groups.shape[0]), 0, None]
            self._args[bool(acc_f64)] = args
            self._keep = keep
        a = list(args)
        a[8], a[9] = x.data_ptr(), y.data_ptr()
        a[10] = None if row_map is None else row_map.data_ptr()
        a[11] = n_out
        a[21] = XCD_REMAP_ROWBLOCK
        a[22] = self._order.stream(y.device, self._keep)
        _abi.check(_abi.lib().fsp_spmv_csr(*a), "fsp_spmv_csr")
        return y


def band_block_offset(cols, rowptr, n_desc):
    """The dominant distance, in row blocks, between a row and the far diagonals it reads, for
    banded / stencil matrices (a 2-D 5-point stencil on a W-wide grid reads rows +-W): the most
    common |column - row| of a sample of entries, converted to blocks, when at least
    BAND_MIN_SHARE of the sample lies on it and it is 2 or more blocks away; else None."""
    nnz = int(cols.numel())
    n_rows = int(rowptr.numel()) - 1
    if nnz == 0 or n_rows == 0 or n_desc == 0:
        return None
    idx = sample_indices(nnz, 1 << 16, cols.device)
    rp = rowptr.to(torch.int64)
    rows = torch.searchsorted(rp, idx, right=True) - 1
    dist = (cols[idx].to(torch.int64) - rows).abs()
    blocks = torch.round(dist.to(torch.float64) * (n_desc / n_rows)).to(torch.int64)
    blocks = blocks[(blocks >= 2) & (blocks < 64)]
    if blocks.numel() == 0:
        return None
    hist = torch.bincount(blocks, minlength=64)
    off = int(torch.argmax(hist).item())
    if hist[off].item() < BAND_MIN_SHARE * idx.numel():
        return None
    return off


def band_launch_order(n_desc, off, device):
    """A launch order of the descriptors in which a block and the blocks +-off from it (its
    far diagonals' x) run on the same XCD, while the eight XCDs stay close together in memory:
    block b = off*k + c (c < off) goes to XCD (c + off * (k // BAND_SEGMENT)) mod 8, each XCD
    takes its blocks in increasing order, and launch slot 8j + x holds XCD x's j-th block."""
    b = torch.arange(n_desc, device=device)
    c, k = b % off, b // off
    xcd = (c + off * (k // BAND_SEGMENT)) % XCD_COUNT
    by_xcd = torch.sort(xcd * n_desc + b)[1]  # XCD-major, block order inside
    count = torch.bincount(xcd, minlength=XCD_COUNT)
    first = torch.cumsum(count, 0) - count
    rank = torch.empty_like(b)
    rank[by_xcd] = b - first[xcd[by_xcd]]
    return torch.sort(rank * XCD_COUNT + xcd)[1]


def tensor_bytes(*tensors):
    """Device bytes held by the given tensors (each storage counted once; None skipped)."""
    seen, total = set(), 0
    for t in tensors:
        if t is None or not isinstance(t, torch.Tensor):
            continue
        st = t.untyped_storage()
        key = st.data_ptr()
        if key not in seen:
            seen.add(key)
            total += st.nbytes()
    return total


def _ceil_log2(v):
    return max(1, int(v - 1).bit_length()) if v > 1 else 1


class XcsLayout:
    """The XCD column-split layout (see the module docstring).  Built on the device."""

    kind = "xcs"

    def __init__(self, data, cols, rowptr, n_cols, panels_per_xcd=None, item_format=None):
        """item_format: 1 (sorted gathers) or 0; None - 1 when SORTED_ITEMS is set and the
        panels need at most xcs_sorted_col_bits column bits."""
        dev = data.device
        caps = _abi.caps()
        item_cap, rows_cap = caps["xcs_item"], caps["xcs_rows"]
        nnz = int(data.numel())
        n_rows = int(rowptr.numel()) - 1
        self.n_rows, self.n_cols, self.nnz = n_rows, int(n_cols), nnz
        lengths = (rowptr[1:] - rowptr[:-1]).to(torch.int64)
        cols = cols.to(torch.int32)

        # 1. P = 8*m column panels of about equal nnz (m panels per XCD, run one after the
        #    other, so that one panel of x - at most PANEL_BYTES - sits in the XCD's L2), each
        #    at most 2^b columns wide with b the fewest bits that can cover n_cols in P panels
        #    (more bits for the row in pidx).
        #    An x of at most XCD_COUNT / 2 panels' worth gets fewer panels than XCDs, each panel
        #    then shared by XCD_COUNT / P XCDs (fewer row splits, so fewer partial slots).
        if panels_per_xcd is not None:
            P = XCD_COUNT * int(panels_per_xcd)
        else:
            P = MIN_PANELS
            while P < XCD_COUNT * 8 and self.n_cols * data.element_size() > P * PANEL_BYTES:
                P *= 2
        m = max(1, P // XCD_COUNT)
        self.n_panels = P
        hist = torch.bincount(cols, minlength=self.n_cols) if nnz else \
            torch.zeros(self.n_cols, dtype=torch.int64, device=dev)
        cum = torch.cumsum(hist, 0)
        targets = torch.tensor([(k * nnz + P - 1) // P for k in range(1, P)], dtype=cum.dtype,
                               device=dev)
        inner = (torch.searchsorted(cum, targets) + 1).cpu().numpy()
        wmax = 1 << _ceil_log2(max(2, -(-self.n_cols // P)))
        cb = [0]
        for k, b in enumerate(inner.tolist(), start=1):
            lo = max(cb[-1], self.n_cols - (P - k) * wmax)
            hi = min(self.n_cols, cb[-1] + wmax)
            cb.append(min(max(int(b), lo), hi))
        cb.append(self.n_cols)
        widths = np.diff(np.array(cb))
        assert int(widths.max()) <= wmax
        self.panel_base_host = cb
        self.col_bits = _ceil_log2(max(int(widths.max()), 2))
        if item_format is None:
            item_format = 1 if SORTED_ITEMS and \
                _entries_per_panel_run(lengths, P) >= SORTED_MIN_RUN else 0
        self.item_format = 1 if item_format == 1 and \
            self.col_bits <= caps["xcs_sorted_col_bits"] else 0
        if self.item_format == 1:  # rows are not packed into the entries
            item_cap = caps["xcs_sorted_item"]
            self.rows_cap = SORTED_TILE_ROWS
        else:
            row_bits = 32 - self.col_bits
            self.rows_cap = min(rows_cap, 1 << row_bits)
        self.panel_base = torch.tensor(cb[:P], dtype=torch.int32, device=dev)
        if self.rows_cap < 256:
            raise ValueError("column panels too wide for the XCS packing")

        # 2. Row tiles.  A row longer than 8 * item_cap entries is a tile of its own (its
        #    partials are one value per item).  The other rows are covered greedily by tiles
        #    of <= rows_cap consecutive rows and <= 8 * item_cap entries, in which the long
        #    rows are rows without entries - they do not cut the run of short rows.
        tile_nnz = P * item_cap * (SORTED_TILE_ITEMS if self.item_format == 1 else 1)
        long_mask = lengths > tile_nnz
        long_rows = torch.nonzero(long_mask).flatten()
        short_ptr = torch.zeros(n_rows + 1, dtype=torch.int64, device=dev)
        torch.cumsum(torch.where(long_mask, 0, lengths), 0, out=short_ptr[1:])
        plan = build_row_block_plan_windows(short_ptr, tile_nnz, self.rows_cap, tile_nnz, 1,
                                            PLAN_WINDOW_BLOCKS * self.rows_cap)
        desc = plan.desc.to(device=dev, dtype=torch.int64)
        n_long = int(long_rows.numel())
        t_r0_d = torch.cat([long_rows, desc[:, 0]])
        t_R_d = torch.cat([torch.ones(n_long, dtype=torch.int64, device=dev),
                           desc[:, 1] - desc[:, 0]])
        n_tiles = int(t_r0_d.numel())
        self.n_tiles = n_tiles
        self.n_long_tiles = n_long
        tile_of_row = torch.repeat_interleave(torch.arange(n_long, n_tiles, device=dev),
                                              t_R_d[n_long:], output_size=n_rows)
        if n_long:
            tile_of_row[long_rows] = torch.arange(n_long, device=dev)

        # 3. Entry -> (tile, panel); stable sort keeps row order (then original order).  The
        #    radix sort's key is 32 bits wide wherever (tile, panel) pairs fit.
        entry_row = torch.repeat_interleave(torch.arange(n_rows, device=dev, dtype=torch.int32),
                                            lengths, output_size=nnz)
        key_type = torch.int32 if n_tiles * P < (1 << 31) else torch.int64
        entry_tile = tile_of_row.to(key_type)[entry_row]
        bounds = torch.tensor(cb[1:P], dtype=torch.int32, device=dev)
        panel = torch.bucketize(cols, bounds, right=True, out_int32=True)
        key = entry_tile * P + panel
        del entry_tile
        key_sorted, perm = torch.sort(key, stable=True)
        key_sorted = key_sorted.to(torch.int64)
        del key

        # 4. Pieces (tile, panel) -> items of <= item_cap entries (equal split).
        n_pieces = n_tiles * P
        # entries per piece: the boundaries of equal keys in the sorted keys
        bnd = torch.searchsorted(key_sorted, torch.arange(n_pieces + 1, device=dev))
        cnt = bnd[1:] - bnd[:-1]
        del bnd
        n_sub = (cnt + item_cap - 1) // item_cap
        n_items = int(n_sub.sum().item())
        piece_first_item = torch.cumsum(n_sub, 0) - n_sub
        base = torch.where(n_sub > 0, cnt // n_sub.clamp(min=1), torch.zeros_like(cnt))
        rem = torch.where(n_sub > 0, cnt % n_sub.clamp(min=1), torch.zeros_like(cnt))
        item_piece = torch.repeat_interleave(torch.arange(n_pieces, device=dev), n_sub,
                                             output_size=n_items)
        item_j = torch.arange(n_items, device=dev) - piece_first_item[item_piece]
        item_len = base[item_piece] + (item_j < rem[item_piece]).to(base.dtype)
        item_off = item_j * base[item_piece] + torch.minimum(item_j, rem[item_piece])
        item_tile = item_piece // P
        item_panel = item_piece % P
        items_per_tile = torch.bincount(item_tile, minlength=n_tiles)
        tile_first_item = torch.cumsum(items_per_tile, 0) - items_per_tile
        item_k = torch.arange(n_items, device=dev) - tile_first_item[item_tile]
        # Thread-major storage inside an item: with Q = ceil(len/4) quads, qp = ceil(Q/256)
        # quads per thread and nt = ceil(Q/qp) threads, thread t owns the logical quads
        # [qp*t, qp*t + qp), stored at memory quads t + nt*u.  A load of quad u by every thread
        # is then one contiguous span, and each thread holds a contiguous run of entries.
        q_tot = (item_len + 3) // 4
        qp = torch.clamp((q_tot + 255) // 256, min=1)
        nt = (q_tot + qp - 1) // qp
        padded = 4 * nt * qp
        if self.item_format == 1:  # 8 entries per thread of 512, in whole waves
            padded = (item_len + 511) // 512 * 512
        item_start = torch.cumsum(padded, 0) - padded
        n_entries = int(padded.sum().item()) if n_items else 0
        if n_entries > _INDEX_LIMIT_INT32:
            raise ValueError("matrix too large for the XCS layout")
        self.n_entries = n_entries

        # 5. Destination of every sorted entry; the new entry arrays.
        piece_start = torch.cumsum(cnt, 0) - cnt
        o = torch.arange(nnz, device=dev) - piece_start[key_sorted]
        b = base[key_sorted]
        rm = rem[key_sorted]
        big = (b + 1) * rm
        j = torch.where(o < big, o // (b + 1), rm + (o - big) // b.clamp(min=1))
        item_of = piece_first_item[key_sorted] + j
        oi = o - item_off[item_of]  # logical position inside the item
        del o, b, rm, big, j
        pan = key_sorted % P
        colp = cols[perm].to(torch.int64) - self.panel_base.to(torch.int64)[pan]
        del pan
        pidx = torch.zeros(max(n_entries, 4), dtype=torch.int64, device=dev)
        if self.item_format == 1:
            # values in row order: position 8t + e at quad (e/4) * P/8 + t, element e % 4
            thr = padded[item_of] // 8
            dest = item_start[item_of] + 4 * ((oi % 8) // 4 * thr + oi // 8) + oi % 4
            # gather words in column order: the k-th gather of thread t is entry
            # (t/64)*512 + 64k + t%64 of the item's column order, at the same quads
            er = entry_row[perm]
            start = torch.ones_like(oi, dtype=torch.bool)
            if nnz > 1:
                start[1:] = (oi[1:] == 0) | (er[1:] != er[:-1])
            del er
            sb = caps["xcs_sorted_col_bits"]
            word = (oi << (sb + 1)) | (start.to(torch.int64) << sb) | colp
            del start
            by_col = torch.sort(item_of * (1 << 20) + colp, stable=True)[1]
            first_entry = torch.cumsum(item_len, 0) - item_len  # items are contiguous
            it_c = item_of[by_col]
            gr = torch.arange(nnz, device=dev) - first_entry[it_c]
            t_g = (gr // 512) * 64 + gr % 64
            kk = (gr % 512) // 64
            gdest = item_start[it_c] + 4 * (kk // 4 * thr[by_col] + t_g) + kk % 4
            pidx[gdest] = word[by_col]
            del word, by_col, it_c, gr, t_g, kk, gdest, thr
        else:
            qpi = qp[item_of]
            lq = oi // 4
            dest = item_start[item_of] + 4 * (lq // qpi + nt[item_of] * (lq % qpi)) + oi % 4
            del qpi, lq
            loc_row = (entry_row[perm] - t_r0_d[key_sorted // P]).to(torch.int64)
            pidx[dest] = (loc_row << self.col_bits) | colp
            del loc_row
        del oi, colp
        vals = torch.zeros(max(n_entries, 4), dtype=data.dtype, device=dev)
        vals[dest] = data[perm]
        self.vals = vals
        self.pidx = torch.where(pidx >= (1 << 31), pidx - (1 << 32), pidx).to(torch.int32)
        del pidx, dest

        # 6. Partial sums: one per (item, row run it holds); per row they are added in item
        #    order (the combine's summation order).  Where each is stored: the combine tables.
        er = entry_row[perm]
        del entry_row, perm, key_sorted
        pair_key = torch.unique_consecutive(item_of * max(n_rows, 1) + er)  # sorted entries
        del er, item_of
        pair_row = pair_key % max(n_rows, 1)
        pair_item = pair_key // max(n_rows, 1)
        del pair_key
        count = torch.bincount(pair_row, minlength=n_rows) if pair_row.numel() else \
            torch.zeros(n_rows, dtype=torch.int64, device=dev)
        self.n_split_rows = int((count > 1).sum().item()) if n_rows else 0
        self.n_runs_total = int(pair_row.numel())
        self._build_combine_windows(pair_item, pair_row, count, n_items, caps)
        del pair_row, pair_item, count

        # 7. Launch order: XCD x runs the items of panels x, x + 8, x + 16, ... (one panel
        #    after the other, each in tile order); with P < 8 panel p's items are dealt in turn
        #    to XCDs p, p + P, p + 2P, ...; lists padded to the same length q so that slot
        #    x*q + j lands on XCD x.
        if P >= XCD_COUNT:
            xcd = item_panel % XCD_COUNT
            phase = item_panel // XCD_COUNT
        else:
            by_panel = torch.sort(item_panel, stable=True)[1]
            pcount = torch.bincount(item_panel, minlength=P)
            rank_in_panel = torch.empty_like(item_panel)
            rank_in_panel[by_panel] = torch.arange(n_items, device=dev) - \
                (torch.cumsum(pcount, 0) - pcount)[item_panel[by_panel]]
            xcd = item_panel + P * (rank_in_panel % (XCD_COUNT // P))
            phase = torch.zeros_like(item_panel)
        per_xcd = torch.bincount(xcd, minlength=XCD_COUNT)
        q = int(per_xcd.max().item()) if n_items else 0
        self.n_slots = XCD_COUNT * q
        skey = (xcd * m + phase) * (n_tiles + 1) + item_tile
        order = torch.sort(skey, stable=True)[1]
        xcd_first = torch.cumsum(per_xcd, 0) - per_xcd
        rank = torch.arange(n_items, device=dev) - xcd_first[xcd[order]]
        slot_of = xcd[order] * q + rank
        d = torch.zeros((max(self.n_slots, 1), 12), dtype=torch.int64, device=dev)
        d[:, 10] = -1
        it = order
        t = item_tile[it]
        z = torch.zeros_like(t)
        d[slot_of] = torch.stack([item_start[it], item_len[it], item_k[it],
                                  self.item_first_run[it], t_r0_d[t], t_R_d[t],
                                  self.panel_base.to(torch.int64)[item_panel[it]],
                                  self.item_n_runs[it], z, z, t, z], 1)
        d = torch.where(d >= (1 << 31), d - (1 << 32), d)
        self.items = d.to(torch.int32).contiguous()
        self.n_items = n_items
        self.max_items_per_panel = q
        self.partials = torch.empty(max(self.n_partials, 1), dtype=torch.float64, device=dev)
        # every array a launch reads or writes (marked as used on a new caller stream)
        self._keep = (self.partials, self.vals, self.pidx, self.items, self.item_runs,
                      self.windows, self.dest, self.row_count)
        self._order = StreamOrder(dev)

    def _build_combine_windows(self, pair_item, pair_row, count, n_items, caps):
        """Where every partial sum is stored, and the tables of the second launch
        (xcs_window_combine_kernel).  pair_item / pair_row: the item and the row of every
        partial sum ("pair"), in (item, row) order - the order in which an item produces them.

        Rows are grouped into windows of consecutive rows with at most WINDOW_SLOTS sums and
        WINDOW_ROWS rows (a row with more sums, or more than ROW_COUNT_MAX, is a window alone,
        "big").  The partials buffer holds the windows one after the other, and inside a
        window one run per item with rows in it (in item order), each run starting on a
        multiple of RUN_ALIGN slots: an item writes whole lines of its own, and the combine
        reads a window as one contiguous range.  dest gives every stored slot its position in
        the window's (row, item) order (-1 for the padding), row_count every row its number of
        sums (one byte; a row's first position is the sum of the counts before it in its
        window)."""
        dev = pair_row.device
        n_rows, n_pairs = self.n_rows, int(pair_row.numel())
        win_slots = min(WINDOW_SLOTS, caps["xcs_window_slots"])
        rows_cap = min(WINDOW_ROWS, caps["xcs_window_rows"])
        rp = torch.zeros(n_rows + 1, dtype=torch.int64, device=dev)
        torch.cumsum(count, 0, out=rp[1:])
        # the planner sees a row of more than ROW_COUNT_MAX sums as longer than a window, so
        # that it becomes a window of its own
        plan_rp = rp
        if n_rows and int(count.max().item()) > ROW_COUNT_MAX:
            plan_rp = torch.zeros_like(rp)
            torch.cumsum(torch.where(count > ROW_COUNT_MAX, win_slots + 1, count), 0,
                         out=plan_rp[1:])
        plan = build_row_block_plan_windows(plan_rp, win_slots, rows_cap, win_slots, 1 << 30,
                                            PLAN_WINDOW_BLOCKS * rows_cap)
        wd = plan.desc.to(device=dev, dtype=torch.int64)
        n_win = int(wd.shape[0])
        big = wd[:, 2] != 0  # {row, 0, 1, -1}: one row with more sums than a window holds
        row0 = wd[:, 0]
        nr = torch.where(big, torch.ones_like(row0), wd[:, 1] - wd[:, 0])
        win_of_row = torch.repeat_interleave(torch.arange(n_win, device=dev), nr,
                                             output_size=n_rows)
        first_pos = rp[row0]  # a window's first sum in (row, item) order
        pair_win = win_of_row[pair_row] if n_pairs else torch.zeros(0, dtype=torch.int64,
                                                                    device=dev)
        # runs: the sums of one item in one window (consecutive in pair order)
        brk = torch.ones(n_pairs, dtype=torch.bool, device=dev)
        if n_pairs > 1:
            brk[1:] = (pair_item[1:] != pair_item[:-1]) | (pair_win[1:] != pair_win[:-1])
        run_first = torch.nonzero(brk).flatten()
        run_len = torch.diff(run_first, append=torch.tensor([n_pairs], device=dev))
        run_item = pair_item[run_first]
        run_win = pair_win[run_first]
        del brk
        n_runs = int(run_first.numel())
        # storage: windows in order, runs of a window in item order, starts aligned unless
        # the padding would cost more than a quarter of the buffer (short runs) or the window
        # is big (its runs hold one sum each)
        wkey = torch.sort(run_win * max(n_items, 1) + run_item, stable=True)[1]
        align = RUN_ALIGN
        padded = (run_len + align - 1) // align * align
        if n_runs and int(padded.sum().item()) > 1.25 * n_pairs:
            align, padded = 1, run_len.clone()
        padded = torch.where(big[run_win], run_len, padded)
        self.run_align = align
        # windows: {row0, rows (-1: big), first stored slot, stored slots, sums, 0, 0, 0};
        # every window starts on a line (WINDOW_ALIGN slots) whatever the run alignment; the
        # slots between windows stay dest -1
        wlen = torch.bincount(run_win, weights=padded.to(torch.float64), minlength=n_win) \
            .to(torch.int64) if n_runs else torch.zeros(n_win, dtype=torch.int64, device=dev)
        wspan = (wlen + WINDOW_ALIGN - 1) // WINDOW_ALIGN * WINDOW_ALIGN
        wbase = torch.cumsum(wspan, 0) - wspan
        n_store = int(wspan.sum().item()) if n_win else 0
        plen = padded[wkey]
        win_sorted = run_win[wkey]
        in_win = torch.cumsum(plen, 0) - plen  # exclusive, over all windows
        wfirst = torch.cumsum(wlen, 0) - wlen  # the same, at each window's first run
        run_base = torch.empty_like(in_win)
        run_base[wkey] = wbase[win_sorted] + in_win - wfirst[win_sorted]
        del plen, win_sorted, in_win, wfirst
        wsum = torch.bincount(pair_win, minlength=n_win) if n_pairs else \
            torch.zeros(n_win, dtype=torch.int64, device=dev)
        z = torch.zeros_like(row0)
        nr_field = torch.where(big, torch.full_like(nr, -1), nr)
        self.windows = torch.stack([row0, nr_field, wbase, wlen, wsum, z, z, z], 1) \
            .to(torch.int32).contiguous()
        self.n_windows = n_win
        # every sum's stored slot, and its position in the window's (row, item) order
        run_of = torch.repeat_interleave(torch.arange(n_runs, device=dev), run_len,
                                         output_size=n_pairs)
        stored = run_base[run_of] + (torch.arange(n_pairs, device=dev) - run_first[run_of])
        by_row = torch.sort(pair_row.to(torch.int32), stable=True)[1]  # a 32-bit radix key
        rank = torch.empty_like(by_row)
        rank[by_row] = torch.arange(n_pairs, device=dev)
        pos = rank - first_pos[pair_win]
        pos = torch.where(big[pair_win], torch.zeros_like(pos), pos)
        dest = torch.full((max(n_store, 1),), -1, dtype=torch.int64, device=dev)
        dest[stored] = pos
        self.dest = dest.to(torch.int16).contiguous()
        row_count = torch.where(big[win_of_row], torch.zeros_like(count), count)
        self.row_count = row_count.to(torch.uint8).contiguous() if n_rows else \
            torch.zeros(1, dtype=torch.uint8, device=dev)
        del by_row, rank, pos, dest, run_of, stored
        # per item: its runs (pair order = item order, then window order), each {stored slot
        # of its first sum, the item's index of that sum, sums, stored length}
        first_of_item = torch.cumsum(torch.bincount(pair_item, minlength=n_items), 0) - \
            torch.bincount(pair_item, minlength=n_items) if n_pairs else \
            torch.zeros(n_items, dtype=torch.int64, device=dev)
        runs_per_item = torch.bincount(run_item, minlength=n_items) if n_runs else \
            torch.zeros(n_items, dtype=torch.int64, device=dev)
        if n_runs and int(runs_per_item.max().item()) > caps["xcs_item_runs"]:
            raise ValueError("an XCS item spans more combine windows than the kernel holds")
        self.item_first_run = torch.cumsum(runs_per_item, 0) - runs_per_item
        self.item_n_runs = runs_per_item
        ir = torch.stack([run_base, run_first - first_of_item[run_item], run_len, padded], 1) \
            if n_runs else torch.zeros((1, 4), dtype=torch.int64, device=dev)
        self.item_runs = ir.to(torch.int32).contiguous()
        self.n_partials = max(n_store, 1)
        self.window_rows_cap = rows_cap
        self.window_slots = win_slots

    def kernel_name(self):
        return "spmv_xcs_sorted_kernel" if self.item_format == 1 else "spmv_xcs_kernel"

    def held_bytes(self, caller=()):
        """Device bytes of the layout's own arrays (the rewritten entries, tables, partials)."""
        return tensor_bytes(self.vals, self.pidx, self.items, self.item_runs, self.windows,
                            self.dest, self.row_count, self.partials, self.panel_base)

    def describe(self):
        return {"layout": self.kind, "panels": self.n_panels, "tiles": self.n_tiles,
                "long_row_tiles": self.n_long_tiles,
                "items": self.n_items,
                "slots": self.n_slots, "split_rows": self.n_split_rows,
                "partials": self.n_partials, "combine_windows": self.n_windows,
                "panel_base": self.panel_base_host,
                "col_bits": self.col_bits, "padded_entries": self.n_entries,
                "item_format": self.item_format}

    def launch(self, x, y, acc_f64, row_map=None, n_out=0, passes=3):
        """Both passes (passes=3), or only the items (1: the partial sums; y zeroed first when
        a row map is given) or only the combine windows (2)."""
        # static arguments converted once per accumulation mode (see RowBlockLayout.launch)
        args = self._args.get(bool(acc_f64)) if hasattr(self, "_args") else None
        if args is None:
            if not hasattr(self, "_args"):
                self._args = {}
            p = lambda t: t.data_ptr() if t is not None and t.numel() else None  # noqa: E731
            args = [_abi.dtype_code(self.vals.dtype), int(acc_f64), p(self.vals), p(self.pidx),
                    self.n_entries, self.col_bits, None, None, None, 0, p(self.items),
                    self.n_slots, p(self.item_runs), p(self.partials), p(self.windows),
                    self.n_windows, self.window_slots, p(self.dest), p(self.row_count),
                    self.item_format, None]
            self._args[bool(acc_f64)] = args
        a = list(args)
        a[6], a[7] = x.data_ptr(), y.data_ptr()
        a[8] = None if row_map is None else row_map.data_ptr()
        a[9] = n_out
        if not passes & 1:
            a[11] = 0
        if not passes & 2:
            a[15] = 0
        a[20] = self._order.stream(y.device, self._keep)
        _abi.check(_abi.lib().fsp_spmv_xcs(*a), "fsp_spmv_xcs")
        return y


def _panel_col_bits(n_cols, value_bytes):
    """Bits of a column inside its panel: 2^bits values fit the LDS copy (and no more than x
    needs)."""
    fit = (_abi.caps()["panel_bytes"] // value_bytes).bit_length() - 1
    return max(1, min(fit, 15, _ceil_log2(max(int(n_cols), 2))))  # 15: the 16-bit entries


def panel_row_min(n_cols, value_bytes):
    """Row length from which a row puts about PANEL_RUNS entries in every x panel."""
    if FORCE_PANEL_ROW_MIN is not None:
        return int(FORCE_PANEL_ROW_MIN)
    n_panels = -(-int(n_cols) >> _panel_col_bits(n_cols, value_bytes))
    return int(PANEL_RUNS * max(1, n_panels))


def plan_panel_chunks_prefix(panel_runs, run_len, chunk, runs_cap):
    """fsp_plan_panel_chunks' plan as a prefix sum of the run lengths, on whatever device the
    tensors live: (run_pos, panel_end), or None where that is not the plan.  Without the run
    cap each panel's runs are packed back to back and only its last chunk is padded; the cap
    changes nothing as long as no chunk would hold more than runs_cap pieces of runs (the runs
    starting in it, plus one when its first entry continues a run), which is checked here -
    the greedy planner closes a chunk early only at a run that would be its runs_cap + 1st."""
    dev = run_len.device
    n_panels = int(panel_runs.numel()) - 1
    n_runs = int(run_len.numel())
    pr = panel_runs.to(device=dev, dtype=torch.int64)
    rl = run_len.to(torch.int64)
    csum = torch.zeros(n_runs + 1, dtype=torch.int64, device=dev)
    torch.cumsum(rl, 0, out=csum[1:])
    panel_len = (csum[pr[1:]] - csum[pr[:-1]] + chunk - 1) // chunk * chunk
    panel_end = torch.cumsum(panel_len, 0)
    if n_runs == 0:
        return torch.zeros(0, dtype=torch.int64, device=dev), panel_end
    panel_of = torch.repeat_interleave(torch.arange(n_panels, device=dev), pr[1:] - pr[:-1],
                                       output_size=n_runs)
    run_pos = (panel_end - panel_len)[panel_of] + csum[:-1] - csum[pr[:-1]][panel_of]
    n_chunks = int(panel_end[-1].item()) // chunk
    first_chunk = run_pos // chunk
    pieces = torch.bincount(first_chunk, minlength=n_chunks)
    at_start = torch.zeros(n_chunks, dtype=torch.int64, device=dev)
    at_start[first_chunk[run_pos % chunk == 0]] = 1
    pieces += 1 - at_start  # every chunk holds entries: a first entry that no run starts
    if int(pieces.max().item()) > runs_cap:
        return None
    return run_pos, panel_end


def plan_panel_chunks(panel_runs, run_len, chunk, runs_cap):
    """(run_pos, panel_end) of fsp_plan_panel_chunks - where each run's first entry is stored,
    and where each panel ends - on the device of run_len: the prefix-sum plan where it is the
    plan, else fsp_plan_panel_chunks_device (one thread per panel, the greedy rule).  Host
    tensors take the host planner."""
    dev = run_len.device
    n_panels = int(panel_runs.numel()) - 1
    if not run_len.is_cuda:
        pr = panel_runs.to("cpu", torch.int64).contiguous()
        rl = run_len.to("cpu", torch.int64).contiguous()
        pos = torch.empty(max(int(rl.numel()), 1), dtype=torch.int64)
        end = torch.empty(max(n_panels, 1), dtype=torch.int64)
        _abi.check(_abi.lib().fsp_plan_panel_chunks(pr.data_ptr(), n_panels, rl.data_ptr(),
                                                    int(chunk), int(runs_cap), pos.data_ptr(),
                                                    end.data_ptr()), "fsp_plan_panel_chunks")
        return pos[:rl.numel()], end[:n_panels]
    plan = plan_panel_chunks_prefix(panel_runs, run_len, chunk, runs_cap)
    if plan is not None:
        return plan
    return plan_panel_chunks_kernel(panel_runs, run_len, chunk, runs_cap)


def plan_panel_chunks_kernel(panel_runs, run_len, chunk, runs_cap):
    """(run_pos, panel_end) of fsp_plan_panel_chunks from fsp_plan_panel_chunks_device (device
    tensors)."""
    dev = run_len.device
    n_panels = int(panel_runs.numel()) - 1
    if run_len.numel() == 0:  # no runs: every panel empty
        return (torch.zeros(0, dtype=torch.int64, device=dev),
                torch.zeros(max(n_panels, 0), dtype=torch.int64, device=dev))
    pr = panel_runs.to(device=dev, dtype=torch.int64).contiguous()
    rl = run_len.to(torch.int64).contiguous()
    local = torch.empty(max(int(rl.numel()), 1), dtype=torch.int64, device=dev)
    panel_len = torch.empty(max(n_panels, 1), dtype=torch.int64, device=dev)
    _abi.check(_abi.lib().fsp_plan_panel_chunks_device(
        pr.data_ptr(), n_panels, rl.data_ptr(), int(chunk), int(runs_cap), local.data_ptr(),
        panel_len.data_ptr(), _abi.raw_stream(dev)), "fsp_plan_panel_chunks_device")
    panel_len = panel_len[:n_panels]
    panel_end = torch.cumsum(panel_len, 0)
    panel_of = torch.repeat_interleave(torch.arange(n_panels, device=dev), pr[1:] - pr[:-1],
                                       output_size=int(rl.numel()))
    return local[:rl.numel()] + (panel_end - panel_len)[panel_of], panel_end


def panel_storage_positions_of(p, chunk):
    """Memory position of the logical entries p of the panel layout: inside a chunk, lane L's
    h-th quad (logical quad 2L + h) is stored at quad 64h + L."""
    lq = (p % chunk) // 4
    return (p // chunk) * chunk + ((lq % 2) * (chunk // 8) + lq // 2) * 4 + p % 4


def panel_storage_positions(n_entries, chunk, device):
    """panel_storage_positions_of for every logical entry 0 .. n_entries - 1."""
    return panel_storage_positions_of(torch.arange(n_entries, device=device), chunk)


class PanelLayout:
    """Rows whose x gathers are served from LDS copies of 128 KiB x panels (module docstring).
    ``rows`` are the output rows of the CSR rows given; built on the device."""

    kind = "panels"

    def __init__(self, data, cols, rowptr, n_cols, rows):
        dev = data.device
        caps = _abi.caps()
        chunk = caps["panel_chunk"]
        self.n_cols, self.nnz = int(n_cols), int(data.numel())
        n_rows = int(rowptr.numel()) - 1
        cb = _panel_col_bits(n_cols, data.element_size())
        if n_rows >= (1 << (63 - cb)):
            raise ValueError("too many rows for the panel layout")
        self.col_bits = cb
        self.rows = rows.to(torch.int32).contiguous()
        rp = rowptr.to(torch.int64)
        nnz = self.nnz
        n_panels = max(1, -(-self.n_cols >> cb))
        cols32 = cols.to(torch.int32)
        # entries by (panel, row): a stable sort by panel keeps each row's entries in order
        # (radix-sorted on a key no wider than the panel count needs: one byte for cfg-sized x)
        panel = cols32 >> cb
        key = panel.to(torch.uint8 if n_panels <= 256 else
                       torch.int16 if n_panels <= (1 << 15) else torch.int32)
        order = torch.sort(key, stable=True)[1]
        del key
        row = torch.repeat_interleave(torch.arange(n_rows, device=dev, dtype=torch.int32),
                                      rp[1:] - rp[:-1], output_size=nnz)
        row_s = row[order]
        del row
        panel = panel[order]
        # runs: the entries of one row in one panel; chunks of at most `chunk` entries and
        # panel_chunk_runs runs (the kernel stages a chunk's run sums one per lane), planned on
        # the device (plan_panel_chunks); the rest of a chunk closed early, and of each panel's
        # last chunk, is padding
        brk = torch.ones(nnz, dtype=torch.bool, device=dev)
        if nnz > 1:
            brk[1:] = (panel[1:] != panel[:-1]) | (row_s[1:] != row_s[:-1])
        run_first = torch.nonzero(brk).flatten()
        n_runs = int(run_first.numel())
        run_len = torch.diff(run_first, append=torch.tensor([nnz], device=dev))
        run_panel = panel[run_first].to(torch.int64)
        del panel
        panel_runs = torch.zeros(n_panels + 1, dtype=torch.int64, device=dev)
        torch.cumsum(torch.bincount(run_panel, minlength=n_panels), 0, out=panel_runs[1:])
        run_pos, panel_end = plan_panel_chunks(panel_runs, run_len, chunk,
                                               caps["panel_chunk_runs"])
        n_entries = int(panel_end[-1].item()) if n_panels else 0
        self.n_entries = n_entries
        n_chunks = n_entries // chunk
        # logical position of every entry: its run's position plus its place in the run
        run_id = torch.cumsum(brk, 0) - 1
        del brk
        dest = torch.arange(nnz, device=dev) + (run_pos - run_first)[run_id]
        del run_id
        # a chunk's runs start at the chunk's first entry and at every run's first entry (the
        # padding closing a chunk continues the run before it, and no chunk opens with padding)
        starts = torch.zeros(n_entries, dtype=torch.bool, device=dev)
        starts[::chunk] = True
        starts[run_pos] = True
        runs = starts.view(n_chunks, chunk).sum(1)
        if n_chunks and int(runs.max().item()) > caps["panel_chunk_runs"]:
            raise AssertionError("panel chunk plan: a chunk holds more runs than the kernel "
                                 "stages")
        # per chunk {first slot, entries in use}: the padding (a chunk closed early, or a
        # panel's last chunk) is the chunk's tail, whose products the kernel takes as 0
        real = torch.zeros(n_entries, dtype=torch.bool, device=dev)
        real[dest] = True
        rv = real.view(n_chunks, chunk)
        used = rv.sum(1)
        if n_chunks and bool((rv[:, 1:] & ~rv[:, :-1]).any()):
            raise AssertionError("panel chunk plan: padding inside a chunk")
        del real, rv
        self.chunk_info = torch.stack([torch.cumsum(runs, 0) - runs, used], 1) \
            .to(torch.int32).contiguous()
        # one partial slot per (chunk, run), in slot order: the row at each run start
        row_at = torch.zeros(n_entries, dtype=torch.int32, device=dev)
        row_at[dest] = row_s
        slot_row = row_at[torch.nonzero(starts).flatten()]
        del row_at
        self.n_partials = int(slot_row.numel())
        if self.n_partials * 8 > _INDEX_LIMIT_INT32:
            raise ValueError("more panel partial sums than the kernel's store range holds")
        self.slots = torch.sort(slot_row, stable=True)[1].to(torch.int32).contiguous()
        row_ptr = torch.zeros(n_rows + 1, dtype=torch.int64, device=dev)
        torch.cumsum(torch.bincount(slot_row, minlength=n_rows), 0, out=row_ptr[1:])
        self.row_ptr = row_ptr.to(torch.int32).contiguous()
        self.n_rows = n_rows
        # values: inside a chunk, logical quad 2L + h at quad 64h + L; 16-bit entries in logical
        # order, the column in the panel | 0x8000 at a run start (the kernel needs only where
        # runs start: a chunk's runs take consecutive slots)
        self.vals = torch.zeros(max(n_entries, 4), dtype=data.dtype, device=dev)
        self.vals[panel_storage_positions_of(dest, chunk)] = data[order]
        pc = torch.zeros(n_entries, dtype=torch.int32, device=dev)
        pc[dest] = cols32[order] & ((1 << cb) - 1)
        pc |= starts.to(torch.int32) << 15
        self.pcol = torch.zeros(max(n_entries, 8), dtype=torch.int16, device=dev)
        self.pcol[:n_entries] = torch.where(pc >= (1 << 15), pc - (1 << 16), pc).to(torch.int16)
        del pc, starts, slot_row, dest, order, row_s, cols32, run_first, run_len, run_pos
        panel_start = torch.cat([panel_end.new_zeros(1), panel_end[:-1]])
        self.panel_chunk0 = panel_start // chunk  # each panel's first chunk
        # jobs: a panel's chunks cut evenly into the fewest jobs of <= PANEL_JOB_CHUNKS (equal
        # sizes keep the rounds of workgroups even)
        per_panel = (panel_end - panel_start) // chunk
        n_jobs_p = (per_panel + PANEL_JOB_CHUNKS - 1) // PANEL_JOB_CHUNKS
        self.job_panel = torch.repeat_interleave(torch.arange(n_panels, device=dev), n_jobs_p)
        job_first = torch.cumsum(n_jobs_p, 0) - n_jobs_p
        k = torch.arange(self.job_panel.numel(), device=dev) - job_first[self.job_panel]
        starts_c = (panel_start // chunk)[self.job_panel] + \
            k * per_panel[self.job_panel] // n_jobs_p[self.job_panel]
        self.jobs = torch.cat([starts_c, torch.tensor([n_chunks], device=dev)]).to(
            torch.int32).contiguous()
        self.job_panel = self.job_panel.to(torch.int32).contiguous()
        self.n_jobs = int(self.job_panel.numel())
        self.n_panels = n_panels
        self.partials = torch.empty(max(self.n_partials, 1), dtype=torch.float64, device=dev)
        # every array a launch reads or writes (marked as used on a new caller stream)
        self._keep = (self.partials, self.vals, self.pcol, self.jobs, self.job_panel,
                      self.chunk_info, self.rows, self.row_ptr, self.slots)
        self._args = {}
        self._order = StreamOrder(dev)

    def kernel_name(self):
        return "spmv_panel_kernel"

    def held_bytes(self, caller=()):
        """Device bytes of the layout's own arrays (the rewritten entries, tables, partials)."""
        return tensor_bytes(self.vals, self.pcol, self.rows, self.chunk_info, self.slots,
                            self.row_ptr, self.jobs, self.job_panel, self.partials)

    def describe(self):
        return {"layout": self.kind, "rows": self.n_rows, "panels": self.n_panels,
                "col_bits": self.col_bits, "jobs": self.n_jobs,
                "chunks": self.n_entries // _abi.caps()["panel_chunk"],
                "partials": self.n_partials, "padded_entries": self.n_entries}

    def launch(self, x, y, acc_f64, row_map=None, passes=3, stream=None):
        """Both passes on the caller's stream (passes=3), or only the entry pass (1) or only
        the combine (2) on the raw ``stream`` given."""
        args = self._args.get(bool(acc_f64))
        if args is None:  # static arguments converted once per accumulation mode
            p = lambda t: t.data_ptr() if t is not None and t.numel() else None  # noqa: E731
            args = [_abi.dtype_code(self.vals.dtype), int(acc_f64), p(self.vals), p(self.pcol),
                    self.n_entries, self.col_bits, None, self.n_cols, None, None, p(self.jobs),
                    p(self.job_panel), self.n_jobs, p(self.chunk_info), p(self.partials),
                    int(self.partials.numel()), p(self.rows), p(self.row_ptr), p(self.slots),
                    self.n_rows, None, 0, None, None, None, None, 0, None]
            self._args[bool(acc_f64)] = args
        a = list(args)
        a[6], a[8] = x.data_ptr(), y.data_ptr()
        a[9] = None if row_map is None else row_map.data_ptr()
        if not passes & 1:
            a[12] = 0
        if not passes & 2:
            a[19] = 0
        a[27] = stream if stream is not None else self._order.stream(y.device, self._keep)
        _abi.check(_abi.lib().fsp_spmv_panels(*a), "fsp_spmv_panels")
        return y


class XcsHybridLayout:
    """Long rows in a PanelLayout, the rest in an XcsLayout (module docstring).  The XCS part
    sees the long rows as rows without entries and writes them as 0; the panel part's combine,
    launched after it on the caller's stream, then writes their sums.

    The first passes of both parts run one after the other on the caller's stream, then one
    launch does both second passes (fsp_spmv_hybrid_combine): the XCS combine windows and the
    panel part's rows, the long rows being marked ROW_SKIP in the XCS part's row counts.
    Measured on MI355X, cfg3: the
    panel kernel on a second stream beside the XCS kernel (fork and join events around it)
    took 275.8 us per call against 279.2 us serial, 1.2 %: a CU that holds a panel workgroup
    (128 KiB of LDS) has no room for an XCS workgroup, so the two kernels take turns and only
    their tails overlap; with the XCS kernel's LDS claim cut so that one of its workgroups
    fits beside a panel workgroup, 282.0 us.  Also measured: the two combines side by side
    282.5 us against 281 us, the panel kernel beside the XCS combine 292 us (two HBM
    streams)."""

    kind = "xcs-hybrid"

    def __init__(self, data, cols, rowptr, n_cols, long_mask, panels_per_xcd=None):
        dev = data.device
        rp = rowptr.to(torch.int64)
        lengths = rp[1:] - rp[:-1]
        self.n_rows, self.n_cols, self.nnz = int(lengths.numel()), int(n_cols), int(data.numel())
        entry_long = torch.repeat_interleave(long_mask, lengths, output_size=self.nnz)
        short_ptr = torch.zeros_like(rp)
        torch.cumsum(torch.where(long_mask, 0, lengths), 0, out=short_ptr[1:])
        pick = torch.nonzero(~entry_long).flatten()
        self.short = xcs_layout(data[pick], cols[pick], short_ptr, n_cols, panels_per_xcd)
        pick = torch.nonzero(entry_long).flatten()
        del entry_long
        long_rows = torch.nonzero(long_mask).flatten()
        long_ptr = torch.zeros(long_rows.numel() + 1, dtype=torch.int64, device=dev)
        torch.cumsum(lengths[long_rows], 0, out=long_ptr[1:])
        self.long = PanelLayout(data[pick], cols[pick], long_ptr, n_cols, long_rows)
        del pick
        # the long rows have no sums in the XCS part: its windows leave them to the panel rows
        if long_rows.numel():
            self.short.row_count[long_rows] = ROW_SKIP
        self._args = {}

    def kernel_name(self):
        return "spmv_xcs_kernel+spmv_panel_kernel"

    def held_bytes(self, caller=()):
        return self.short.held_bytes(caller) + self.long.held_bytes(caller)

    def describe(self):
        return {"layout": self.kind, "long_rows": self.long.n_rows,
                "long_entries": self.long.nnz, "xcs_part": self.short.describe(),
                "panel_part": self.long.describe()}

    def launch(self, x, y, acc_f64, row_map=None, n_out=0):
        # each part's arrays ordered after their previous user and marked as used here
        st = self.short._order.stream(y.device, self.short._keep)
        self.long._order.stream(y.device, self.long._keep)
        if HYBRID_PANEL_FIRST:
            self.long.launch(x, y, acc_f64, row_map, passes=1, stream=st)
            self.short.launch(x, y, acc_f64, row_map, n_out, passes=1)  # zeroes y[0..n_out)
        else:
            self.short.launch(x, y, acc_f64, row_map, n_out, passes=1)  # zeroes y[0..n_out)
            self.long.launch(x, y, acc_f64, row_map, passes=1, stream=st)
        args = self._args.get(bool(acc_f64))
        if args is None:  # static arguments converted once per accumulation mode
            p = lambda t: t.data_ptr() if t is not None and t.numel() else None  # noqa: E731
            sh, lg = self.short, self.long
            args = [_abi.dtype_code(sh.vals.dtype), int(acc_f64), None, None, p(sh.partials),
                    p(sh.windows), sh.n_windows, sh.window_slots, p(sh.dest), p(sh.row_count),
                    p(lg.partials), p(lg.rows), p(lg.row_ptr), p(lg.slots), lg.n_rows, None]
            self._args[bool(acc_f64)] = args
        a = list(args)
        a[2] = y.data_ptr()
        a[3] = None if row_map is None else row_map.data_ptr()
        a[15] = st
        _abi.check(_abi.lib().fsp_spmv_hybrid_combine(*a), "fsp_spmv_hybrid_combine")
        return y


class XstageLayout:
    """Long rows in a PanelLayout (``self.long``, None when there are none), the other rows
    staged (module docstring).  Built on the device.  ValueError when the staged entries pass
    the kernels' 32-bit offsets (or the long rows the panel layout's limits)."""

    kind = "xstage"

    def __init__(self, data, cols, rowptr, n_cols, long_mask):
        dev = data.device
        caps = _abi.caps()
        rp = rowptr.to(torch.int64)
        lengths = rp[1:] - rp[:-1]
        n_rows = int(lengths.numel())
        self.n_rows, self.n_cols, self.nnz = n_rows, int(n_cols), int(data.numel())
        cb = _panel_col_bits(n_cols, data.element_size())
        P = max(1, -(-self.n_cols >> cb))
        self.col_bits, self.n_panels = cb, P
        chunk = caps["stage_chunk"]
        # Windows of the larger size where the smaller would leave each panel's segment of a
        # window under STAGE_SEGMENT_MIN entries: the panel jobs write the segments of a window
        # from many CUs, and short segments share more lines (measured on MI355X, cfg3 - 256
        # panels -: 8192 against 4096 entries 195.4 against 207.2 us a call; cfg4 - 64 panels
        # -: 132.9 against 133.5 us, its panel pass 5.6 us faster and its combine 4.6 slower).
        win_cap, win_rows = caps["stage_window"], caps["stage_window_rows"]
        if FORCE_STAGE_WINDOW:
            win_cap = int(FORCE_STAGE_WINDOW)
        elif (win_cap // 2) // P >= STAGE_SEGMENT_MIN:
            win_cap //= 2
        win_rows = win_rows * win_cap // caps["stage_window"]
        self.window_cap = win_cap
        # A window holds every entry of its rows: rows longer than a quarter window go to the
        # panel part whatever their length per panel, so that windows stay nearly full.
        long_mask = long_mask | (lengths > caps["stage_window"] // 8)
        short_len = torch.where(long_mask, 0, lengths)

        # 1. Windows: consecutive rows whose short entries start in [kC, (k + 1) C), so that
        #    a window holds at most C - 1 + (the longest short row) <= win_cap entries, cut
        #    again wherever a window would pass win_rows rows.
        maxlen = int(short_len.max().item()) if n_rows else 0
        C = win_cap - maxlen + 1 if maxlen > 0 else win_cap
        start = torch.cumsum(short_len, 0) - short_len
        w0 = start // C
        n_w0 = int(w0[-1].item()) + 1 if n_rows else 0
        w0_first = torch.searchsorted(w0, torch.arange(n_w0, device=dev))
        sub = (torch.arange(n_rows, device=dev) - w0_first[w0]) // win_rows
        key = w0 * (n_rows // win_rows + 2) + sub
        _, win_of_row = torch.unique_consecutive(key, return_inverse=True)
        del key, sub, w0, w0_first, start
        W = int(win_of_row[-1].item()) + 1 if n_rows else 0
        win_row0 = torch.searchsorted(win_of_row, torch.arange(W, device=dev))
        win_rows_n = torch.diff(win_row0, append=win_row0.new_full((1,), n_rows))
        short_end = torch.cumsum(short_len, 0)  # entries of the rows up to each one
        sstart = short_end - short_len
        win_first = sstart[win_row0] if W else sstart[:0]
        win_len = torch.diff(win_first, append=short_end[-1:]) if W else win_first
        if W and (int(win_len.max().item()) > win_cap or int(win_rows_n.max().item()) > win_rows):
            raise AssertionError("staged-x windows: a window past its caps")
        self.n_windows = W

        # 2. Short entries (CSR order) and their panels.  Staged order (panel, window, row); a
        #    segment is one (panel, window) pair's entries, its first marked in the 16-bit
        #    column.  Each panel's segments fill chunks of `chunk` entries, a chunk closing
        #    early rather than hold more than 64 segments (the kernel's offsets per chunk, the
        #    panel layout's chunk planner with segments for runs); the rest is padding.
        n_short = int(short_end[-1].item()) if n_rows else 0
        self.n_entries = n_short
        ar = torch.arange(n_short, device=dev)
        short_rows = torch.nonzero(short_len).flatten()
        er = torch.repeat_interleave(short_rows, short_len[short_rows], output_size=n_short)
        del short_rows
        pick = rp[er] + (ar - sstart[er])  # the short entries' CSR positions, in order
        ec = cols[pick].to(torch.int64)
        pan = ec >> cb
        ew = win_of_row[er]
        Wk = max(W, 1)
        key = pan * Wk + ew
        if P * Wk < (1 << 31):
            key = key.to(torch.int32)  # half the radix passes
        ks, perm = torch.sort(key, stable=True)  # stable: row order inside a segment
        del key
        seg_start = torch.ones(n_short, dtype=torch.bool, device=dev)
        if n_short > 1:
            seg_start[1:] = ks[1:] != ks[:-1]
        seg_id = torch.cumsum(seg_start, 0) - 1  # segments numbered in staged order
        first_e = torch.nonzero(seg_start).flatten()  # each segment's first sorted entry
        n_seg = int(first_e.numel())
        self.n_segments = n_seg
        seg_len = torch.diff(first_e, append=torch.tensor([n_short], device=dev))
        seg_ks = ks[first_e].to(torch.int64)  # each segment's (panel, window) key
        seg_panel = seg_ks // Wk
        panel_segs = torch.zeros(P + 1, dtype=torch.int64, device=dev)
        torch.cumsum(torch.bincount(seg_panel, minlength=P), 0, out=panel_segs[1:])
        seg_pos, panel_end = plan_panel_chunks(panel_segs, seg_len, chunk, 64)
        seg_pos = seg_pos.to(device=dev, dtype=torch.int64)
        panel_end = panel_end.to(device=dev, dtype=torch.int64)
        n_staged = int(panel_end[-1].item()) if P else 0
        if n_staged > (1 << 30) or n_short > _INDEX_LIMIT_INT32 - 64:
            raise ValueError("too many entries for the staged-x layout")
        self.n_staged = n_staged
        panel_len = torch.diff(panel_end, prepend=panel_end.new_zeros(1))
        pstart = panel_end - panel_len
        spos = seg_pos[seg_id] + ar - first_e[seg_id]  # staged position of every sorted entry
        sc = torch.zeros(n_staged + chunk, dtype=torch.int32, device=dev)
        sc[spos] = (ec[perm] & ((1 << cb) - 1)).to(torch.int32) | \
            (seg_start.to(torch.int32) << 15)
        self.scol = torch.where(sc >= (1 << 15), sc - (1 << 16), sc).to(torch.int16)
        del sc
        # per chunk: the segment of its first entry (always a real one) and its entries in use
        n_chunks = n_staged // chunk
        self.stage_info = torch.zeros((max(n_chunks, 1), 2), dtype=torch.int32, device=dev)
        if n_chunks:
            real = torch.zeros(n_staged, dtype=torch.bool, device=dev)
            real[spos] = True
            seg_at = torch.zeros(n_staged, dtype=torch.int64, device=dev)
            seg_at[spos] = seg_id
            rv = real.view(n_chunks, chunk)
            if not bool(rv[:, 0].all()) or bool((rv[:, 1:] & ~rv[:, :-1]).any()):
                raise AssertionError("staged-x chunks: padding before an entry")
            self.stage_info[:, 0] = seg_at[::chunk].to(torch.int32)
            self.stage_info[:, 1] = rv.sum(1).to(torch.int32)
            del real, seg_at, rv

        # 3. The jobs of the first launch: panel p's chunks of long rows (if any) and its
        #    staged chunks are split evenly over n_p >= 1 jobs, n_p the most of what its long
        #    chunks need (PANEL_JOB_CHUNKS each) and its share of about STAGE_JOBS jobs for all
        #    the staged chunks (rounded: panels of about the average share keep one job), so
        #    that a matrix without long rows still fills the GPU.
        long_rows = torch.nonzero(long_mask).flatten()
        self.long = None
        chunk0 = torch.zeros(P + 1, dtype=torch.int64, device=dev)
        if long_rows.numel():
            long_ptr = torch.zeros(long_rows.numel() + 1, dtype=torch.int64, device=dev)
            torch.cumsum(lengths[long_rows], 0, out=long_ptr[1:])
            n_long = self.nnz - n_short
            lr = torch.repeat_interleave(torch.arange(long_rows.numel(), device=dev),
                                         lengths[long_rows], output_size=n_long)
            lpick = rp[long_rows][lr] + (torch.arange(n_long, device=dev) - long_ptr[lr])
            del lr
            self.long = PanelLayout(data[lpick], cols[lpick], long_ptr, n_cols, long_rows)
            del lpick
            lg = self.long
            if lg.col_bits != cb or lg.n_panels != P:
                raise AssertionError("staged-x layout: the panel parts disagree on the panels")
            chunk0[:P] = lg.panel_chunk0.to(torch.int64)
            chunk0[P] = int(lg.jobs[-1].item())
        per_panel = chunk0[1:] - chunk0[:-1]
        sch = panel_len // chunk  # staged chunks per panel
        per_job = max(-(-STAGE_JOB_MIN // chunk), -(-n_chunks // STAGE_JOBS))
        nj = torch.maximum((per_panel + PANEL_JOB_CHUNKS - 1) // PANEL_JOB_CHUNKS,
                           (2 * sch + per_job) // (2 * per_job)).clamp(min=1)
        job_panel = torch.repeat_interleave(torch.arange(P, device=dev), nj)
        n_jobs = int(job_panel.numel())
        k = torch.arange(n_jobs, device=dev) - (torch.cumsum(nj, 0) - nj)[job_panel]
        starts = chunk0[job_panel] + k * per_panel[job_panel] // nj[job_panel]
        self.jobs = torch.cat([starts, chunk0[P:]]).to(torch.int32).contiguous()
        self.job_panel = job_panel.to(torch.int32).contiguous()
        self.n_jobs = n_jobs
        s_lo = pstart[job_panel] // chunk + k * sch[job_panel] // nj[job_panel]
        self.stage_jobs = torch.cat([s_lo, torch.tensor([n_chunks], device=dev)]).to(
            torch.int32).contiguous()
        del k, starts

        # 4. Window order: in each window its segments by (XCD of the job that stages it -
        #    workgroup j runs on XCD j mod 8 -, panel), so that the XCD's jobs write the lines
        #    of their segments together; every entry's values, LDS position (its rank in the
        #    window's (row, panel) order) and staged x there; seg_delta takes a segment's staged
        #    positions to its window positions.
        seg_chunk = seg_pos // chunk
        seg_job = torch.searchsorted(s_lo, seg_chunk, right=True) - 1
        seg_key = (seg_ks % Wk) * (XCD_COUNT * P) + \
            (seg_job % XCD_COUNT) * P * int(STAGE_XCD_ORDER) + seg_ks // Wk
        seg_order = torch.sort(seg_key)[1]
        ordered_len = seg_len[seg_order]
        seg_wpos = torch.empty_like(seg_len)
        seg_wpos[seg_order] = torch.cumsum(ordered_len, 0) - ordered_len  # window-major start
        # each window starts at a multiple of 8 entries (the combine's 16-byte loads)
        win_pad = (win_len + 7) // 8 * 8
        win_start = torch.cumsum(win_pad, 0) - win_pad
        n_pos = int((win_start[-1] + win_pad[-1]).item()) if W else 0
        if n_pos > _INDEX_LIMIT_INT32 - 64:
            raise ValueError("too many entries for the staged-x layout")
        seg_wpos += (win_start - win_first)[seg_ks % Wk]
        del seg_key, seg_order, ordered_len, seg_chunk, seg_job, s_lo, win_pad
        sdelta = torch.zeros(n_seg + 64, dtype=torch.int64, device=dev)
        sdelta[:n_seg] = seg_wpos - seg_pos
        self.seg_delta = sdelta.to(torch.int32).contiguous()
        wpos = seg_wpos[seg_id] + ar - first_e[seg_id]
        del seg_len, seg_wpos, first_e, seg_start, seg_id, spos, seg_pos
        # rank in (row, panel) order: CSR order is row order, and where each row's panels
        # already rise (sorted columns) it is the CSR order itself; else a stable sort
        unordered = n_short > 1 and bool(((er[1:] == er[:-1]) & (pan[1:] < pan[:-1])).any())
        if unordered:
            order2 = torch.sort(er * P + pan, stable=True)[1]
            rank = torch.empty_like(order2)
            rank[order2] = ar
            del order2
        else:
            rank = ar
        del ar
        slot = rank - win_first[ew]
        del rank
        self.n_positions = n_pos
        self.vals = torch.zeros(n_pos + 8, dtype=data.dtype, device=dev)
        self.vals[wpos] = data[pick][perm]
        dest = torch.zeros(n_pos + 8, dtype=torch.int32, device=dev)
        dest[wpos] = slot[perm].to(torch.int32)
        self.dest = dest.to(torch.int16)
        self.xs = torch.zeros(n_pos + 8, dtype=data.dtype, device=dev)
        del dest, slot, wpos, perm, pick, ec, pan, ew, er, ks
        # per row the end of its positions in its window (| 0x8000: a row left to the panel
        # part); per window a bit per position where a row starts
        rstart = sstart - win_first[win_of_row] if n_rows else sstart
        re = (rstart + short_len) | torch.where(long_mask, 0x8000, 0)
        self.row_end = torch.where(re >= (1 << 15), re - (1 << 16), re).to(torch.int16)
        del re
        opens = torch.nonzero(short_len > 0).flatten()
        bits = torch.zeros(W * win_cap + 8, dtype=torch.uint8, device=dev)
        bits[rstart[opens] + win_of_row[opens] * win_cap] = 1
        weight = torch.tensor([1, 2, 4, 8, 16, 32, 64, 128], dtype=torch.uint8, device=dev)
        self.heads = (bits.view(-1, 8) * weight).sum(1, dtype=torch.uint8)
        del bits, opens, rstart
        self.windows = torch.stack([win_row0, win_rows_n, win_len, win_start], 1).to(
            torch.int32).contiguous()
        self._keep = (self.scol, self.stage_info, self.seg_delta, self.xs, self.vals, self.dest,
                      self.row_end, self.heads, self.windows, self.jobs, self.job_panel,
                      self.stage_jobs)
        if self.long is not None:
            self._keep = self._keep + self.long._keep
        self._args = {}
        self._order = StreamOrder(dev)

    def kernel_name(self):
        return "spmv_panel_kernel+stage_combine_kernel"

    def held_bytes(self, caller=()):
        own = tensor_bytes(*self._keep[:12])
        return own + (self.long.held_bytes(caller) if self.long is not None else 0)

    def describe(self):
        d = {"layout": self.kind, "panels": self.n_panels, "col_bits": self.col_bits,
             "window_cap": self.window_cap,
             "staged_entries": self.n_entries, "segments": self.n_segments,
             "windows": self.n_windows, "jobs": self.n_jobs,
             "long_rows": 0 if self.long is None else self.long.n_rows,
             "long_entries": 0 if self.long is None else self.long.nnz}
        if self.long is not None:
            d["panel_part"] = self.long.describe()
        return d

    def launch(self, x, y, acc_f64, row_map=None, n_out=0, passes=3):
        """Both launches (passes=3), or only the panel jobs (1: long-row partial sums and the
        staged x) or only the row sums (2), on the caller's stream."""
        args = self._args.get(bool(acc_f64))
        if args is None:  # static arguments converted once per accumulation mode
            p = lambda t: t.data_ptr() if t is not None and t.numel() else None  # noqa: E731
            lg = self.long
            dt = _abi.dtype_code(self.vals.dtype)
            first = [dt, int(acc_f64), p(lg.vals) if lg else None,
                     p(lg.pcol) if lg else None, lg.n_entries if lg else 0, self.col_bits, None,
                     self.n_cols, None, None, p(self.jobs), p(self.job_panel), self.n_jobs,
                     p(lg.chunk_info) if lg else None, p(lg.partials) if lg else None,
                     int(lg.partials.numel()) if lg else 0, None, None, None, 0, p(self.scol),
                     self.n_staged, p(self.stage_jobs), p(self.stage_info), p(self.seg_delta),
                     p(self.xs), int(self.xs.numel()), None]
            second = [dt, int(acc_f64), None, None, 0, p(self.windows), self.n_windows,
                      self.window_cap, p(self.vals), p(self.dest), p(self.xs),
                      int(self.vals.numel()),
                      p(self.row_end), p(self.heads), p(lg.partials) if lg else None,
                      p(lg.rows) if lg else None, p(lg.row_ptr) if lg else None,
                      p(lg.slots) if lg else None, lg.n_rows if lg else 0, None]
            args = (first, second)
            self._args[bool(acc_f64)] = args
        st = self._order.stream(y.device, self._keep)
        L = _abi.lib()
        if passes & 1:
            a = list(args[0])
            a[6], a[8] = x.data_ptr(), y.data_ptr()
            a[27] = st
            _abi.check(L.fsp_spmv_panels(*a), "fsp_spmv_panels")
        if passes & 2:
            a = list(args[1])
            a[2] = y.data_ptr()
            a[3] = None if row_map is None else row_map.data_ptr()
            a[4] = n_out
            a[19] = st
            _abi.check(L.fsp_spmv_stage_combine(*a), "fsp_spmv_stage_combine")
        return y


def sample_indices(n, k, device):
    """min(n, k) indices spread evenly over [0, n), computed in exact int64 arithmetic."""
    if n <= k:
        return torch.arange(n, device=device)
    return torch.arange(k, device=device, dtype=torch.int64) * (n - 1) // (k - 1)


def prefers_xcs(cols, rowptr, n_cols, value_bytes):
    """True when most entries gather x far from their row's diagonal position and x does not
    fit one XCD's L2 (the row-block layout would then miss L2 on almost every gather)."""
    nnz = int(cols.numel())
    n_rows = int(rowptr.numel()) - 1
    if nnz == 0 or n_rows == 0 or int(n_cols) * value_bytes <= L2_BYTES:
        return False
    idx = sample_indices(nnz, SAMPLE, cols.device)
    rp = rowptr.to(torch.int64)
    rows = torch.searchsorted(rp, idx, right=True) - 1
    diag = rows.to(torch.float64) * (float(n_cols) / float(n_rows))
    far = (cols[idx].to(torch.float64) - diag).abs() > NEAR_COLUMNS
    return bool(far.to(torch.float32).mean().item() > 0.5)


def _entries_per_panel_run(lengths, P):
    """Expected entries per (row, panel) pair for rows of the given lengths with columns spread
    evenly over P panels: a row of k entries reaches P (1 - (1 - 1/P)^k) panels."""
    k = lengths.to(torch.float64)
    reached = float((P * (1.0 - torch.pow(1.0 - 1.0 / P, k))).sum().item())
    return float(k.sum().item()) / reached if reached > 0 else 0.0


def xcs_layout(data, cols, rowptr, n_cols, panels_per_xcd=None):
    """XcsLayout with sorted-gather items where they fit, else the row-order items: the taller
    tiles of the sorted format can reach more combine windows than an item's run table holds
    (rows with many sums, small windows).  ValueError when neither packing fits."""
    try:
        return XcsLayout(data, cols, rowptr, n_cols, panels_per_xcd)
    except ValueError:
        if not SORTED_ITEMS:
            raise
    return XcsLayout(data, cols, rowptr, n_cols, panels_per_xcd, item_format=0)


def build_layout(data, cols, rowptr, n_cols, one_shot=False):
    """The layout for one CSR (or COO row-run) matrix: XCS when it pays, else row blocks.
    one_shot: the layout serves a single call (no prepared object), so the row-block layout,
    which builds in about a millisecond, is taken; the XCS layouts take tens of milliseconds to
    build (cfg3: 46 ms for a 0.32 ms product, against 3.3 ms for the row-block product)."""
    mode = FORCE
    nnz = int(data.numel())
    if mode is None and one_shot:
        mode = "rowblock"
    if mode is None:
        mode = ("xstage" if STAGED else "xcs") \
            if prefers_xcs(cols, rowptr, n_cols, data.element_size()) else "rowblock"
    if mode == "xstage" and nnz <= _INDEX_LIMIT_INT32 // 2 and int(rowptr.numel()) > 1:
        rp = rowptr.to(torch.int64)
        lengths = rp[1:] - rp[:-1]
        try:
            return XstageLayout(data, cols, rowptr, n_cols,
                                lengths >= panel_row_min(n_cols, data.element_size()))
        except ValueError:
            mode = "xcs"  # x too wide for the staged-x combine: the XCS layouts
    if mode in ("xcs", "xcs-l2", "xcs-hybrid") and nnz <= _INDEX_LIMIT_INT32 // 2 and \
            int(n_cols) <= (1 << 27) and int(rowptr.numel()) > 1:
        if mode != "xcs-l2":
            rp = rowptr.to(torch.int64)
            lengths = rp[1:] - rp[:-1]
            long_mask = lengths >= panel_row_min(n_cols, data.element_size())
            long_nnz = int(lengths[long_mask].sum().item())
            if long_nnz > 0 and (mode == "xcs-hybrid" or long_nnz >= PANEL_MIN_SHARE * nnz):
                try:
                    return XcsHybridLayout(data, cols, rowptr, n_cols, long_mask,
                                           FORCE_PANELS_PER_XCD)
                except ValueError:
                    pass  # a part too large for its packing: XCS alone, else row blocks
        try:
            return xcs_layout(data, cols, rowptr, n_cols, FORCE_PANELS_PER_XCD)
        except ValueError:
            pass  # too large for the packing: row blocks
    return RowBlockLayout(data, cols, rowptr)


__all__ = ["RowBlockLayout", "XcsLayout", "PanelLayout", "XcsHybridLayout", "XstageLayout",
           "build_layout",
           "xcs_layout",
           "prefers_xcs", "sample_indices", "FORCE"]
