"""C-ABI library checks that need no GPU: it loads, exports every function declared in
include/flagsparse_hip.h, reports its capacities, and its host-side row-block planner
(fsp_plan_row_blocks) produces tables with the invariants the kernels rely on.  Argument
checks of the kernel entry points are exercised where they reject a call before any HIP
runtime call is made."""

import ctypes
import os
import re

import numpy as np
import pytest

import flagsparse_amd as fs
from flagsparse_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flagsparse_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fsp_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_abi.LIB_PATH)
    names = _declared_functions()
    assert len(names) >= 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes table covers exactly the declared functions
    assert sorted(_abi.SIGNATURES) == names


_CTYPE = {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "double": ctypes.c_double}


def _declared_signatures():
    """{name: (return ctype, [argument ctypes])} parsed from the header's prototypes."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    sigs = {}
    for ret, name, params in re.findall(r"\b(int|int64_t|const char\*)\s+(fsp_\w+)\s*\(([^)]*)\)\s*;",
                                        text):
        args = []
        params = params.strip()
        if params and params != "void":
            for prm in params.split(","):
                prm = " ".join(prm.split())
                if prm.startswith("const char*"):
                    args.append(ctypes.c_char_p)
                else:
                    args.append(ctypes.c_void_p if "*" in prm else _CTYPE[prm.rsplit(" ", 1)[0]])
        sigs[name] = (ctypes.c_char_p if "char" in ret else _CTYPE[ret], args)
    return sigs


def test_ctypes_table_matches_header_prototypes():
    sigs = _declared_signatures()
    assert sorted(sigs) == _declared_functions()
    for name, (ret, args) in sigs.items():
        want_ret, want_args = _abi.SIGNATURES[name]
        assert want_ret == ret, name
        assert list(want_args) == args, name


def test_abi_version_and_caps():
    L = _abi.lib()
    assert L.fsp_abi_version() == _abi.ABI_VERSION
    caps = _abi.caps()
    assert caps["spmv_stream_nnz"] >= 1 and caps["spmv_chunk_nnz"] >= caps["spmv_stream_nnz"]
    assert caps["spmv_stream_rows"] >= 1 and caps["spmm_block_nnz"] >= 1
    assert L.fsp_last_error() is not None


def _plan(rowptr, nnz_cap, rows_cap, thr, chunk):
    L = _abi.lib()
    rp = np.ascontiguousarray(rowptr, dtype=np.int64)
    nd, npart, nsplit = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    args = (rp.ctypes.data_as(ctypes.c_void_p), rp.size - 1, nnz_cap, rows_cap, thr, chunk)
    rc = L.fsp_plan_row_blocks(*args, None, ctypes.byref(nd), ctypes.byref(npart),
                               ctypes.byref(nsplit))
    if rc != 0:
        return rc, L.fsp_last_error().decode(), None, None, None
    desc = np.zeros((nd.value, 4), dtype=np.int32)
    rc = L.fsp_plan_row_blocks(*args, desc.ctypes.data_as(ctypes.c_void_p), ctypes.byref(nd),
                               ctypes.byref(npart), ctypes.byref(nsplit))
    return rc, desc, npart.value, nsplit.value, None


def _check_plan(lengths, nnz_cap, rows_cap, thr, chunk):
    rowptr = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    rc, desc, n_parts, n_split, _ = _plan(rowptr, nnz_cap, rows_cap, thr, chunk)
    assert rc == 0, desc
    n = len(lengths)
    next_row = 0
    part_cursor = 0
    split_rows = 0
    i = 0
    while i < desc.shape[0]:
        a, b, c, d = (int(v) for v in desc[i])
        if c == 0:  # short-row block [a, b)
            assert a == next_row and b > a
            assert b - a <= rows_cap
            blk = lengths[a:b]
            assert np.all(blk <= thr) and blk.sum() <= nnz_cap
            # greedy: the block stops only where the next row breaks a cap
            if b < n:
                nxt = lengths[b]
                assert b - a == rows_cap or nxt > thr or blk.sum() + nxt > nnz_cap
            next_row = b
            i += 1
        else:  # chunks of a long row
            row, nch = a, c
            assert row == next_row and lengths[row] > thr
            assert nch == -(-lengths[row] // chunk)
            for k in range(nch):
                assert tuple(int(v) for v in desc[i + k][:3]) == (row, k, nch)
                assert int(desc[i + k][3]) == (part_cursor if nch > 1 else -1)
            if nch > 1:
                part_cursor += nch
                split_rows += 1
            next_row = row + 1
            i += nch
    assert next_row == n
    assert n_parts == part_cursor and n_split == split_rows
    # the entry ranges handed to the kernels: consecutive, covering [0, nnz) exactly once
    from flagsparse_amd._plan import build_row_block_plan
    plan = build_row_block_plan(rowptr, None, nnz_cap, rows_cap, thr, chunk)
    rg = plan.ranges.numpy()
    if rg.shape[0]:
        assert rg[0, 0] == 0 and rg[-1, 1] == rowptr[-1]
        assert np.array_equal(rg[1:, 0], rg[:-1, 1]) and np.all(rg[:, 1] >= rg[:, 0])


@pytest.mark.parametrize("seed", range(4))
def test_planner_invariants_random(seed):
    rng = np.random.default_rng(seed)
    lengths = rng.zipf(1.7, 3000).clip(max=20000) - 1 + (rng.random(3000) < 0.2)
    lengths[rng.integers(0, 3000, 50)] = 0
    for nnz_cap, rows_cap, thr, chunk in ((2045, 1024, 2045, 4093), (2045, 16, 128, 512),
                                         (100, 7, 50, 33), (1, 1, 1, 1)):
        _check_plan(lengths.astype(np.int64), nnz_cap, rows_cap, thr, chunk)


def test_planner_edges():
    _check_plan(np.zeros(0, dtype=np.int64), 10, 4, 5, 5)
    _check_plan(np.zeros(5000, dtype=np.int64), 2045, 1024, 2045, 4093)
    _check_plan(np.array([2045, 2046, 4093, 4094, 1, 0]), 2045, 1024, 2045, 4093)


def test_planner_rejects_bad_arguments():
    rp = np.array([0, 3, 2], dtype=np.int64)
    rc, msg, *_ = _plan(rp, 10, 4, 5, 5)
    assert rc == -1 and "non-decreasing" in msg  # FSP_EINVAL
    rc, msg, *_ = _plan(np.array([0, 1]), 10, 4, 11, 5)  # long_threshold > nnz_cap
    assert rc == -1 and "long_threshold" in msg
    rc, msg, *_ = _plan(np.array([0, 1]), 10, 0, 5, 5)
    assert rc == -1


def test_panel_chunk_planner_rejects_bad_arguments():
    L = _abi.lib()
    pr = np.array([0, 2], dtype=np.int64)
    pos = np.zeros(2, dtype=np.int64)
    end = np.zeros(1, dtype=np.int64)

    def plan(run_len, panel_runs=pr, chunk=8, cap=2, n_panels=1):
        rl = np.asarray(run_len, dtype=np.int64)
        return L.fsp_plan_panel_chunks(panel_runs.ctypes.data, n_panels, rl.ctypes.data, chunk,
                                       cap, pos.ctypes.data, end.ctypes.data)

    assert plan([3, 4]) == 0 and pos.tolist() == [0, 3] and end.tolist() == [8]
    assert plan([3, 0]) == -1 and b"empty run" in L.fsp_last_error()
    assert plan([3, 4], chunk=0) == -1
    assert plan([3, 4], cap=0) == -1
    assert plan([3, 4], panel_runs=np.array([1, 2], dtype=np.int64)) == -1
    assert plan([3, 4], panel_runs=np.array([0, 2, 1], dtype=np.int64), n_panels=2) == -1
    assert L.fsp_plan_panel_chunks(None, 1, None, 8, 2, None, None) == -1  # null pointers
    assert L.fsp_plan_panel_chunks(None, 0, None, 8, 2, None, None) == 0   # nothing to plan


def test_device_planner_rejects_bad_arguments():
    L = _abi.lib()
    # (rowptr, bits, n_rows, window_rows, nnz_cap, rows_cap, long_threshold, chunk, counts,
    #  stream)
    assert L.fsp_plan_windows_count(None, 16, 0, 4, 10, 4, 5, 5, None, None) == -1
    assert b"rowptr_bits" in L.fsp_last_error()
    assert L.fsp_plan_windows_count(None, 32, 0, 4, 10, 4, 11, 5, None, None) == -1
    assert b"long_threshold" in L.fsp_last_error()
    assert L.fsp_plan_windows_count(None, 32, 0, 0, 10, 4, 5, 5, None, None) == -1
    assert b"window_rows" in L.fsp_last_error()
    assert L.fsp_plan_windows_count(None, 32, 3, 4, 10, 4, 5, 5, None, None) == -1  # null rowptr
    assert L.fsp_plan_windows_emit(None, 64, -1, 4, 10, 4, 5, 5, None, None, None, None, None,
                                   None, None) == -1
    assert L.fsp_plan_windows_count(None, 32, 0, 4, 10, 4, 5, 5, None, None) == 0  # nothing


def test_kernel_entry_points_reject_before_any_hip_call():
    L = _abi.lib()

    def spmv(dtype=0, bits=32, chunk=1, n_groups=0):
        return L.fsp_spmv_csr(dtype, 0, None, None, None, bits, 0, 0, None, None, None, 0, None,
                              None, 0, chunk, None, None, None, None, n_groups, 0, None)

    def spmm(dtype=0, lanes=1, vec=1):
        return L.fsp_spmm_csr(dtype, 0, None, None, None, 32, 0, 0, None, 0, 0, None, 0, None, 0,
                              1, lanes, vec, None, None, None, None, 0, 0, None)

    assert spmv(dtype=7) == -3                    # unsupported dtype code
    assert b"dtype" in L.fsp_last_error()
    assert spmv(bits=16) == -1                    # bad rowptr width
    assert spmv(chunk=10**9) == -1                # chunk beyond the compiled capacity
    assert spmv(n_groups=3) == -1                 # split-row groups without their arrays
    assert b"split-row" in L.fsp_last_error()
    # the allocation-free variant refuses a plan larger than its static workspace before it
    # resolves the workspace (no HIP call)
    cap = L.fsp_spmv_scratch_slots()
    assert cap == 1 << 17
    assert L.fsp_spmv_csr_static(0, 0, None, None, None, 32, 0, 0, None, None, None, 0, None,
                                 None, 0, 1, cap + 1, None, None, None, 0, 0, None) == -1
    assert b"static workspace" in L.fsp_last_error()
    assert spmm(lanes=3) == -1                    # lanes_per_row not a power of two
    assert spmm(dtype=1, lanes=4, vec=4) == -1    # 4-wide vectors are fp32 only
    def xcs(col_bits=10, n_windows=0, item_format=0):
        return L.fsp_spmv_xcs(0, 0, None, None, 0, col_bits, None, None, None, 0, None, 0, None,
                              None, None, n_windows, 1024, None, None, item_format, None)

    # fsp_index_stats(a, a_bits, b, b_bits, n, partial, out, stream)
    assert L.fsp_index_stats(None, 16, None, 32, 0, None, None, None) == -1
    assert b"widths" in L.fsp_last_error()
    assert L.fsp_index_stats(None, 32, None, 32, -1, None, None, None) == -1
    assert L.fsp_index_stats(None, 32, None, 64, 0, None, None, None) == -1  # null partial
    assert b"null" in L.fsp_last_error()
    assert L.fsp_index_stats_partial_len() == 5 * 1024

    assert xcs() == 0                             # nothing to run
    assert xcs(col_bits=25) == -1                 # col_bits > 24
    assert xcs(n_windows=4) == -1                 # combine without its tables
    assert b"null" in L.fsp_last_error()
    assert xcs(item_format=2) == -1               # no such item format
    assert xcs(col_bits=20, item_format=1) == -1  # sorted-gather items take <= 19 column bits
    assert b"col_bits" in L.fsp_last_error()
    assert xcs(col_bits=19, item_format=1) == 0
    assert L.fsp_spmv_coo_atomic(0, None, None, None, -1, None, None, 0, 1, None) == -1

    def panels(dtype=0, n_entries=0, col_bits=10, n_jobs=0, n_rows=0, n_partials=0,
               n_staged=0):
        return L.fsp_spmv_panels(dtype, 0, None, None, n_entries, col_bits, None, 1, None, None,
                                 None, None, n_jobs, None, None, n_partials, None, None, None,
                                 n_rows, None, n_staged, None, None, None, None, 0, None)

    assert panels() == 0                          # nothing to run
    assert panels(dtype=5) == -3
    assert panels(n_entries=100) == -1            # not a whole number of chunks
    assert b"multiple" in L.fsp_last_error()
    assert panels(n_partials=1 << 28) == -1       # partials beyond the buffer resource range
    assert b"partial" in L.fsp_last_error()
    assert panels(col_bits=16) == -1              # beyond the 16-bit entries (and 128 KiB)
    assert panels(dtype=1, col_bits=15) == -1     # 2^15 fp64 > 128 KiB of LDS
    assert b"LDS" in L.fsp_last_error()
    assert panels(n_entries=512, n_jobs=1) == -1  # jobs without arrays
    assert panels(n_rows=3) == -1                 # combine without its arrays
    assert b"null" in L.fsp_last_error()
    # a chunk table that is not 8-byte aligned (two int32 per chunk): refused before any
    # launch (the other pointers are never dereferenced on the host)
    fake = 1 << 20
    assert L.fsp_spmv_panels(0, 0, fake, fake, 512, 10, fake, 1024, None, None, fake, fake, 1,
                             fake + 4, fake, 64, None, None, None, 0, None, 0, None, None, None,
                             None, 0, None) == -1
    assert b"chunk_info" in L.fsp_last_error() and b"aligned" in L.fsp_last_error()
    # staging (the staged-x layout's first pass): whole chunks, its arrays given
    chunk = L.fsp_stage_chunk()
    assert chunk == 512
    assert panels(n_staged=100) == -1
    assert b"multiple" in L.fsp_last_error()
    assert L.fsp_spmv_panels(0, 0, None, None, 0, 10, fake, 1024, None, None, fake, fake, 1,
                             None, None, 0, None, None, None, 0, None, chunk, None, None, None,
                             None, 4, None) == -1
    assert b"staging" in L.fsp_last_error()
    assert L.fsp_spmv_panels(0, 0, None, None, 0, 10, fake, 1024, None, None, fake, fake, 1,
                             None, None, 0, None, None, None, 0, fake, chunk, fake, fake + 4,
                             fake, fake, 4, None) == -1
    assert b"stage_info" in L.fsp_last_error() and b"aligned" in L.fsp_last_error()

    def stage(dtype=0, n_windows=0, n_rows=0, tables=False):
        t = fake if tables else None
        return L.fsp_spmv_stage_combine(dtype, 1, t, None, 0, t, n_windows, 4096, t, t, t, 64,
                                        t, t, None, None, None, None, n_rows, None)

    assert stage() == 0                           # nothing to run
    assert stage(dtype=7) == -3
    assert stage(n_windows=2) == -1               # windows without their tables
    assert b"null" in L.fsp_last_error()
    assert stage(n_rows=4) == -1                  # panel rows without their arrays
    assert b"panel-row" in L.fsp_last_error()
    assert L.fsp_spmv_stage_combine(0, 1, fake, None, 0, fake + 4, 2, 4096, fake, fake, fake,
                                    64, fake, fake, None, None, None, None, 0, None) == -1
    assert b"windows" in L.fsp_last_error() and b"aligned" in L.fsp_last_error()
    assert L.fsp_spmv_stage_combine(0, 1, fake, None, 0, fake, 2, 1000, fake, fake, fake, 64,
                                    fake, fake, None, None, None, None, 0, None) == -1
    assert b"window_cap" in L.fsp_last_error()
    for k in range(3):  # vals, dest, xs: 16-byte loads
        tabs = [fake + 8 if j == k else fake for j in range(3)]
        assert L.fsp_spmv_stage_combine(0, 1, fake, None, 0, fake, 2, 4096, *tabs, 64, fake,
                                        fake, None, None, None, None, 0, None) == -1
        assert b"16-byte" in L.fsp_last_error()
    assert L.fsp_stage_window_cap() == 8192 and L.fsp_stage_window_rows_cap() == 4096


def test_build_flags_kernels_with_scratch():
    # the build reads each kernel's resource-usage remarks and refuses one that uses scratch
    # memory per lane (registers spilled, or a local array kept in memory)
    from flagsparse_amd import _build

    log = "\n".join([
        "a.hip:1:1: remark: Function Name: _Z4goodPf [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     VGPRs: 40 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark: Function Name: _Z3badPf [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark:     ScratchSize [bytes/lane]: 12 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert _build._scratch_kernels(log) == {"_Z3badPf"}
    assert _build._scratch_kernels("") == set()
