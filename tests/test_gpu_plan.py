"""The device row-block planner (fsp_plan_windows_count / _emit) on the GPU.

Its contract: the rows are cut into windows of window_rows rows and each window is planned
with the host planner's rules (fsp_plan_row_blocks).  So the device table must equal, exactly,
the concatenation of host-planner tables of the windows (row ids and partial-slot bases
shifted), and its entry ranges and combine groups must match the descriptors.  Windows wider
than rows_cap with long_threshold == nnz_cap take the binary-search block end; with
long_threshold < nnz_cap the row-by-row scan; a single window reproduces the host plan.
"""

import ctypes

import numpy as np
import pytest
import torch

from flagsparse_amd import _abi
from flagsparse_amd._plan import build_row_block_plan_device

pytestmark = pytest.mark.gpu

CAPS = [(2045, 16, 128, 2045), (2045, 64, 128, 1024), (2045, 256, 128, 256),
        (2045, 1024, 2045, 4093), (100, 7, 50, 33), (1, 1, 1, 1)]


def _host_plan(rowptr, nnz_cap, rows_cap, thr, chunk):
    L = _abi.lib()
    rp = np.ascontiguousarray(rowptr, dtype=np.int64)
    nd, npart, nsplit = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    args = (rp.ctypes.data_as(ctypes.c_void_p), rp.size - 1, nnz_cap, rows_cap, thr, chunk)
    assert L.fsp_plan_row_blocks(*args, None, ctypes.byref(nd), ctypes.byref(npart),
                                 ctypes.byref(nsplit)) == 0
    desc = np.zeros((nd.value, 4), dtype=np.int64)
    d32 = np.zeros((nd.value, 4), dtype=np.int32)
    assert L.fsp_plan_row_blocks(*args, d32.ctypes.data_as(ctypes.c_void_p), ctypes.byref(nd),
                                 ctypes.byref(npart), ctypes.byref(nsplit)) == 0
    desc[:] = d32
    return desc, npart.value, nsplit.value


def _windowed_expectation(rowptr, nnz_cap, rows_cap, thr, chunk, window=None):
    n = rowptr.size - 1
    window = rows_cap if window is None else window
    tables, parts, splits = [], 0, 0
    for w0 in range(0, n, window):
        w1 = min(w0 + window, n)
        desc, np_w, ns_w = _host_plan(rowptr[w0:w1 + 1] - rowptr[w0], nnz_cap, rows_cap, thr,
                                      chunk)
        short = desc[:, 2] == 0
        desc[:, 0] += w0
        desc[short, 1] += w0
        split = (~short) & (desc[:, 3] >= 0)
        desc[split, 3] += parts
        tables.append(desc)
        parts += np_w
        splits += ns_w
    desc = np.concatenate(tables) if tables else np.zeros((0, 4), dtype=np.int64)
    return desc, parts, splits


def _lengths(seed, n):
    rng = np.random.default_rng(seed)
    lengths = rng.zipf(1.7, n).clip(max=30000) - 1 + (rng.random(n) < 0.2)
    lengths[rng.integers(0, n, max(1, n // 60))] = 0
    return lengths.astype(np.int64)


@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("caps", CAPS)
@pytest.mark.parametrize("bits", [32, 64])
@pytest.mark.parametrize("wmul", [1, 3, 100])
def test_device_plan_matches_windowed_host_plan(dev, seed, caps, bits, wmul):
    nnz_cap, rows_cap, thr, chunk = caps
    window = rows_cap * wmul
    lengths = _lengths(seed, 3000)
    rowptr = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    rp_dev = torch.from_numpy(rowptr).to(dev).to(torch.int32 if bits == 32 else torch.int64)
    print(f"device plan seed={seed} caps={caps} bits={bits} window={window}", flush=True)
    plan = build_row_block_plan_device(rp_dev, nnz_cap, rows_cap, thr, chunk, window)
    want, parts, splits = _windowed_expectation(rowptr, nnz_cap, rows_cap, thr, chunk, window)
    got = plan.desc.cpu().numpy().astype(np.int64)
    assert np.array_equal(got, want)
    assert (plan.n_parts, plan.n_split_rows) == (parts, splits)
    # entry ranges
    rg = plan.ranges.cpu().numpy()
    short = want[:, 2] == 0
    lo = np.where(short, rowptr[want[:, 0]], rowptr[want[:, 0]] + want[:, 1] * chunk)
    hi = np.where(short, rowptr[np.where(short, want[:, 1], want[:, 0])],
                  np.minimum(lo + chunk, rowptr[np.minimum(want[:, 0] + 1, lengths.size)]))
    assert np.array_equal(rg[:, 0], lo) and np.array_equal(rg[:, 1], hi)
    # combine groups: one per split row, in row order, {s, 1, nch, 0} / first part / row
    groups, base, rows = (t.cpu().numpy() for t in plan.split_groups())
    first = (~short) & (want[:, 3] >= 0) & (want[:, 1] == 0)
    assert np.array_equal(rows, want[first, 0])
    assert np.array_equal(base, want[first, 3])
    assert np.array_equal(groups[:, 0], np.arange(rows.size))
    assert np.all(groups[:, 1] == 1) and np.array_equal(groups[:, 2], want[first, 2])


def test_device_plan_edges(dev):
    for lengths in (np.zeros(0, np.int64), np.zeros(5000, np.int64),
                    np.array([2045, 2046, 4093, 4094, 1, 0], np.int64),
                    np.array([200000], np.int64)):
        rowptr = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
        rp_dev = torch.from_numpy(rowptr).to(dev)
        for caps in ((2045, 16, 128, 2045), (2045, 1024, 2045, 4093)):
            for window in (None, 16 * caps[1]):
                plan = build_row_block_plan_device(rp_dev, *caps, window_rows=window)
                want, parts, splits = _windowed_expectation(rowptr, *caps, window=window)
                assert np.array_equal(plan.desc.cpu().numpy().astype(np.int64), want)
                assert (plan.n_parts, plan.n_split_rows) == (parts, splits)


def test_device_plan_bisect_on_uniform_rows(dev):
    # a Poisson-like pattern (rows of 3..5 entries) in one window equals the host plan, and in
    # windows of 16 * rows_cap differs from it only by blocks cut at window ends
    n = 70000
    rng = np.random.default_rng(5)
    lengths = rng.integers(3, 6, n).astype(np.int64)
    rowptr = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    rp_dev = torch.from_numpy(rowptr).to(dev).to(torch.int32)
    caps = (2045, 1024, 2045, 4093)
    whole = build_row_block_plan_device(rp_dev, *caps, window_rows=n)
    want, _, _ = _host_plan(rowptr, *caps)
    assert np.array_equal(whole.desc.cpu().numpy().astype(np.int64), want)
    wide = build_row_block_plan_device(rp_dev, *caps, window_rows=16 * 1024)
    assert wide.n_desc <= want.shape[0] + -(-n // (16 * 1024))


@pytest.mark.parametrize("seed", range(4))
def test_device_panel_chunk_plan_matches_host(dev, seed):
    # the panel layout's chunk plan on the device (fsp_plan_panel_chunks_device, one thread per
    # panel) equals the host planner on random panels, with run caps that close chunks early
    # and runs longer than a chunk; plan_panel_chunks on device tensors (its prefix route or
    # the kernel) equals it too
    from flagsparse_amd import _spmv_layouts

    rng = np.random.default_rng(40 + seed)
    for chunk in (8, 512):
        for trial in range(12):
            n_panels = int(rng.integers(1, 40))
            counts = rng.integers(0, 300, n_panels)
            counts[rng.integers(0, n_panels)] = 0  # an empty panel
            lens = rng.integers(1, 3 * chunk, int(counts.sum()))
            short = rng.random(lens.size) < rng.random()
            lens[short] = rng.integers(1, 4, int(short.sum()))
            cap = int(rng.integers(1, 70))
            pr = torch.as_tensor(np.r_[0, np.cumsum(counts)])
            rl = torch.as_tensor(lens)
            print(f"panel plan seed {seed} chunk {chunk} trial {trial} cap {cap}", flush=True)
            host = _spmv_layouts.plan_panel_chunks(pr, rl, chunk, cap)
            kern = _spmv_layouts.plan_panel_chunks_kernel(pr.to(dev), rl.to(dev), chunk, cap)
            auto = _spmv_layouts.plan_panel_chunks(pr.to(dev), rl.to(dev), chunk, cap)
            for got in (kern, auto):
                assert torch.equal(got[0].cpu(), host[0]) and torch.equal(got[1].cpu(), host[1])
