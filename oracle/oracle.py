"""CPU oracle for the flagsparse_amd hot path (CSR/COO SpMV, CSR SpMM).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg may import this module, and only as the checker; the product package
``flagsparse_amd`` never imports it.

Two kinds of restatement live here, each citing the FlagSparse source it follows (paths
relative to ``src/flagsparse/sparse_operations/`` unless stated):

* fp64 arithmetic (``spmv_csr``, ``spmv_coo``, ``spmm_csr``, ``spmm_coo``, ``sddmm_csr``):
  thin ctypes wrappers over ``fsp_oracle.c``, a plain row-by-row fp64 sum - the definition of
  correctness every reference test of this path uses (tests/test_spmv.py:143-174,
  tests/test_spmv_coo.py:56-71, tests/test_spmm.py:270-311, tests/test_spmm_coo.py:98-140,
  tests/test_sddmm.py:155-168).
* integer planning semantics that change results or observable attributes: the SpMV
  ``block_nnz`` doubling, the ``max_segments`` row truncation of both SpMV paths, the SpMM
  ALG1 launch table and its ``max_segments`` ValueError, the SpMM opt buckets and split
  metadata, COO lexicographic sort and row runs, and COO -> CSR conversion (numpy).

How each function is pinned (golden fixtures, scipy, exact sums, brute force, closed forms)
is listed in tests/test_oracle.py.
"""

import ctypes
import math
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build():
    """Compile fsp_oracle.c into oracle/liboracle.so (gcc via oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        lib = ctypes.CDLL(LIB_PATH)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        lib.oracle_spmv_csr_f64.argtypes = [i64, p, p, p, p, p, p]
        lib.oracle_spmv_csr_f64.restype = None
        lib.oracle_spmv_coo_f64.argtypes = [i64, p, p, p, p, i64, p]
        lib.oracle_spmv_coo_f64.restype = None
        lib.oracle_spmm_csr_f64.argtypes = [i64, p, p, p, p, i64, i64, p, i64]
        lib.oracle_spmm_csr_f64.restype = None
        lib.oracle_spmm_coo_f64.argtypes = [i64, p, p, p, p, i64, i64, i64, p, i64]
        lib.oracle_spmm_coo_f64.restype = None
        d = ctypes.c_double
        lib.oracle_sddmm_csr_f64.argtypes = [i64, p, p, p, i64, p, i64, i64, p, d, d, p]
        lib.oracle_sddmm_csr_f64.restype = None
        _lib = lib
    return _lib


def _np(a, dtype):
    """Contiguous numpy copy/view of a numpy array or (CPU/GPU) torch tensor."""
    if hasattr(a, "detach"):
        a = a.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(a), dtype=dtype)


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------------------------------
# fp64 arithmetic
# ----------------------------------------------------------------------------------------


def spmv_csr(indptr, indices, data, x, row_cap=None):
    """fp64 y = A @ x, rows summed in storage order (fsp_oracle.c: oracle_spmv_csr_f64).

    ``row_cap`` (optional, per row) limits how many leading entries of each row are summed,
    which is how the reference's ``max_segments`` truncation shows up in results
    (spmv_csr.py:111-118, 183-189).
    """
    ip = _np(indptr, np.int64)
    ix = _np(indices, np.int64)
    dv = _np(data, np.float64)
    xv = _np(x, np.float64)
    n_rows = ip.size - 1
    y = np.zeros(max(n_rows, 0), dtype=np.float64)
    cap = None if row_cap is None else _np(row_cap, np.int64)
    if n_rows > 0:
        _load().oracle_spmv_csr_f64(
            n_rows, _ptr(ip), _ptr(ix), _ptr(dv), _ptr(xv),
            None if cap is None else _ptr(cap), _ptr(y))
    return y


def spmv_coo(row, col, data, x, n_rows):
    """fp64 y = A @ x for COO entries, duplicates summed (oracle_spmv_coo_f64)."""
    r = _np(row, np.int64)
    c = _np(col, np.int64)
    dv = _np(data, np.float64)
    xv = _np(x, np.float64)
    y = np.zeros(n_rows, dtype=np.float64)
    _load().oracle_spmv_coo_f64(r.size, _ptr(r), _ptr(c), _ptr(dv), _ptr(xv), n_rows, _ptr(y))
    return y


def spmm_csr(indptr, indices, data, B):
    """fp64 C = A @ B for row-major B (oracle_spmm_csr_f64)."""
    ip = _np(indptr, np.int64)
    ix = _np(indices, np.int64)
    dv = _np(data, np.float64)
    Bv = _np(B, np.float64)
    n_rows = ip.size - 1
    N = Bv.shape[1] if Bv.ndim == 2 else 0
    C = np.zeros((max(n_rows, 0), N), dtype=np.float64)
    if n_rows > 0 and N > 0:
        _load().oracle_spmm_csr_f64(n_rows, _ptr(ip), _ptr(ix), _ptr(dv), _ptr(Bv), N, N,
                                    _ptr(C), N)
    return C


def spmm_coo(row, col, data, B, n_rows):
    """fp64 C = A @ B for COO entries (any order, duplicates summed), row-major B
    (oracle_spmm_coo_f64)."""
    r = _np(row, np.int64)
    c = _np(col, np.int64)
    dv = _np(data, np.float64)
    Bv = _np(B, np.float64)
    N = Bv.shape[1] if Bv.ndim == 2 else 0
    C = np.zeros((n_rows, N), dtype=np.float64)
    if n_rows > 0 and N > 0 and r.size > 0:
        _load().oracle_spmm_coo_f64(r.size, _ptr(r), _ptr(c), _ptr(dv), _ptr(Bv), N, N, n_rows,
                                    _ptr(C), N)
    return C


def sddmm_csr(indptr, indices, x, y, data=None, alpha=1.0, beta=0.0):
    """fp64 SDDMM on a CSR pattern: alpha * dot(x[row], y[col]) + beta * data per entry
    (oracle_sddmm_csr_f64)."""
    ip = _np(indptr, np.int64)
    ix = _np(indices, np.int64)
    xv = _np(x, np.float64)
    yv = _np(y, np.float64)
    n_rows = ip.size - 1
    K = xv.shape[1] if xv.ndim == 2 else 0
    out = np.zeros(ix.size, dtype=np.float64)
    dv = None if data is None else _np(data, np.float64)
    if ix.size > 0:
        _load().oracle_sddmm_csr_f64(n_rows, _ptr(ip), _ptr(ix), _ptr(xv), max(K, 1), _ptr(yv),
                                     max(K, 1), K, None if dv is None else _ptr(dv),
                                     float(alpha), float(beta), _ptr(out))
    return out


def time_spmv_csr(indptr, indices, data, x, min_seconds=10.0, max_passes=1000):
    """Time the fp64 oracle SpMV on one core: full passes until ``min_seconds`` elapsed.

    Inputs are converted once, outside the timing.  Returns (passes, seconds).  Used only as
    bench.py's reported CPU baseline.
    """
    import time

    ip = _np(indptr, np.int64)
    ix = _np(indices, np.int64)
    dv = _np(data, np.float64)
    xv = _np(x, np.float64)
    n_rows = ip.size - 1
    y = np.zeros(n_rows, dtype=np.float64)
    fn = _load().oracle_spmv_csr_f64
    args = (n_rows, _ptr(ip), _ptr(ix), _ptr(dv), _ptr(xv), None, _ptr(y))
    passes = 0
    t0 = time.perf_counter()
    while True:
        fn(*args)
        passes += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= min_seconds or passes >= max_passes:
            return passes, elapsed


def time_spmm_csr(indptr, indices, data, B, min_seconds=10.0, max_passes=1000, row_limit=None):
    """Time the fp64 oracle SpMM on one core over the first ``row_limit`` rows (all by
    default).  Returns (passes, seconds, rows, nnz_in_rows)."""
    import time

    ip = _np(indptr, np.int64)
    n_rows = ip.size - 1 if row_limit is None else min(int(row_limit), ip.size - 1)
    ix = _np(indices, np.int64)
    dv = _np(data, np.float64)
    Bv = _np(B, np.float64)
    N = Bv.shape[1]
    C = np.zeros((n_rows, N), dtype=np.float64)
    fn = _load().oracle_spmm_csr_f64
    args = (n_rows, _ptr(ip), _ptr(ix), _ptr(dv), _ptr(Bv), N, N, _ptr(C), N)
    passes = 0
    t0 = time.perf_counter()
    while True:
        fn(*args)
        passes += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= min_seconds or passes >= max_passes:
            return passes, elapsed, n_rows, int(ip[n_rows] - ip[0])


def time_spmv_coo(row, col, data, x, n_rows, min_seconds=10.0, max_passes=1000):
    """Time the fp64 oracle COO SpMV on one core.  Returns (passes, seconds)."""
    import time

    r = _np(row, np.int64)
    c = _np(col, np.int64)
    dv = _np(data, np.float64)
    xv = _np(x, np.float64)
    y = np.zeros(n_rows, dtype=np.float64)
    fn = _load().oracle_spmv_coo_f64
    args = (r.size, _ptr(r), _ptr(c), _ptr(dv), _ptr(xv), n_rows, _ptr(y))
    passes = 0
    t0 = time.perf_counter()
    while True:
        fn(*args)
        passes += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= min_seconds or passes >= max_passes:
            return passes, elapsed


# ----------------------------------------------------------------------------------------
# SpMV planning semantics
# ----------------------------------------------------------------------------------------

# (max_row_nnz, block_size, batch_rows) per bucket - spmv_csr.py:64-75 (fp32), 77-89 (fp64).
SPMV_OPT_BUCKETS_FP32 = ((64, 32, 16), (512, 256, 1), (4096, 512, 1), (None, 1024, 1))
SPMV_OPT_BUCKETS_FP64 = ((64, 32, 4), (256, 64, 1), (2048, 128, 1), (8192, 256, 1),
                         (None, 512, 1))


def spmv_prepare_knobs(max_row_nnz, block_nnz=256, max_segments=None):
    """(block_nnz, max_segments) stored on PreparedCsrSpmv - spmv_csr.py:465-475.

    With max_segments None the tile count covers the longest row, doubling block_nnz (up to
    65536) while more than 2048 tiles would be needed; a caller's max_segments is kept as is.
    """
    if max_segments is not None:
        return block_nnz, max_segments
    b = block_nnz
    seg = max(-(-max_row_nnz // b), 1)
    while seg > 2048 and b < 65536:
        b *= 2
        seg = max(-(-max_row_nnz // b), 1)
    return b, seg


def spmv_opt_buckets(row_lengths, max_row_nnz, fp64, max_segments=None):
    """Row buckets of the opt path - spmv_csr.py:281-327.

    Returns a list of dicts {rows, block_size, max_segs, batch_rows} for non-empty buckets.
    Rows of length 0 fall in the first bucket; each row appears exactly once.
    """
    lengths = _np(row_lengths, np.int64)
    specs = SPMV_OPT_BUCKETS_FP64 if fp64 else SPMV_OPT_BUCKETS_FP32
    out = []
    lower = 0
    for upper, bs, batch in specs:
        if upper is None:
            mask = lengths > lower
            bucket_max = max_row_nnz
        elif lower == 0:
            mask = lengths <= upper
            bucket_max = upper
        else:
            mask = (lengths > lower) & (lengths <= upper)
            bucket_max = upper
        rows = np.nonzero(mask)[0]
        if rows.size:
            segs = max(-(-bucket_max // bs), 1) if max_segments is None else max_segments
            out.append({"rows": rows, "block_size": bs, "max_segs": segs, "batch_rows": batch})
        if upper is not None:
            lower = upper
    return out


def spmv_row_caps(row_lengths, use_opt, fp64, block_nnz, max_segments, user_max_segments):
    """Number of leading entries of each row that the reference sums.

    Base path (spmv_csr.py:111-118): tiles seg = 0..MAX_SEGMENTS-1 of BLOCK_NNZ lanes starting
    at the row start, i.e. min(len, max_segments * block_nnz) with the prepared knobs.
    Opt path (spmv_csr.py:183-189, 243-249): the same with the bucket's block_size and
    max_segs.  Without a caller max_segments both cover every row entirely.
    """
    lengths = _np(row_lengths, np.int64)
    if not use_opt:
        return np.minimum(lengths, max(0, int(max_segments)) * int(block_nnz))
    caps = lengths.copy()
    if user_max_segments is None:
        return caps
    max_row = int(lengths.max()) if lengths.size else 0
    for b in spmv_opt_buckets(lengths, max_row, fp64, user_max_segments):
        caps[b["rows"]] = np.minimum(lengths[b["rows"]], max(0, b["max_segs"]) * b["block_size"])
    return caps


# ----------------------------------------------------------------------------------------
# SpMM planning semantics
# ----------------------------------------------------------------------------------------


def spmm_alg1_config(n_dense_cols, max_row_nnz, block_n=None, block_nnz=None,
                     max_segments=None):
    """ALG1 launch configuration - spmm_csr.py:284-334.

    (warp, factor) from the dense width; block_n = warp*factor, block_nnz = warp unless given;
    ValueError when a caller's max_segments is smaller than ceil(max_row_nnz / block_nnz).
    """
    n = n_dense_cols
    if n > 64:
        warp, factor = 32, 4
    elif n > 32:
        warp, factor = 32, 2
    elif n > 16:
        warp, factor = 32, 1
    elif n > 8:
        warp, factor = 16, 1
    elif n > 4:
        warp, factor = 8, 1
    else:
        warp, factor = 4, 1
    if block_n is None:
        block_n = warp * factor
    if block_nnz is None:
        block_nnz = warp
    if block_n <= 0 or block_nnz <= 0:
        raise ValueError("block_n and block_nnz must be positive when provided")
    if max_segments is not None and max_segments <= 0:
        raise ValueError("max_segments must be positive when provided")
    required = -(-max_row_nnz // block_nnz) if max_row_nnz > 0 else 0
    if max_segments is not None and required > int(max_segments):
        raise ValueError("row nnz requires more CSR segments than max_segments allows")
    return {"block_n": int(block_n), "block_nnz": int(block_nnz),
            "max_segments": None if max_segments is None else int(max_segments),
            "required_segments": int(required), "warp_size": warp, "factor": factor,
            "max_row_nnz": int(max_row_nnz), "auto_max_segments": max_segments is None}


def spmm_opt_block_n(n_dense_cols):
    """spmm_csr.py:405-414: smallest of 8/16/32/64 covering N, else 128."""
    for b in (8, 16, 32, 64):
        if n_dense_cols <= b:
            return b
    return 128


# (max_row_nnz, kind, batch_rows, block_nnz) - spmm_csr.py:395-401.
SPMM_OPT_BUCKETS = ((32, "batched", 8, 32), (128, "batched", 4, 64), (512, "vector", 1, 128),
                    (2048, "vector", 1, 128), (None, "split", 1, 256))


def spmm_opt_buckets(row_lengths):
    """Row buckets of prepare_spmm_csr_opt - spmm_csr.py:444-477 (returns buckets, long rows)."""
    lengths = _np(row_lengths, np.int64)
    out = []
    lower = 0
    long_rows = np.zeros(0, dtype=np.int64)
    for upper, kind, batch, bnnz in SPMM_OPT_BUCKETS:
        if upper is None:
            mask = lengths > lower
        elif lower == 0:
            mask = lengths <= upper
        else:
            mask = (lengths > lower) & (lengths <= upper)
        rows = np.nonzero(mask)[0]
        if rows.size:
            out.append({"kind": kind, "rows": rows, "batch_rows": batch, "block_nnz": bnnz})
            if kind == "split":
                long_rows = rows
        if upper is not None:
            lower = upper
    return out, long_rows


def spmm_opt_split_metadata(indptr, long_rows, part_block_nnz=256):
    """Long-row parts - spmm_csr.py:417-441: (part_rows, part_starts, part_ends, row_part_ptr).

    Each long row [start, end) is cut at start, start+part, ... ; row_part_ptr[j] is the first
    part of the j-th long row.
    """
    ip = _np(indptr, np.int64)
    rows = []
    starts = []
    ends = []
    ptr = [0]
    for r in _np(long_rows, np.int64).tolist():
        cur, end = int(ip[r]), int(ip[r + 1])
        while cur < end:
            rows.append(r)
            starts.append(cur)
            cur = min(cur + part_block_nnz, end)
            ends.append(cur)
        ptr.append(len(rows))
    return (np.array(rows, dtype=np.int64), np.array(starts, dtype=np.int64),
            np.array(ends, dtype=np.int64), np.array(ptr, dtype=np.int64))


# ----------------------------------------------------------------------------------------
# COO semantics
# ----------------------------------------------------------------------------------------


def coo_sort_lex(data, row, col, n_cols):
    """Sort entries by (row, col) - spmv_coo.py:153-164 (key = row * max(1, n_cols) + col).

    The reference uses an unstable argsort; a stable one is used here, which fixes the order
    of duplicate (row, col) entries (only the rounding of their sum can depend on it).
    """
    r = _np(row, np.int64)
    c = _np(col, np.int64)
    d = np.asarray(data)
    if r.size == 0:
        return d.copy(), r, c
    order = np.argsort(r * max(1, int(n_cols)) + c, kind="stable")
    return d[order], r[order], c[order]


def coo_seg_starts(sorted_rows):
    """Run boundaries of constant row in sorted COO - spmv_coo.py:167-179 (None if empty)."""
    r = _np(sorted_rows, np.int64)
    if r.size == 0:
        return None
    breaks = np.nonzero(r[1:] != r[:-1])[0] + 1
    return np.concatenate([[0], breaks, [r.size]]).astype(np.int64)


def coo_to_csr(data, row, col, n_rows, n_cols, assume_sorted=False):
    """COO -> CSR for the COO-to-CSR SpMV route - spmv_csr.py:613-647.

    Sorted (or assumed sorted) input is kept in order; otherwise entries are sorted by
    (row, col).  indptr from per-row counts.  Returns (data, indices, indptr).
    """
    r = _np(row, np.int64)
    c = _np(col, np.int64)
    d = np.asarray(data)
    if r.size == 0:
        return d.copy(), c.astype(np.int64), np.zeros(n_rows + 1, dtype=np.int64)
    key = r * max(1, int(n_cols)) + c
    if not (assume_sorted or bool(np.all(key[1:] >= key[:-1]))):
        order = np.argsort(key, kind="stable")
        r, c, d = r[order], c[order], d[order]
    indptr = np.zeros(n_rows + 1, dtype=np.int64)
    indptr[1:] = np.cumsum(np.bincount(r, minlength=n_rows))
    return d, c, indptr


# ----------------------------------------------------------------------------------------
# Metrics and tolerances
# ----------------------------------------------------------------------------------------

# north_star: relative L2 error against an fp64 accumulation.
REL_L2_BOUND = {"float32": 1e-5, "float64": 1e-12}
# (atol, rtol) of the reference's SpMV opt / COO / SpMM-opt test scripts
# (tests/test_spmv_opt.py:204-207, tests/test_spmv_coo.py:323-326, test_spmm_opt.py:202-224).
REF_SCRIPT_TOL = {"float32": (1e-4, 1e-2), "float64": (1e-12, 1e-10)}
# (atol, rtol) of the library's allclose checks (_common.py:76-85).
REF_LIB_TOL = {"float32": (1e-6, 1e-5), "float64": (1e-10, 1e-8)}


def rel_l2(actual, ref):
    """||actual - ref||_2 / ||ref||_2 in fp64 (0 when both are zero)."""
    a = _np(actual, np.float64).ravel()
    r = _np(ref, np.float64).ravel()
    den = math.sqrt(float(np.dot(r, r)))
    num = math.sqrt(float(np.dot(a - r, a - r)))
    if den == 0.0:
        return 0.0 if num == 0.0 else math.inf
    return num / den


def allclose_ratio(actual, ref, atol, rtol):
    """max |a - r| / (atol + rtol |r|) - tests/test_spmv.py:106-111; <= 1 passes."""
    a = _np(actual, np.float64).ravel()
    r = _np(ref, np.float64).ravel()
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - r) / (atol + rtol * np.abs(r))))
