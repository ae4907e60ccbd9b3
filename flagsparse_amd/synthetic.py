"""Seeded synthetic matrices for the five benchmark configurations.

Every random number comes from a SplitMix64 counter stream (Steele, Lea and Flood,
"Fast splittable pseudorandom number generators", OOPSLA 2014) evaluated with torch int64
arithmetic, so the same arrays come out on the CPU and on the GPU and do not depend on the
numpy or torch RNG versions.  Uniform-derived arrays are bit-identical across devices;
normal variates use Box-Muller through torch.log / torch.cos, whose last bit may differ
between the CPU and GPU libraries (their SHA-256 is therefore recorded per device).

The reference builds its test matrices with unseeded torch RNG
(sparse_operations/_common.py:149-181); ``build_random_csr`` below keeps that generator's
shape (sorted random rows -> bincount -> cumsum, unsorted and possibly repeated columns) with
a seed.
"""

import hashlib
import math

import numpy as np
import torch

_GOLDEN = 0x9E3779B97F4A7C15
_M1 = 0xBF58476D1CE4E5B9
_M2 = 0x94D049BB133111EB
_U64 = (1 << 64) - 1


def _s64(v):
    """Python int (mod 2^64) -> the int64 with the same bits."""
    v &= _U64
    return v - (1 << 64) if v >= (1 << 63) else v


def _mix_int(z):
    z &= _U64
    z = ((z ^ (z >> 30)) * _M1) & _U64
    z = ((z ^ (z >> 27)) * _M2) & _U64
    return z ^ (z >> 31)


def _srl(z, k):
    """Logical right shift of an int64 tensor."""
    return (z >> k) & ((1 << (64 - k)) - 1)


def _mix(z):
    z = (z ^ _srl(z, 30)) * _s64(_M1)
    z = (z ^ _srl(z, 27)) * _s64(_M2)
    return z ^ _srl(z, 31)


def stream_u64(seed, stream, counters):
    """SplitMix64 outputs for counters of stream ``stream`` (int64 tensor, any device)."""
    key = _mix_int(_mix_int(seed * _GOLDEN + 1) ^ (stream * _M2))
    z = (counters + 1) * _s64(_GOLDEN) + _s64(key)
    return _mix(z)


def _counters(n, device, offset=0):
    return torch.arange(offset, offset + n, dtype=torch.int64, device=device)


def uniform01(seed, stream, n, device, offset=0):
    """float64 uniforms in [0, 1) with 53 random bits."""
    z = stream_u64(seed, stream, _counters(n, device, offset))
    return _srl(z, 11).to(torch.float64) * (2.0 ** -53)


def randint(seed, stream, n, high, device, offset=0):
    """int64 in [0, high) (high <= 2^62; modulo bias below 2^-30 for the sizes used)."""
    z = stream_u64(seed, stream, _counters(n, device, offset))
    return _srl(z, 1) % int(high)


def uniform_values(seed, stream, n, dtype, device, lo=-1.0, hi=1.0):
    u = uniform01(seed, stream, n, device)
    return (lo + (hi - lo) * u).to(dtype)


def normal_values(seed, stream, n, dtype, device):
    """Box-Muller normals (one per pair of uniforms)."""
    u1 = uniform01(seed, stream, n, device)
    u2 = uniform01(seed, stream + 1, n, device)
    r = torch.sqrt(-2.0 * torch.log1p(-u1))
    return (r * torch.cos((2.0 * math.pi) * u2)).to(dtype)


def sha256(t):
    """SHA-256 of a tensor's bytes (as stored)."""
    a = t.detach().contiguous().cpu()
    if a.dtype == torch.bfloat16:
        a = a.view(torch.int16)
    return hashlib.sha256(a.numpy().tobytes()).hexdigest()


def _rows_of(lengths):
    n = lengths.numel()
    return torch.repeat_interleave(torch.arange(n, dtype=torch.int64, device=lengths.device),
                                   lengths)


def _distinct_sorted_columns(lengths, n_cols, seed, stream, window_lo=None, width=None,
                             fixed_keys=None):
    """Per-row distinct uniform columns, sorted.  Returns the sorted int64 keys row*n_cols+col.

    Columns are drawn from [window_lo[r], window_lo[r] + width) when a window is given, else
    from [0, n_cols).  Repeats (and collisions with ``fixed_keys``, which are kept) are
    redrawn from fresh counters until every row holds lengths[r] distinct new columns.
    """
    device = lengths.device
    want = lengths.clone()
    drawn = 0
    span = n_cols if width is None else width

    def draw(rows):
        nonlocal drawn
        c = randint(seed, stream, rows.numel(), span, device, offset=drawn)
        drawn += rows.numel()
        if window_lo is not None:
            c = c + window_lo[rows]
        return rows * n_cols + c

    new_keys = draw(_rows_of(want))
    fixed = fixed_keys if fixed_keys is not None else torch.empty(0, dtype=torch.int64,
                                                                 device=device)
    while True:
        # tag: fixed keys (0) sort before new keys (1) with the same (row, col)
        comp = torch.cat([fixed * 2, new_keys * 2 + 1])
        comp, _ = torch.sort(comp)
        keys = comp >> 1
        tag = comp & 1
        dup = torch.zeros_like(tag, dtype=torch.bool)
        if keys.numel() > 1:
            dup[1:] = keys[1:] == keys[:-1]
        keep_new = (tag == 1) & ~dup
        new_keys = keys[keep_new]
        have = _sorted_counts(new_keys // n_cols, lengths.numel())
        deficit = want - have
        if int(deficit.sum().item()) == 0:
            break
        new_keys = torch.cat([new_keys, draw(_rows_of(deficit))])
    if fixed_keys is None:
        return new_keys
    allk, _ = torch.sort(torch.cat([fixed, new_keys]))
    return allk


def _sorted_counts(sorted_rows, n_rows):
    """bincount of non-decreasing row numbers: the boundaries of equal values (a histogram by
    atomics serialises on the long rows of a power law, 37 ms for cfg3 on MI355X)."""
    bounds = torch.searchsorted(sorted_rows,
                                torch.arange(n_rows + 1, device=sorted_rows.device,
                                             dtype=sorted_rows.dtype))
    return bounds[1:] - bounds[:-1]


def _csr_from_keys(keys, n_rows, n_cols):
    """CSR row pointers and columns of sorted keys row * n_cols + col."""
    rows = keys // n_cols
    cols = keys % n_cols
    indptr = torch.zeros(n_rows + 1, dtype=torch.int64, device=keys.device)
    indptr[1:] = torch.cumsum(_sorted_counts(rows, n_rows), 0)
    return indptr, cols


# ------------------------------------------------------------------------------------------
# The five configurations (BASELINE.json "configs", in order)
# ------------------------------------------------------------------------------------------


def csr_uniform_rows(n_rows=4096, n_cols=4096, per_row=16, dtype=torch.float32,
                     index_dtype=torch.int32, seed=0, device="cpu"):
    """cfg1: exactly ``per_row`` distinct uniform columns per row (sorted), values and x
    U(-1, 1).  Returns (data, indices, indptr, x, shape)."""
    lengths = torch.full((n_rows,), per_row, dtype=torch.int64, device=device)
    keys = _distinct_sorted_columns(lengths, n_cols, seed, 1)
    indptr, cols = _csr_from_keys(keys, n_rows, n_cols)
    data = uniform_values(seed, 10, cols.numel(), dtype, device)
    x = uniform_values(seed, 20, n_cols, dtype, device)
    return data, cols.to(index_dtype), indptr.to(index_dtype), x, (n_rows, n_cols)


def csr_poisson2d(grid=2048, dtype=torch.float64, index_dtype=torch.int32, seed=0,
                  device="cpu"):
    """cfg2: 5-point Poisson stencil on a grid x grid mesh, natural ordering i = r*grid + c,
    diagonal 4, neighbours -1, columns sorted; x ~ U(-1, 1)."""
    n = grid * grid
    i = torch.arange(n, dtype=torch.int64, device=device)
    r = i // grid
    c = i % grid
    offs = (-grid, -1, 0, 1, grid)
    valid = torch.stack([r > 0, c > 0, torch.ones_like(r, dtype=torch.bool), c < grid - 1,
                         r < grid - 1], dim=1)
    colm = i[:, None] + torch.tensor(offs, dtype=torch.int64, device=device)[None, :]
    valm = torch.tensor([-1.0, -1.0, 4.0, -1.0, -1.0], dtype=torch.float64,
                        device=device)[None, :].expand(n, 5)
    cols = colm[valid]
    vals = valm[valid].to(dtype)
    lengths = valid.sum(dim=1)
    indptr = torch.zeros(n + 1, dtype=torch.int64, device=device)
    indptr[1:] = torch.cumsum(lengths, 0)
    x = uniform_values(seed, 20, n, dtype, device)
    return vals, cols.to(index_dtype), indptr.to(index_dtype), x, (n, n)


def zipf_row_lengths(n_rows, alpha=1.8, mean=12, cap=200000, seed=0, device="cpu",
                     table_size=1 << 21):
    """Power-law row lengths: L = min(ceil(c * Z), cap), Z ~ Zipf(alpha) by inverse CDF,
    with c the largest scale whose total stays <= mean * n_rows; the shortfall (a few
    entries) is then added one per row, in row order, to rows below the cap, so
    sum(L) == mean * n_rows exactly."""
    k = np.arange(1, table_size + 1, dtype=np.float64)
    w = k ** (-alpha)
    tail = (table_size + 0.5) ** (1.0 - alpha) / (alpha - 1.0)
    cdf = np.cumsum(w) / (w.sum() + tail)
    cdf_t = torch.from_numpy(cdf).to(device)
    u = uniform01(seed, 30, n_rows, device)
    z = torch.searchsorted(cdf_t, u, right=True).to(torch.float64) + 1.0  # > table -> table+1
    target = int(mean) * n_rows

    def total(c):
        return int(torch.clamp(torch.ceil(c * z), max=cap).sum().item())

    lo, hi = 0.0, 1.0
    while total(hi) <= target:
        hi *= 2.0
    for _ in range(80):
        mid = 0.5 * (lo + hi)
        if total(mid) <= target:
            lo = mid
        else:
            hi = mid
    lengths = torch.clamp(torch.ceil(lo * z), max=cap).to(torch.int64)
    short = target - int(lengths.sum().item())
    if short > 0:
        below = torch.nonzero(lengths < cap).flatten()[:short]
        lengths[below] += 1
    return lengths, lo


def csr_powerlaw(n=8 * 1024 * 1024, alpha=1.8, mean=12, cap=200000, dtype=torch.float32,
                 index_dtype=torch.int64, seed=0, device="cpu"):
    """cfg3: power-law row lengths (zipf_row_lengths), distinct uniform columns per row
    (sorted), values and x ~ N(0, 1).  Returns (data, indices, indptr, x, shape)."""
    lengths, _ = zipf_row_lengths(n, alpha, mean, cap, seed, device)
    keys = _distinct_sorted_columns(lengths, n, seed, 2)
    indptr, cols = _csr_from_keys(keys, n, n)
    del keys
    data = normal_values(seed, 40, cols.numel(), dtype, device)
    x = normal_values(seed, 50, n, dtype, device)
    return data, cols.to(index_dtype), indptr.to(index_dtype), x, (n, n)


def coo_uniform(n=2 * 1024 * 1024, draws=40 * 1024 * 1024, dtype=torch.float32,
                index_dtype=torch.int32, seed=0, device="cpu"):
    """cfg4: ``draws`` uniform (row, col) pairs, duplicates removed, sorted by (row, col);
    values and x ~ U(-1, 1).  Returns (data, row, col, x, shape)."""
    rr = randint(seed, 3, draws, n, device)
    cc = randint(seed, 4, draws, n, device)
    keys = torch.unique(rr * n + cc, sorted=True)
    del rr, cc
    row = keys // n
    col = keys % n
    data = uniform_values(seed, 10, keys.numel(), dtype, device)
    x = uniform_values(seed, 20, n, dtype, device)
    return data, row.to(index_dtype), col.to(index_dtype), x, (n, n)


def csr_banded_random(n=1024 * 1024, band_nnz=16, band_width=512, rand_nnz=16,
                      dtype=torch.float32, index_dtype=torch.int32, seed=0, device="cpu"):
    """cfg5 matrix: per row ``band_nnz`` distinct columns in the window
    [clamp(i - width/2, 0, n - width), + width) plus ``rand_nnz`` distinct uniform columns
    not already present, sorted; values ~ U(-1, 1).  Returns (data, indices, indptr, shape)."""
    i = torch.arange(n, dtype=torch.int64, device=device)
    lo = torch.clamp(i - band_width // 2, min=0, max=max(n - band_width, 0))
    width = min(band_width, n)
    band = _distinct_sorted_columns(torch.full((n,), band_nnz, dtype=torch.int64, device=device),
                                    n, seed, 5, window_lo=lo, width=width)
    keys = _distinct_sorted_columns(torch.full((n,), rand_nnz, dtype=torch.int64, device=device),
                                    n, seed, 6, fixed_keys=band)
    indptr, cols = _csr_from_keys(keys, n, n)
    data = uniform_values(seed, 10, cols.numel(), dtype, device)
    return data, cols.to(index_dtype), indptr.to(index_dtype), (n, n)


def dense_uniform(rows, cols, dtype=torch.float32, seed=0, stream=60, device="cpu"):
    """Row-major [rows, cols] matrix ~ U(-1, 1) (cfg5's B)."""
    return uniform_values(seed, stream, rows * cols, dtype, device).reshape(rows, cols)


def build_random_csr(n_rows, n_cols, nnz, value_dtype, index_dtype, device, seed=0):
    """Seeded counterpart of the reference's _build_random_csr (_common.py:166-181): nnz row
    draws sorted -> bincount -> cumsum; columns uniform, unsorted, possibly repeated;
    values ~ N(0, 1)."""
    if nnz <= 0 or n_rows <= 0 or n_cols <= 0:
        indptr = torch.zeros(n_rows + 1, dtype=torch.int64, device=device)
        return (torch.empty(0, dtype=value_dtype, device=device),
                torch.empty(0, dtype=index_dtype, device=device), indptr)
    rows, _ = torch.sort(randint(seed, 70, nnz, n_rows, device))
    indptr = torch.zeros(n_rows + 1, dtype=torch.int64, device=device)
    indptr[1:] = torch.cumsum(torch.bincount(rows, minlength=n_rows), 0)
    indices = randint(seed, 71, nnz, n_cols, device).to(index_dtype)
    data = normal_values(seed, 72, nnz, value_dtype, device)
    return data, indices, indptr


def build_random_coo(n_rows, n_cols, nnz, value_dtype, index_dtype, device, seed=0):
    """Random COO for the COO SpMM benchmark case: nnz independent uniform (row, col) draws in
    draw order (unsorted, duplicates possible), values ~ N(0, 1).  The reference's benchmark
    calls a ``_build_random_coo`` helper (spmm_coo.py:866) that its sources do not define;
    this is the natural COO counterpart of its _build_random_csr (_common.py:166-181)."""
    if nnz <= 0 or n_rows <= 0 or n_cols <= 0:
        empty = torch.empty(0, dtype=index_dtype, device=device)
        return torch.empty(0, dtype=value_dtype, device=device), empty, empty.clone()
    row = randint(seed, 73, nnz, n_rows, device).to(index_dtype)
    col = randint(seed, 74, nnz, n_cols, device).to(index_dtype)
    data = normal_values(seed, 75, nnz, value_dtype, device)
    return data, row, col


def build_random_dense(size, value_dtype, device, seed=0, stream=80):
    """Seeded counterpart of _build_random_dense (_common.py:149-157): N(0, 1) values."""
    shape = (size,) if isinstance(size, int) else tuple(size)
    numel = int(np.prod(shape)) if len(shape) else 1
    return normal_values(seed, stream, numel, value_dtype, device).reshape(shape)
