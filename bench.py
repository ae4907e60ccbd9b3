"""Benchmark of the flagsparse_amd hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg3] [--no-targets]

Prints ONE JSON line.  A step is one call of the public API over the workload's matrix with
the inputs already resident in HBM and the prepare step outside the timed region, as the
reference's harness does (sparse_operations/benchmarks.py:249-262).  The default workload is
cfg3 (CSR SpMV, float32, the 8M-row power-law matrix, the
reference's default use_opt=False path), the configuration north_star's SpMV target is quoted
on; --workload selects the others, and the two probe workloads.

value        algorithmic bytes per step / time per step (HIP events around the K steps); the
             untimed warm-up before them runs W steps at a time until at least 50 ms have
             passed (``warmup_steps_run`` reports how many)
roofline     the same bytes / the path's kernel time (all the kernels of one launch), timed
             with HIP events around K back-to-back launches on the stream the kernels run on
             (the median of 5 such trials; all five in ``kernel_ms_trials``), against the
             8 TB/s HBM3E peak.  From the committed rocprofv3 summaries
             (profiles/<tag>_traffic.txt): ``traffic`` = FETCH_SIZE + WRITE_SIZE per launch,
             ``l2_hit_rate`` and ``occupancy_percent`` per kernel; ``traffic_gbs`` and
             ``frac_traffic``: that traffic over the kernel time measured now (the rate at
             which the kernel moves the bytes it does move).  ``bytes_gather_inclusive``
             counts x (SpMV) or B (SpMM) once per entry instead of once, and
             ``frac_gather_inclusive`` is that count over the same time against the peak.
             ``gather_bound`` (cfg5; cfg3 with the XCS layouts): the probe kernels timed in
             the same run on the workload's own gather count and pattern - the rate the
             gathers alone reach;
             ``kernel_ms_over_bound`` divides the whole path's kernel time by it, and for cfg3
             ``part_ms_over_bound`` the XCS part's (its kernel and combine, ``parts_ms``).
             ``stream_bound`` (cfg3): a plain read of the bytes the panel kernel reads
             (fsp_probe_stream), and the panel kernel's time alone over it (with the
             staged-x layout the panel kernel also writes the staged x values)
cpu_baseline the reference's own CPU path (its tests' torch comparison): torch.sparse.mm on
             CPU sparse tensors of the same matrix, on all of torch's host threads (``cores``,
             OMP_NUM_THREADS: the box's CPU share), ~10 s of full products, with the same byte
             and flop counts ("kind": "reference"); reported only, never a target.  For the
             workloads without one (SDDMM, COO SpMM) the C oracle
cpu_port     the C oracle (fp64 restatement, one core) on the same arrays, ~5 s of passes (a
             bounded row sample for SpMM)
cpu_reference_path
             scipy.sparse (one core) on the same matrix, ~5 s
config       also ``lib_load_ms`` (loading the HIP library, once per process), ``prepare_ms``
             (the prepare call and the first layout build, synchronised; ``prepare_call_ms``
             and ``layout_build_ms`` separately), ``plan.layout_bytes`` (device memory the
             prepared layout holds beyond the caller's arrays), ``first_call_ms`` (the first
             step after prepare, cold) and ``inputs_sha256`` (SHA-256 of every generated input
             array, so that runs on different machines provably use the same data)
targets      north_star's two targets measured in the same run, each with the same roofline
             block: CSR SpMV fp32 on the 8M power-law matrix (>= 70% of HBM peak; the headline
             itself when the workload is cfg3) and CSR SpMM fp32 N=64 (>= 60%), the latter with
             its own bounded CPU baseline; omitted with --no-targets

Probe workloads (measurement only; the access patterns the kernels are bound by, alone):
  probe-gather  random 4-byte gathers (fsp_probe_gather) from an fp32 x of --probe-bytes
                (default 33.5 MB, cfg3's x), 16 per thread in flight; --probe-xcd restricts
                the gathers of XCD k to the k-th eighth of x (the XCS layout's placement);
                --probe-group G --probe-range W [--probe-sorted]: each group of G gathers
                (an XCS item's worth) draws from one range of W bytes of its eighth, sorted
                and laid out lane-major on request (neighbouring lanes, neighbouring lines)
  probe-rows    random 256-byte row gathers (fsp_probe_rows) from an fp32 B[rows, 64] of
                --probe-bytes (default 268 MB, cfg5 N=64's B): 16.8M gathers, cfg5's random half
  --cfg5-part band|random   cfg5 with only its banded or only its random half (16 entries per
                row), to price each half of the matrix separately

Algorithmic bytes count each array once at the width the kernel reads:
  SpMV  nnz*(v + i) + (n_rows + 1)*p + n_cols*v + n_rows*v
  SpMM  nnz*(v + i) + (n_rows + 1)*p + n_cols*N*v + n_rows*N*v
"""

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "CSR SpMV/SpMM effective HBM GB/s + GFLOP/s, % of MI355X HBM roofline"
HBM_PEAK_GBS = 8000.0

WORKLOADS = {
    "cfg1": "CSR SpMV fp32 4096x4096, 16 distinct uniform columns per row, int32, U(-1,1), seed 0",
    "cfg2": "CSR SpMV fp64 2D 5-point Poisson 2048x2048 (4,194,304 rows, 20,963,328 nnz), "
            "int32, x~U(-1,1)",
    "cfg3": "CSR SpMV fp32 8M x 8M power-law rows (Zipf 1.8, mean 12, max 200k), uniform "
            "columns, int64 indices narrowed to int32 in prepare, N(0,1)",
    "cfg4": "COO SpMV fp32 2M x 2M, 40M uniform draws deduplicated, row-sorted, int32, U(-1,1)",
    "cfg5": "CSR SpMM A 1M x 1M, 32 nnz/row (16 in a 512-wide band + 16 uniform), B row-major "
            "1M x N, int32, U(-1,1)",
    "coo5": "COO SpMM: cfg5's matrix as row-sorted COO (int32 row/col), B row-major 1M x N, "
            "through flagsparse_spmm_coo (per-call row-order check, bincount row pointer and "
            "plan inside the step, as the reference's per-call coalesce/sort)",
    "sddmm": "CSR SDDMM on cfg5's pattern (1M x 1M, 32 nnz/row), x [1M, K] and y [1M, K] "
             "row-major ~U(-1,1), alpha 1, beta 0, fp32 accumulation (the reference's baseline)",
    "copy": "plain device copy of 1 GiB (PMC calibration kernel)",
    "probe-gather": "random 4-byte gathers from an fp32 x (fsp_probe_gather), 16 per thread",
    "probe-rows": "random 256-byte row gathers from an fp32 B[rows, 64] (fsp_probe_rows)",
}


def _parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="cfg3", choices=sorted(WORKLOADS))
    ap.add_argument("--dtype", default=None, choices=("f32", "f64"),
                    help="value type for cfg5 / coo5 / sddmm (default f32)")
    ap.add_argument("--n", type=int, default=64,
                    help="dense columns N for cfg5 / coo5, K for sddmm")
    ap.add_argument("--cfg5-part", default="all", choices=("all", "band", "random"),
                    help="cfg5: the whole matrix, or only its banded or only its random half "
                         "(16 entries per row each) - the cost of each half")
    ap.add_argument("--opt", action="store_true",
                    help="SpMV: use_opt=True (native accumulation) instead of the default path")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU baseline: seconds of torch CPU products (the C oracle and "
                         "scipy half as long each)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-targets", action="store_true",
                    help="skip the north_star target measurements")
    ap.add_argument("--probe-bytes", type=int, default=None,
                    help="probe workloads: bytes of x (probe-gather) or B (probe-rows)")
    ap.add_argument("--probe-n", type=int, default=None,
                    help="probe workloads: number of gathers")
    ap.add_argument("--probe-xcd", action="store_true",
                    help="probe-gather: XCD k gathers only from the k-th eighth of x")
    ap.add_argument("--probe-group", type=int, default=0,
                    help="probe-gather with --probe-xcd: gathers per group (a multiple of 1024 "
                         "dividing 4096, one workgroup's share or half of it); each group draws "
                         "from one --probe-range of its XCD's eighth")
    ap.add_argument("--probe-range", type=int, default=0,
                    help="probe-gather with --probe-group: bytes of x one group draws from")
    ap.add_argument("--probe-sorted", action="store_true",
                    help="probe-gather with --probe-group: each group sorted and laid out "
                         "lane-major (the 64 lanes of a gather instruction take neighbouring "
                         "sorted indices)")
    return ap.parse_args()


def _profile(tag):
    """What the committed profiles/<tag>_traffic.txt records: ``traffic_bytes_per_launch`` and
    the per-kernel ``l2_hit_rate[...]`` / ``occupancy_percent[...]`` lines ({} if absent)."""
    path = os.path.join(ROOT, "profiles", f"{tag}_traffic.txt")
    if not os.path.exists(path):
        return {}
    with open(path) as fh:
        text = fh.read()
    out = {}
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", text, re.M)
    if m:
        out["traffic"] = float(m.group(1))
    for key in ("l2_hit_rate", "occupancy_percent"):
        vals = {k: float(v) for k, v in re.findall(rf"^{key}\[([^\]]+)\]:\s*([0-9.]+)", text, re.M)}
        if vals:
            out[key] = vals
    return out


def _event_loop(fn, count, torch):
    """Average milliseconds of ``fn`` over ``count`` back-to-back calls, measured with HIP
    events on torch's current stream (the stream every flagsparse_amd launch uses)."""
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(count):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / count


def _timed_prepare(fn, torch):
    """(result, milliseconds) of a prepare call, synchronised on both sides."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = fn()
    torch.cuda.synchronize()
    return out, round((time.perf_counter() - t0) * 1000.0, 3)


def _digests(arrays, synthetic):
    """{name: SHA-256 of the array's bytes} for the generated inputs."""
    return {name: synthetic.sha256(t) for name, t in arrays.items()}


def _host_info(torch):
    model = None
    try:
        with open("/proc/cpuinfo") as fh:
            m = re.search(r"^model name\s*:\s*(.+)$", fh.read(), re.M)
            model = m.group(1).strip() if m else None
    except OSError:
        pass
    return {"os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "cpu_model": model}


def _tag(kernel):
    """File-name form of a kernel label ("a+b" for a path of two main kernels)."""
    return kernel.replace("+", "_")


def _time_passes(fn, seconds, max_passes=10000):
    fn()  # warm-up (first-touch, library set-up)
    passes, t0 = 0, time.perf_counter()
    while True:
        fn()
        passes += 1
        secs = time.perf_counter() - t0
        if secs >= seconds or passes >= max_passes:
            return passes, secs


def _cpu_torch(fmt, mats, rhs, shape, seconds, nbytes, flops, torch):
    """The reference's CPU path (its tests' torch comparison, tests/test_spmv.py:143-174):
    torch.sparse.mm on CPU sparse tensors built from the host copy of the same matrix and
    right-hand side, on all of torch's host threads (torch.get_num_threads(), which follows
    OMP_NUM_THREADS: the box's CPU share).  fmt "csr": mats = (indptr, indices, data); "coo":
    (row, col, data)."""
    import warnings

    warnings.filterwarnings("ignore", message="Sparse CSR tensor support is in beta")
    a, b, data = (t.detach().cpu() for t in mats)
    r = rhs.detach().cpu()
    try:
        if fmt == "csr":
            At = torch.sparse_csr_tensor(a.to(torch.int64), b.to(torch.int64), data, size=shape)
        else:
            At = torch.sparse_coo_tensor(torch.stack([a, b]).to(torch.int64), data,
                                         size=shape).coalesce()
        rt = r if r.dim() == 2 else r.unsqueeze(1)
        passes, secs = _time_passes(lambda: torch.sparse.mm(At, rt), seconds)
    except Exception as exc:  # report, never fail the benchmark
        return {"error": f"{type(exc).__name__}: {exc}", "kind": "reference"}
    return {"value": round(nbytes * passes / secs / 1e9, 3), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "reference",
            "path": f"torch.sparse.mm, {fmt.upper()} on the CPU",
            "sample": f"{passes} full products (torch.sparse.mm, {fmt.upper()} on the CPU, "
                      f"{data.dtype}, {torch.get_num_threads()} threads) over the whole "
                      f"matrix in {secs:.1f} s",
            "gflops": round(flops * passes / secs / 1e9, 3)}


def _cpu_scipy(fmt, mats, rhs, shape, seconds, nbytes, flops):
    """scipy.sparse (single-threaded) on the host copy of the same matrix and right-hand side:
    the other CPU library the reference's scripts compare against."""
    import numpy as np
    import scipy.sparse as sp

    a, b, data = (t.detach().cpu() for t in mats)
    r = rhs.detach().cpu()
    try:
        if fmt == "csr":
            A = sp.csr_matrix((data.numpy(), b.numpy(), a.numpy()), shape=shape)
        else:
            A = sp.coo_matrix((data.numpy(), (a.numpy(), b.numpy())), shape=shape).tocsr()
        rn = np.ascontiguousarray(r.numpy())
        passes, secs = _time_passes(lambda: A @ rn, seconds)
    except Exception as exc:  # report, never fail the benchmark
        return {"error": f"{type(exc).__name__}: {exc}"}
    return {"value": round(nbytes * passes / secs / 1e9, 3), "unit": "GB/s",
            "gflops": round(flops * passes / secs / 1e9, 3), "cores": 1,
            "sample": f"{passes} full products (scipy.sparse csr_matrix @ dense, "
                      f"{data.dtype}) in {secs:.1f} s"
                      + ("; COO converted to CSR first" if fmt == "coo" else "")}


def _cpu_lib(fmt, mats, rhs, shape, nbytes, flops, torch):
    """(torch timer, scipy timer) for a workload: each takes the seconds to spend."""
    return (lambda s: _cpu_torch(fmt, mats, rhs, shape, s, nbytes, flops, torch),
            lambda s: _cpu_scipy(fmt, mats, rhs, shape, s, nbytes, flops))


def _spmv_csr_workload(name, dev, opt, torch, fs, synthetic):
    if name == "cfg1":
        data, idx, ptr, x, shape = synthetic.csr_uniform_rows(device=dev)
    elif name == "cfg2":
        data, idx, ptr, x, shape = synthetic.csr_poisson2d(2048, device=dev)
    else:
        data, idx, ptr, x, shape = synthetic.csr_powerlaw(device=dev)
    from flagsparse_amd import spmv_csr as mod

    prepared, prep_call_ms = _timed_prepare(lambda: fs.prepare_spmv_csr(data, idx, ptr, shape),
                                            torch)
    use_opt = bool(opt and prepared.supports_opt)
    # the layout and launch arguments are built on first use; count them as prepare work
    _, layout_ms = _timed_prepare(lambda: prepared._kernel(use_opt), torch)
    y = torch.empty(shape[0], dtype=data.dtype, device=dev)
    kc = prepared._kernel(use_opt)
    v = data.element_size()
    p_k = prepared.kernel_indptr.element_size()
    nnz = int(data.numel())
    nbytes = nnz * (v + 4) + (shape[0] + 1) * p_k + shape[1] * v + shape[0] * v
    from flagsparse_amd._spmv_layouts import tensor_bytes

    caller = (data, idx, ptr)
    narrowed = [t for t in (prepared.kernel_indices, prepared.kernel_indptr)
                if all(t.untyped_storage().data_ptr() != c.untyped_storage().data_ptr()
                       for c in caller)]
    plan = dict(kc.describe(), layout_bytes=int(kc.held_bytes(caller)),
                narrowed_index_bytes=int(tensor_bytes(*narrowed)))
    # the first prepare of a process also pays one-time set-up (the first use of each torch
    # operation it runs); a second prepare of the same matrix shows the steady cost
    _, prep_again_ms = _timed_prepare(
        lambda: fs.prepare_spmv_csr(data, idx, ptr, shape)._kernel(use_opt), torch)
    torch.cuda.empty_cache()
    info = {"n_rows": shape[0], "n_cols": shape[1], "nnz": nnz,
            "index_supplied": str(idx.dtype).replace("torch.", ""), "index_kernel": "int32",
            "rowptr_kernel": f"int{8 * p_k}",
            "path": "use_opt=True" if use_opt else "default (use_opt=False)",
            "bytes_as_supplied": nnz * (v + idx.element_size()) +
            (shape[0] + 1) * ptr.element_size() + shape[1] * v + shape[0] * v,
            "plan": plan, "prepare_ms": round(prep_call_ms + layout_ms, 3),
            "prepare_call_ms": prep_call_ms, "layout_build_ms": layout_ms,
            "prepare_ms_repeat": prep_again_ms,
            "inputs": {"data": data, "indices": idx, "indptr": ptr, "x": x}}
    acc_f64 = (not use_opt) or data.dtype == torch.float64
    parts = None
    stream_bound = None
    if kc.kind == "xstage":  # the two launches, each timed alone
        # the first launch reads the long rows' entries (a value and 16 bits each), x once (the
        # panels), the chunk table and the staged entries' 16-bit columns, and writes the
        # staged x values and the long rows' partial sums; the probe streams its reads alone
        lg = kc.long
        read = shape[1] * v + kc.n_staged * 2
        if lg is not None:
            read += lg.n_entries * (v + 2) + int(lg.chunk_info.numel()) * 4
        parts = {"panel_kernel": lambda: kc.launch(x, y, acc_f64, passes=1),
                 "combine": lambda: kc.launch(x, y, acc_f64, passes=2)}
        stream_bound = lambda: _stream_bound(read, dev, torch,  # noqa: E731
                                             f"a plain read of {read} bytes (what the panel "
                                             f"kernel reads: entries, staged columns, x and "
                                             f"chunk table; not its {kc.n_staged * v} bytes of "
                                             f"staged x written)")
    if kc.kind == "xcs-hybrid":  # the two parts of the launch, each timed alone
        from flagsparse_amd import _abi

        parts = {"xcs_part": lambda: kc.short.launch(x, y, acc_f64),
                 "panel_part": lambda: kc.long.launch(x, y, acc_f64),
                 "panel_kernel": lambda: kc.long.launch(x, y, acc_f64, passes=1,
                                                        stream=_abi.raw_stream(dev))}
        # what the panel kernel reads: its entries (a value and 16 bits each), x once (the
        # panels) and the chunk table - streamed alone by the probe
        lg = kc.long
        read = lg.n_entries * (v + 2) + shape[1] * v + int(lg.chunk_info.numel()) * 4
        stream_bound = lambda: _stream_bound(read, dev, torch,  # noqa: E731
                                             f"a plain read of {read} bytes (the panel "
                                             f"kernel's entries, x and chunk table)")

    def cpu(seconds):
        from oracle import oracle

        passes, secs = oracle.time_spmv_csr(ptr, idx, data, x, min_seconds=seconds)
        return {"value": round(nbytes * passes / secs / 1e9, 3), "unit": "GB/s", "cores": 1,
                "kind": "port",
                "sample": f"{passes} full passes of the fp64 C oracle (oracle/fsp_oracle.c) over "
                          f"the same matrix in {secs:.1f} s",
                "gflops": round(2 * nnz * passes / secs / 1e9, 3)}

    gather_bound = None
    if name == "cfg3" and kc.kind == "xcs-hybrid":
        # the XCS part's gathers: its entries, from per-XCD panels of x (P panels, P / 8 per
        # XCD in turn: an x of 8 / P of the whole, each XCD gathering from its eighth)
        n_g = kc.short.nnz // 4 * 4
        x_len = max(8, shape[1] * 8 // kc.short.n_panels)
        gather_bound = lambda: _gather_bound(x_len, n_g, True, dev, torch,  # noqa: E731
                                             f"{n_g} random 4-byte gathers (the XCS part's "
                                             f"entries), XCD k from the k-th eighth of an x of "
                                             f"{x_len * 4} bytes (one of the XCS panels per XCD)")
    return {
        "step": lambda: fs.flagsparse_spmv_csr(x=x, prepared=prepared, use_opt=use_opt, out=y),
        "launch": lambda: mod._run_spmv_csr(prepared, x, use_opt, y),
        "parts": parts, "gather_bound": gather_bound, "bound_part": "xcs_part",
        "stream_bound": stream_bound, "stream_part": "panel_kernel",
        "bytes_gather_inclusive": nnz * (v + 4 + v) + (shape[0] + 1) * p_k + shape[0] * v,
        "nbytes": nbytes, "flops": 2 * nnz, "info": info, "cpu": cpu,
        "cpu_lib": _cpu_lib("csr", (ptr, idx, data), x, shape, nbytes, 2 * nnz, torch),
        "dtype": "f64" if data.dtype == torch.float64 else "f32",
        "kernel": kc.kernel_name(), "tag": f"{_tag(kc.kernel_name())}_{name}",
    }


def _spmv_coo_workload(dev, torch, fs, synthetic):
    from flagsparse_amd import spmv_coo as mod

    data, row, col, x, shape = synthetic.coo_uniform(device=dev)
    prepared, prep_call_ms = _timed_prepare(
        lambda: fs.prepare_spmv_coo(data, row, col, shape), torch)
    y = torch.empty(shape[0], dtype=data.dtype, device=dev)
    v = data.element_size()
    nnz = int(data.numel())
    runs = prepared.n_segs
    layout, layout_ms = _timed_prepare(prepared._run_layout, torch)  # built on first use
    nbytes = nnz * (v + 4) + (runs + 1) * 4 + shape[1] * v + shape[0] * v
    if prepared._run_rows is not None:  # the run -> row map, and y zeroed first
        nbytes += runs * 4 + shape[0] * v
    plan = dict(prepared._kernel_plan_description(),
                layout_bytes=int(layout.held_bytes((data, row, col))))
    info = {"n_rows": shape[0], "n_cols": shape[1], "nnz": nnz, "row_runs": runs,
            "bytes_literal_row_col_val": nnz * (v + 8) + shape[1] * v + shape[0] * v,
            "plan": plan, "prepare_ms": round(prep_call_ms + layout_ms, 3),
            "prepare_call_ms": prep_call_ms, "layout_build_ms": layout_ms,
            "inputs": {"data": data, "row": row, "col": col, "x": x}}

    def cpu(seconds):
        from oracle import oracle

        passes, secs = oracle.time_spmv_coo(row, col, data, x, shape[0], min_seconds=seconds)
        return {"value": round(nbytes * passes / secs / 1e9, 3), "unit": "GB/s", "cores": 1,
                "kind": "port",
                "sample": f"{passes} full passes of the fp64 C oracle COO SpMV in {secs:.1f} s",
                "gflops": round(2 * nnz * passes / secs / 1e9, 3)}

    return {
        "step": lambda: fs.flagsparse_spmv_coo(x=x, prepared=prepared, out=y),
        "launch": lambda: mod._run_spmv_coo(prepared, x, y, 256),
        "bytes_gather_inclusive": nbytes - shape[1] * v + nnz * v,
        "nbytes": nbytes, "flops": 2 * nnz, "info": info, "cpu": cpu, "dtype": "f32",
        "cpu_lib": _cpu_lib("coo", (row, col, data), x, shape, nbytes, 2 * nnz, torch),
        "kernel": prepared._kernel_name(), "tag": f"{_tag(prepared._kernel_name())}_cfg4",
    }


def _spmm_workload(dev, dtype_name, N, torch, fs, synthetic, part="all"):
    from flagsparse_amd import spmm_csr as mod

    vdt = torch.float64 if dtype_name == "f64" else torch.float32
    halves = {"all": {}, "band": {"rand_nnz": 0}, "random": {"band_nnz": 0}}[part]
    data, idx, ptr, shape = synthetic.csr_banded_random(dtype=vdt, device=dev, **halves)
    B = synthetic.dense_uniform(shape[1], N, dtype=vdt, device=dev)
    prepared, prep_call_ms = _timed_prepare(
        lambda: fs.prepare_spmm_csr_opt(data, idx, ptr, shape), torch)
    C = torch.empty((shape[0], N), dtype=vdt, device=dev)
    kc, layout_ms = _timed_prepare(prepared._kernel_csr, torch)
    v = data.element_size()
    nnz = int(data.numel())
    p_k = 4 if kc.rowptr_bits == 32 else 8
    nbytes = nnz * (v + 4) + (shape[0] + 1) * p_k + shape[1] * N * v + shape[0] * N * v
    launch = lambda: mod._run_spmm(kc, B, C, acc_f64=vdt == torch.float64)  # noqa: E731
    launch()  # the plan for this N and its workspace are built on the first launch
    torch.cuda.synchronize()
    from flagsparse_amd._spmv_layouts import tensor_bytes

    theirs = {t.untyped_storage().data_ptr() for t in (data, idx, ptr)}
    held = tensor_bytes(*[t for t in kc._keep if t.untyped_storage().data_ptr() not in theirs])
    info = {"n_rows": shape[0], "n_cols": shape[1], "nnz": nnz, "N": N,
            "path": "flagsparse_spmm_csr_opt (native accumulation)",
            "plan": dict(kc.describe(), layout_bytes=int(held)),
            "prepare_ms": round(prep_call_ms + layout_ms, 3), "prepare_call_ms": prep_call_ms,
            "layout_build_ms": layout_ms,
            "inputs": {"data": data, "indices": idx, "indptr": ptr, "B": B}}
    if part != "all":
        info["path"] += f"; only the {part} half of cfg5's rows (16 entries per row)"
    gather_bound = None
    if N == 64 and vdt == torch.float32 and part != "band":
        # cfg5: 16 of the 32 entries of every row at uniform random columns
        n_rand = nnz if part == "random" else nnz // 2
        gather_bound = lambda: _rows_bound(shape[1], n_rand, dev, torch,  # noqa: E731
                                           f"{n_rand} random 256-byte row gathers (cfg5's "
                                           f"random half) from a B of {shape[1] * 256} bytes")

    def cpu(seconds):
        from oracle import oracle

        rows = max(1, min(shape[0], int(20e6 // max(1, 32 * N))))
        passes, secs, r, nz = oracle.time_spmm_csr(ptr, idx, data, B, min_seconds=seconds,
                                                   row_limit=rows)
        frac = r / shape[0]
        return {"value": round(nbytes * frac * passes / secs / 1e9, 3), "unit": "GB/s",
                "cores": 1, "kind": "port",
                "sample": f"{passes} passes of the fp64 C oracle SpMM over the first {r} rows "
                          f"({nz} nnz) in {secs:.1f} s; bytes scaled by the row fraction",
                "gflops": round(2 * nz * N * passes / secs / 1e9, 3)}

    return {
        "step": lambda: fs.flagsparse_spmm_csr_opt(B=B, prepared=prepared, out=C),
        "launch": launch, "gather_bound": gather_bound,
        "bytes_gather_inclusive": nnz * (v + 4 + N * v) + (shape[0] + 1) * p_k +
        shape[0] * N * v,
        "nbytes": nbytes, "flops": 2 * nnz * N, "info": info, "cpu": cpu,
        "cpu_lib": _cpu_lib("csr", (ptr, idx, data), B, shape, nbytes, 2 * nnz * N, torch),
        "dtype": dtype_name, "kernel": kc.kernel_name(),
        "tag": f"{kc.kernel_name()}_cfg5_{dtype_name}_n{N}" + ("" if part == "all" else
                                                                f"_{part}_half"),
    }


def _spmm_coo_workload(dev, dtype_name, N, torch, fs, synthetic):
    from flagsparse_amd import spmm_coo as mod

    vdt = torch.float64 if dtype_name == "f64" else torch.float32
    data, idx, ptr, shape = synthetic.csr_banded_random(dtype=vdt, device=dev)
    row = torch.repeat_interleave(torch.arange(shape[0], device=dev, dtype=torch.int32),
                                  (ptr[1:] - ptr[:-1]).to(torch.int64))
    col = idx.to(torch.int32)
    del ptr, idx
    B = synthetic.dense_uniform(shape[1], N, dtype=vdt, device=dev)
    C = torch.empty((shape[0], N), dtype=vdt, device=dev)
    coo = mod._CooRowOrder(data, row, col, shape[0], shape[1])
    kc = coo.kernel_csr()
    v = data.element_size()
    nnz = int(data.numel())
    # the kernel reads the CSR view: values, int32 columns, int32 row pointers
    nbytes = nnz * (v + 4) + (shape[0] + 1) * 4 + shape[1] * N * v + shape[0] * N * v
    info = {"n_rows": shape[0], "n_cols": shape[1], "nnz": nnz, "N": N,
            "path": "flagsparse_spmm_coo (row-run route, fp64 accumulation for fp32)",
            "bytes_literal_row_col_val": nnz * (v + 8) + shape[1] * N * v + shape[0] * N * v,
            "inputs": {"data": data, "row": row, "col": col, "B": B}}

    def cpu(seconds):
        from oracle import oracle

        n = max(1, min(nnz, int(20e6 // max(1, N))))
        r, c, d = row[:n].cpu(), col[:n].cpu(), data[:n].cpu()
        Bh = B.cpu()
        n_rows = int(r[-1]) + 1
        passes, t0 = 0, time.perf_counter()
        while True:
            oracle.spmm_coo(r, c, d, Bh, n_rows)
            passes += 1
            secs = time.perf_counter() - t0
            if secs >= seconds or passes >= 1000:
                break
        frac = n / nnz
        return {"value": round(nbytes * frac * passes / secs / 1e9, 3), "unit": "GB/s",
                "cores": 1, "kind": "port",
                "sample": f"{passes} passes of the fp64 C oracle COO SpMM over the first {n} "
                          f"entries in {secs:.1f} s; bytes scaled by the entry fraction",
                "gflops": round(2 * n * N * passes / secs / 1e9, 3)}

    return {
        "step": lambda: fs.flagsparse_spmm_coo(data, row, col, B, shape, out=C),
        "launch": lambda: mod._run_spmm(kc, B, C, acc_f64=True),
        "nbytes": nbytes, "flops": 2 * nnz * N, "info": info, "cpu": cpu,
        "dtype": dtype_name, "kernel": kc.kernel_name(),
        "tag": f"{kc.kernel_name()}_coo5_{dtype_name}_n{N}",
    }


def _sddmm_workload(dev, dtype_name, K, torch, fs, synthetic):
    from flagsparse_amd import sddmm_csr as mod

    vdt = torch.float64 if dtype_name == "f64" else torch.float32
    _, idx, ptr, shape = synthetic.csr_banded_random(dtype=vdt, device=dev)
    x = synthetic.dense_uniform(shape[0], K, dtype=vdt, seed=1, device=dev)
    y = synthetic.dense_uniform(shape[1], K, dtype=vdt, seed=2, device=dev)
    prepared, prep_ms = _timed_prepare(lambda: fs.prepare_sddmm_csr(idx, ptr, shape, k_hint=K),
                                       torch)
    out = torch.empty(prepared.nnz, dtype=vdt, device=dev)
    v = x.element_size()
    nnz = prepared.nnz
    # per entry: column, row id, result; x and y rows once each
    nbytes = nnz * (4 + 4 + v) + shape[0] * K * v + shape[1] * K * v
    info = {"n_rows": shape[0], "n_cols": shape[1], "nnz": nnz, "K": K,
            "path": "flagsparse_sddmm_csr (baseline variant)", "prepare_ms": prep_ms,
            "inputs": {"indices": idx, "indptr": ptr, "x": x, "y": y}}

    def cpu(seconds):
        from oracle import oracle

        rows = max(1, min(shape[0], int(20e6 // max(1, 32 * K))))
        ip = ptr[:rows + 1].cpu()
        ix = idx[:int(ip[-1])].cpu()
        xh, yh = x[:rows].cpu(), y.cpu()
        passes, t0 = 0, time.perf_counter()
        while True:
            oracle.sddmm_csr(ip, ix, xh, yh)
            passes += 1
            secs = time.perf_counter() - t0
            if secs >= seconds or passes >= 1000:
                break
        frac = rows / shape[0]
        return {"value": round(nbytes * frac * passes / secs / 1e9, 3), "unit": "GB/s",
                "cores": 1, "kind": "port",
                "sample": f"{passes} passes of the fp64 C oracle SDDMM over the first {rows} rows "
                          f"in {secs:.1f} s; bytes scaled by the row fraction",
                "gflops": round(2 * int(ip[-1]) * K * passes / secs / 1e9, 3)}

    return {
        "step": lambda: fs.flagsparse_sddmm_csr(x=x, y=y, prepared=prepared, out=out),
        "launch": lambda: mod._launch_sddmm(prepared, x, y, None, 1.0, 0.0, out, False),
        "bytes_gather_inclusive": nnz * (4 + 4 + v + 2 * K * v),
        "nbytes": nbytes, "flops": 2 * nnz * K, "info": info, "cpu": cpu,
        "dtype": dtype_name, "kernel": "sddmm_csr_kernel",
        "tag": f"sddmm_csr_kernel_{dtype_name}_k{K}",
    }


def _probe_indices(n, hi, xcd, dev, torch, per_block, group=0, range_len=0, sort=False):
    """n int32 indices uniform in [0, hi) (seed fixed); with xcd, the indices of workgroup b
    (per_block consecutive ones) lie in the (b mod 8)-th eighth of [0, hi) - workgroup b runs
    on XCD b mod 8.  With a group size, each group of that many consecutive indices draws from
    one range of range_len values (chosen at random) inside its eighth, and with sort the group
    is sorted and laid out lane-major: a thread of fsp_probe_gather takes 16 consecutive
    indices, so sorted index 64k + lane of a wave's 1024 goes to position 16 * lane + k."""
    g = torch.Generator(device=dev)
    g.manual_seed(20260)
    if not xcd:
        return torch.randint(0, hi, (n,), generator=g, device=dev, dtype=torch.int32)
    w = max(1, hi // 8)
    blk = torch.arange(n, device=dev, dtype=torch.int64) // per_block
    if not group:
        r = torch.randint(0, w, (n,), generator=g, device=dev, dtype=torch.int64)
        return ((blk % 8) * w + r).to(torch.int32)
    if group % 1024 or per_block % group or n % per_block:
        raise SystemExit("--probe-group must be a multiple of 1024 dividing 4096, and the "
                         "gather count a multiple of 4096")
    span = min(w, range_len or w)
    n_groups = n // group
    first = (torch.arange(n_groups, device=dev) * group // per_block % 8) * w +         torch.randint(0, w // span, (n_groups,), generator=g, device=dev) * span
    idx = first.repeat_interleave(group) +         torch.randint(0, span, (n,), generator=g, device=dev, dtype=torch.int64)
    if sort:
        idx = torch.sort(idx.view(n_groups, group), dim=1)[0]
        idx = idx.view(-1, 16, 64).transpose(1, 2).contiguous().view(-1)
    return idx.to(torch.int32)


def _probe_gather_call(x_len, n, xcd, dev, torch, group=0, range_len=0, sort=False):
    from flagsparse_amd import _abi

    L = _abi.lib()
    x = torch.ones(x_len, dtype=torch.float32, device=dev)
    idx = _probe_indices(n, x_len, xcd, dev, torch, 256 * 16, group, range_len, sort)
    out = torch.empty(max(1, int(L.fsp_probe_gather_blocks(n))), dtype=torch.float32, device=dev)
    args = (x.data_ptr(), x_len, idx.data_ptr(), n, out.data_ptr())

    def call():
        _abi.check(L.fsp_probe_gather(*args, _abi.raw_stream(dev)), "fsp_probe_gather")

    call.keep = (x, idx, out)
    return call


def _probe_rows_call(n_rows, n, dev, torch):
    from flagsparse_amd import _abi

    L = _abi.lib()
    B = torch.ones((n_rows, 64), dtype=torch.float32, device=dev)
    rows = _probe_indices(n, n_rows, False, dev, torch, 64)
    out = torch.empty(max(1, int(L.fsp_probe_rows_blocks(n))), dtype=torch.float32, device=dev)
    args = (B.data_ptr(), n_rows, 64, rows.data_ptr(), n, out.data_ptr())

    def call():
        _abi.check(L.fsp_probe_rows(*args, _abi.raw_stream(dev)), "fsp_probe_rows")

    call.keep = (B, rows, out)
    return call


def _bound(call, n, what, torch):
    """The probe's time (median of 5 runs of 20 back-to-back launches) as a gather bound."""
    for _ in range(3):
        call()
    ms = sorted(_event_loop(call, 20, torch) for _ in range(5))[2]
    return {"pattern": what, "gathers": int(n), "ms": round(ms, 6),
            "G_per_s": round(n / (ms * 1e-3) / 1e9, 2)}


def _stream_bound(nbytes, dev, torch, what):
    """A plain read of nbytes (fsp_probe_stream) timed as _bound times the gather probes."""
    from flagsparse_amd import _abi

    L = _abi.lib()
    n16 = max(1, int(nbytes) // 16)
    src = torch.empty(n16 * 16, dtype=torch.uint8, device=dev)
    out = torch.empty(max(1, int(L.fsp_probe_stream_blocks(n16))), dtype=torch.float32,
                      device=dev)

    def call():
        _abi.check(L.fsp_probe_stream(src.data_ptr(), n16, out.data_ptr(),
                                      _abi.raw_stream(dev)), "fsp_probe_stream")

    for _ in range(3):
        call()
    ms = sorted(_event_loop(call, 20, torch) for _ in range(5))[2]
    del src, out
    return {"pattern": what, "bytes": n16 * 16, "ms": round(ms, 6),
            "GB_per_s": round(n16 * 16 / (ms * 1e-3) / 1e9, 1)}


def _gather_bound(x_len, n, xcd, dev, torch, what):
    return _bound(_probe_gather_call(x_len, n, xcd, dev, torch), n, what, torch)


def _rows_bound(n_rows, n, dev, torch, what):
    return _bound(_probe_rows_call(n_rows, n, dev, torch), n, what, torch)


def _probe_workload(name, args, dev, torch):
    if name == "probe-gather":
        x_len = (args.probe_bytes or 8 * (1 << 20) * 4) // 4
        n = (args.probe_n or 100 * (1 << 20)) // 4 * 4
        group = args.probe_group if args.probe_xcd else 0
        if group:
            n = n // 4096 * 4096
        call = _probe_gather_call(x_len, n, args.probe_xcd, dev, torch, group,
                                  args.probe_range // 4, args.probe_sorted)
        nbytes = n * 8  # an index and a gathered value per gather
        info = {"x_bytes": x_len * 4, "gathers": n, "xcd_panels": bool(args.probe_xcd),
                "bytes_counted": "4-byte index + 4-byte value per gather"}
        tag = f"probe_gather_{x_len * 4}{'_xcd' if args.probe_xcd else ''}"
        if group:
            span = min(x_len // 8, args.probe_range // 4 or x_len // 8) * 4
            info.update({"group": group, "group_range_bytes": span,
                         "sorted_lane_major": bool(args.probe_sorted)})
            tag += f"_g{group}_r{span}{'_sorted' if args.probe_sorted else ''}"
    else:
        n_rows = (args.probe_bytes or (1 << 20) * 256) // 256
        n = args.probe_n or 16 * (1 << 20)
        call = _probe_rows_call(n_rows, n, dev, torch)
        nbytes = n * (256 + 4)
        info = {"b_bytes": n_rows * 256, "row_gathers": n,
                "bytes_counted": "256-byte row + 4-byte index per gather"}
        tag = f"probe_rows_{n_rows * 256}"
    return {"step": call, "launch": call, "nbytes": nbytes, "flops": 0, "info": info,
            "cpu": None, "dtype": "f32", "kernel": f"{name.replace('-', '_')}_kernel",
            "tag": tag, "gathers": n}


def _copy_workload(dev, torch):
    n = (1 << 30) // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)

    def step():
        dst.copy_(src)

    return {"step": step, "launch": step, "nbytes": 2 * n * 4, "flops": 0,
            "info": {"bytes_read": n * 4, "bytes_written": n * 4}, "cpu": None, "dtype": "f32",
            "kernel": "copy", "tag": "copy_1gib"}


def _build(name, args, dev, torch):
    import flagsparse_amd as fs
    from flagsparse_amd import synthetic

    if name in ("cfg1", "cfg2", "cfg3"):
        return _spmv_csr_workload(name, dev, args.opt, torch, fs, synthetic)
    if name == "cfg4":
        return _spmv_coo_workload(dev, torch, fs, synthetic)
    if name == "cfg5":
        return _spmm_workload(dev, args.dtype or "f32", int(args.n), torch, fs, synthetic,
                              getattr(args, "cfg5_part", "all"))
    if name == "coo5":
        return _spmm_coo_workload(dev, args.dtype or "f32", int(args.n), torch, fs, synthetic)
    if name == "sddmm":
        return _sddmm_workload(dev, args.dtype or "f32", int(args.n), torch, fs, synthetic)
    if name.startswith("probe-"):
        return _probe_workload(name, args, dev, torch)
    return _copy_workload(dev, torch)


KERNEL_TRIALS = 5


# Warm-up runs in chunks of W steps until at least this much time has passed: measured on
# MI355X, the first ~10 ms of back-to-back work run about 4 % slower (cfg2: 58.9 us per step
# in the first 200 steps after 20 warm-up steps, 56.6 us after).
WARM_SECONDS = 0.05


def _warm(fn, warmup, torch, seconds=WARM_SECONDS):
    """Run ``fn`` in chunks of ``warmup`` calls, synchronising after each chunk, until at least
    ``seconds`` have passed; returns the number of calls (0 when warmup is 0)."""
    if warmup <= 0:
        return 0
    n, t0 = 0, time.perf_counter()
    while True:
        for _ in range(warmup):
            fn()
        n += warmup
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return n


def _measure(w, steps, warmup, torch, trials=KERNEL_TRIALS):
    """(ms per step, host wall ms per step, median kernel ms, [kernel ms of each trial],
    first-call ms, warm-up steps run).  The first step after prepare is timed on its own, cold;
    then the warm-up (W steps at a time, untimed), the K timed steps, and ``trials`` runs of K
    back-to-back kernel launches."""
    first_ms = _event_loop(w["step"], 1, torch)
    warm_run = _warm(w["step"], warmup, torch)
    t0 = time.perf_counter()
    ms_step = _event_loop(w["step"], steps, torch)
    wall_ms = (time.perf_counter() - t0) * 1000.0 / steps
    for _ in range(max(1, warmup // 2)):
        w["launch"]()
    runs = [_event_loop(w["launch"], steps, torch) for _ in range(max(1, trials))]
    ms_kernel = sorted(runs)[len(runs) // 2]
    return ms_step, wall_ms, ms_kernel, runs, first_ms, warm_run


def _roofline(w, ms_kernel, kernel_runs, torch):
    """The roofline block of a workload measured at ms_kernel per launch (see the module
    docstring), with what the committed profile records and the gather bound measured now."""
    nbytes = w["nbytes"]
    achieved = nbytes / (ms_kernel * 1e-3) / 1e9
    prof = _profile(w["tag"])
    out = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
           "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
           "traffic": prof.get("traffic"), "kernel": w["kernel"],
           "kernel_ms": round(ms_kernel, 6),
           "kernel_ms_trials": [round(t, 6) for t in kernel_runs],
           "profile_tag": w["tag"]}
    if prof.get("traffic"):
        out["traffic_over_algorithmic"] = round(prof["traffic"] / nbytes, 3)
        # the rate the kernel moves what it does move: the profiled bytes over the time now
        rate = prof["traffic"] / (ms_kernel * 1e-3) / 1e9
        out["traffic_gbs"] = round(rate, 2)
        out["frac_traffic"] = round(rate / HBM_PEAK_GBS, 4)
    for key in ("l2_hit_rate", "occupancy_percent"):
        if key in prof:
            out[key] = prof[key]
    gi = w.get("bytes_gather_inclusive")
    if gi:
        out["bytes_gather_inclusive"] = int(gi)
        out["frac_gather_inclusive"] = round(gi / (ms_kernel * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    if w.get("parts"):
        out["parts_ms"] = {k: round(sorted(_event_loop(fn, 20, torch) for _ in range(3))[1], 6)
                           for k, fn in w["parts"].items()}
    if w.get("gather_bound"):
        gb = w["gather_bound"]()
        gb["kernel_ms_over_bound"] = round(ms_kernel / gb["ms"], 3)
        if w.get("bound_part") and w["bound_part"] in out.get("parts_ms", {}):
            # the part whose gathers the probe restates (its kernel and combine)
            gb["part"] = w["bound_part"]
            gb["part_ms_over_bound"] = round(out["parts_ms"][w["bound_part"]] / gb["ms"], 3)
        out["gather_bound"] = gb
    if w.get("stream_bound"):
        sb = w["stream_bound"]()
        part = w.get("stream_part")
        if part and part in out.get("parts_ms", {}):
            sb["part"] = part
            sb["part_ms_over_bound"] = round(out["parts_ms"][part] / sb["ms"], 3)
        out["stream_bound"] = sb
    return out


def _cpu_baselines(w, seconds, torch):
    """(cpu_baseline, cpu_port, cpu_reference_path) of a workload.  cpu_baseline: the
    reference's own CPU path (torch.sparse.mm on all of torch's host threads) for ``seconds``
    where the workload has one, else the C oracle; cpu_port: the fp64 C oracle on one core;
    cpu_reference_path: scipy.sparse on one core.  Reported only, never a target."""
    host = _host_info(torch)
    if w.get("cpu_lib") is None:
        port = w["cpu"](seconds)
        port["host"] = host
        return port, None, None
    torch_fn, scipy_fn = w["cpu_lib"]
    base = torch_fn(seconds)
    base["host"] = host
    return base, w["cpu"](seconds / 2), {"scipy": scipy_fn(seconds / 2)}


def _target(name, args, dev, torch, steps, cpu_seconds):
    class A:
        pass

    a = A()
    a.opt, a.dtype, a.n = False, "f32", 64
    w = _build(name, a, dev, torch)
    _, _, ms_kernel, runs, _, _ = _measure(w, steps, 5, torch, trials=3)
    out = {"workload": name if name != "cfg5" else "cfg5 (f32, N=64)",
           "bytes_per_launch": int(w["nbytes"]),
           "gflops": round(w["flops"] / (ms_kernel * 1e-3) / 1e9, 2),
           "roofline": _roofline(w, ms_kernel, runs, torch),
           "prepare_ms": w["info"].get("prepare_ms"), "plan": w["info"].get("plan")}
    if cpu_seconds > 0 and w["cpu"] is not None:
        out["cpu_baseline"], out["cpu_port"], out["cpu_reference_path"] = \
            _cpu_baselines(w, cpu_seconds, torch)
    del w
    torch.cuda.empty_cache()
    return out


def _lib_load_ms(torch):
    """Loading the HIP library and reading its capacities (once per process)."""
    from flagsparse_amd import _abi

    t0 = time.perf_counter()
    _abi.lib()
    _abi.caps()
    return round((time.perf_counter() - t0) * 1000.0, 3)


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (a "
              "multi-GPU version would shard A by row slabs balanced by entries, with x or B "
              "replicated on every GPU; it is not built)", file=sys.stderr)
        sys.exit(2)

    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib_ms = _lib_load_ms(torch)
    w = _build(args.workload, args, dev, torch)
    ms_step, wall_ms, ms_kernel, kernel_runs, first_ms, warm_run = _measure(
        w, args.steps, args.warmup, torch)
    nbytes, flops = w["nbytes"], w["flops"]
    value = nbytes / (ms_step * 1e-3) / 1e9
    roofline = _roofline(w, ms_kernel, kernel_runs, torch)
    cpu = cpu_port = cpu_lib = None
    if w["cpu"] is not None and not args.no_cpu and args.cpu_seconds > 0:
        cpu, cpu_port, cpu_lib = _cpu_baselines(w, args.cpu_seconds, torch)
    workload = f"{args.workload}: {WORKLOADS[args.workload]}"
    if args.workload in ("cfg5", "coo5"):
        workload = f"{args.workload} ({w['dtype']}, N={args.n}): {WORKLOADS[args.workload]}"
    if args.workload == "sddmm":
        workload = f"sddmm ({w['dtype']}, K={args.n}): {WORKLOADS['sddmm']}"
    info, dtype = dict(w["info"]), w["dtype"]
    inputs = info.pop("inputs", None)
    if inputs:
        from flagsparse_amd import synthetic

        info["inputs_sha256"] = _digests(inputs, synthetic)
    del inputs
    info["first_call_ms"] = round(first_ms, 6)
    info["lib_load_ms"] = lib_ms
    metric, unit = METRIC, "GB/s"
    if args.workload.startswith("probe-"):
        metric, unit = "random gather rate (measurement probe)", "G gathers/s"
        value = w["gathers"] / (ms_step * 1e-3) / 1e9
    del w
    torch.cuda.empty_cache()
    targets = None
    if not args.no_targets:
        cpu_s = 0.0 if args.no_cpu else args.cpu_seconds / 2
        targets = []
        if args.workload == "cfg3" and not args.opt:
            targets.append({"workload": "cfg3", "roofline": "the headline line"})
        else:
            targets.append(_target("cfg3", args, dev, torch, 20, cpu_s))
        targets.append(_target("cfg5", args, dev, torch, 20, cpu_s))
    out = {
        "metric": metric,
        "value": round(value, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm_run,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded SplitMix64 generators, flagsparse_amd/synthetic.py)",
        "config": dict({"workload": workload}, **info, bytes_per_step=int(nbytes),
                       flops_per_step=int(flops),
                       gflops=round(flops / (ms_step * 1e-3) / 1e9, 2),
                       host_wall_ms_per_step=round(wall_ms, 6)),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_port": cpu_port,
        "cpu_reference_path": cpu_lib,
        "targets": targets,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
