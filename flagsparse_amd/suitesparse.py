"""SuiteSparse-style batch runs over .mtx files (the reference's test drivers: run_one_mtx /
run_mtx_batch / CSV export of tests/test_spmv.py:106-520, tests/test_spmm.py, tests/test_sddmm.py
:232-512), for SpMV, SpMM and SDDMM.

Each file is loaded with flagsparse_amd.mtx (the reference's .mtx rules), run through the public
entry point, timed with HIP events on the current stream (steady state, after warm-up; the
prepare step outside the timed loop, as benchmarks.py:249-262 does) and checked against a
float64 torch computation of the same product with the reference scripts' tolerance
(float32: atol 1e-4, rtol 1e-2; float64: atol 1e-12, rtol 1e-10).

    python -m flagsparse_amd.suitesparse matrices/ --op spmv --csv results.csv
"""

import argparse
import csv
import glob
import os

import torch

from . import mtx
from .sddmm_csr import flagsparse_sddmm_csr, prepare_sddmm_csr
from .spmm_csr import flagsparse_spmm_csr_opt, prepare_spmm_csr_opt
from .spmv_csr import flagsparse_spmv_csr, prepare_spmv_csr
from .synthetic import dense_uniform, uniform_values

SCRIPT_TOL = {torch.float32: (1e-4, 1e-2), torch.float64: (1e-12, 1e-10)}
OPS = ("spmv", "spmm", "sddmm")
CSV_FIELDS = ("path", "op", "dtype", "n_rows", "n_cols", "nnz", "dense_cols", "ms", "gbs",
              "gflops", "rel_l2", "err_ratio", "ok", "error")


def expand_mtx_paths(raw_paths):
    """.mtx files and directories (their *.mtx, sorted) -> unique absolute paths, in order."""
    out, seen = [], set()
    for p in raw_paths:
        found = ([p] if os.path.isfile(p) and p.lower().endswith(".mtx")
                 else sorted(glob.glob(os.path.join(p, "*.mtx"))) if os.path.isdir(p) else [])
        for f in found:
            a = os.path.abspath(f)
            if a not in seen:
                seen.add(a)
                out.append(a)
    return out


def _time_ms(fn, warmup, iters):
    for _ in range(max(0, warmup)):
        fn()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(max(1, iters)):
        out = fn()
    end.record(stream)
    torch.cuda.synchronize()
    return out, start.elapsed_time(end) / max(1, iters)


def _compare(out, ref, dtype):
    out64 = out.to(torch.float64)
    denom = float(torch.linalg.vector_norm(ref))
    rel = float(torch.linalg.vector_norm(out64 - ref)) / denom if denom > 0 else \
        float(torch.linalg.vector_norm(out64 - ref))
    atol, rtol = SCRIPT_TOL[dtype]
    ratio = float(torch.max((out64 - ref).abs() / (atol + rtol * ref.abs()))) \
        if out.numel() else 0.0
    return rel, ratio


def run_mtx_case(path, op="spmv", value_dtype=torch.float32, dense_cols=32, warmup=5, iters=20,
                 use_opt=False, seed=0):
    """One .mtx file through one operation; returns a result row (CSV_FIELDS)."""
    if op not in OPS:
        raise ValueError(f"op must be one of {OPS}")
    dev = torch.device("cuda")
    row = {"path": path, "op": op, "dtype": str(value_dtype).replace("torch.", ""),
           "dense_cols": dense_cols if op != "spmv" else 0, "error": None, "ok": False}
    try:
        data, indices, indptr, shape = mtx.load_mtx_to_csr_torch(path, dtype=value_dtype,
                                                                 device=dev)
        n_rows, n_cols = shape
        nnz = int(data.numel())
        row.update(n_rows=n_rows, n_cols=n_cols, nnz=nnz)
        v = data.element_size()
        A64 = torch.sparse_csr_tensor(indptr, indices, data.to(torch.float64), size=shape)
        if op == "spmv":
            x = uniform_values(seed, 90, n_cols, value_dtype, dev)
            p = prepare_spmv_csr(data, indices, indptr, shape)
            out, ms = _time_ms(lambda: flagsparse_spmv_csr(x=x, prepared=p, use_opt=use_opt),
                               warmup, iters)
            ref = (A64 @ x.to(torch.float64)[:, None])[:, 0]
            nbytes = nnz * (v + 4) + (n_rows + 1) * 4 + n_cols * v + n_rows * v
            flops = 2 * nnz
        elif op == "spmm":
            B = dense_uniform(n_cols, dense_cols, value_dtype, seed=seed, stream=91, device=dev)
            p = prepare_spmm_csr_opt(data, indices, indptr, shape)
            out, ms = _time_ms(lambda: flagsparse_spmm_csr_opt(B=B, prepared=p), warmup, iters)
            ref = A64 @ B.to(torch.float64)
            nbytes = nnz * (v + 4) + (n_rows + 1) * 4 + (n_cols + n_rows) * dense_cols * v
            flops = 2 * nnz * dense_cols
        else:
            X = dense_uniform(n_rows, dense_cols, value_dtype, seed=seed, stream=92, device=dev)
            Y = dense_uniform(n_cols, dense_cols, value_dtype, seed=seed, stream=93, device=dev)
            p = prepare_sddmm_csr(indices.to(torch.int32), indptr, shape, k_hint=dense_cols)
            out, ms = _time_ms(lambda: flagsparse_sddmm_csr(x=X, y=Y, prepared=p), warmup, iters)
            rows = torch.repeat_interleave(torch.arange(n_rows, device=dev), indptr[1:] - indptr[:-1])
            ref = (X.to(torch.float64)[rows] * Y.to(torch.float64)[indices]).sum(1)
            nbytes = nnz * (4 + 4 + v) + (n_rows + n_cols) * dense_cols * v
            flops = 2 * nnz * dense_cols
        rel, ratio = _compare(out, ref, value_dtype)
        row.update(ms=ms, gbs=nbytes / (ms * 1e-3) / 1e9, gflops=flops / (ms * 1e-3) / 1e9,
                   rel_l2=rel, err_ratio=ratio, ok=bool(ratio <= 1.0))
    except Exception as exc:  # one bad file must not stop a batch
        row["error"] = f"{type(exc).__name__}: {exc}"
    return row


def run_mtx_batch(paths, op="spmv", value_dtype=torch.float32, dense_cols=32, warmup=5,
                  iters=20, use_opt=False, csv_path=None):
    """All .mtx files of ``paths`` (files or directories) through ``op``; optionally written to
    ``csv_path``.  Returns the result rows."""
    rows = [run_mtx_case(p, op, value_dtype, dense_cols, warmup, iters, use_opt)
            for p in expand_mtx_paths(paths)]
    if csv_path:
        parent = os.path.dirname(os.path.abspath(csv_path))
        os.makedirs(parent, exist_ok=True)
        with open(csv_path, "w", newline="") as fh:
            w = csv.DictWriter(fh, fieldnames=CSV_FIELDS, extrasaction="ignore")
            w.writeheader()
            for r in rows:
                w.writerow(r)
    return rows


def main(argv=None):
    ap = argparse.ArgumentParser(description="flagsparse_amd SuiteSparse .mtx batch runs")
    ap.add_argument("mtx", nargs="+", help=".mtx files or directories")
    ap.add_argument("--op", default="spmv", choices=OPS)
    ap.add_argument("--dtype", default="float32", choices=("float32", "float64"))
    ap.add_argument("--dense-cols", type=int, default=32, help="N for spmm, K for sddmm")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--use-opt", action="store_true", help="spmv: native accumulation")
    ap.add_argument("--csv", default=None)
    a = ap.parse_args(argv)
    dtype = torch.float32 if a.dtype == "float32" else torch.float64
    rows = run_mtx_batch(a.mtx, a.op, dtype, a.dense_cols, a.warmup, a.iters, a.use_opt, a.csv)
    for r in rows:
        if r["error"]:
            print(f"{os.path.basename(r['path']):40s} ERROR {r['error']}")
        else:
            print(f"{os.path.basename(r['path']):40s} {r['n_rows']}x{r['n_cols']} nnz={r['nnz']} "
                  f"{r['ms']:.4f} ms {r['gbs']:.1f} GB/s rel_l2={r['rel_l2']:.2e} "
                  f"{'PASS' if r['ok'] else 'FAIL'}")
    return 0 if all(r["ok"] for r in rows) else 1


if __name__ == "__main__":
    raise SystemExit(main())
