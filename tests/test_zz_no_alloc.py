"""fsp_spmv_csr_static (the allocation-free CSR SpMV entry point) against fsp_spmv_csr.

Both are called through the C ABI with the same row-block plan, matrix and x; the static entry
point keeps its split-row partial sums in the library's static device array instead of the
caller's workspace.  The results must be bit-identical (same kernels, same summation order),
on two calls in a row - the second with a smaller matrix, whose plan uses fewer partial slots
than the first left in the shared array - and both must match the fp64 oracle.  A plan that
needs more slots than the array holds is rejected before any launch.
"""

import numpy as np
import pytest
import torch

from flagsparse_amd import _abi, synthetic
from flagsparse_amd._spmv_layouts import RowBlockLayout
from oracle import oracle

pytestmark = pytest.mark.gpu


def _matrix(lengths, n_cols, seed, dtype):
    keys = synthetic._distinct_sorted_columns(torch.as_tensor(lengths, dtype=torch.int64),
                                              n_cols, seed, 1)
    ip, cols = synthetic._csr_from_keys(keys, len(lengths), n_cols)
    vals = synthetic.uniform_values(seed, 2, cols.numel(), dtype, "cpu")
    x = synthetic.uniform_values(seed, 3, n_cols, dtype, "cpu")
    return vals, cols.to(torch.int32), ip, x


def _args(lay, x, y, acc_f64, stream):
    plan = lay.plan
    groups, group_base, split_rows = plan.split_groups()
    p = lambda t: t.data_ptr() if t is not None and t.numel() else None  # noqa: E731
    head = [_abi.dtype_code(lay.data.dtype), int(acc_f64), p(lay.data), p(lay.cols), p(lay.rowptr),
            lay.rowptr_bits, lay.n_rows, lay.nnz, p(x), p(y), None, 0, p(plan.desc),
            p(plan.ranges), plan.n_desc, plan.chunk]
    tail = [p(groups), p(group_base), p(split_rows), int(groups.shape[0]), 0, stream]
    return head, tail, plan


def _both(dev, vals, cols, ip, x, acc_f64):
    L = _abi.lib()
    lay = RowBlockLayout(vals.to(dev), cols.to(dev), ip.to(dev))
    xd = x.to(dev)
    y_ws = torch.full((lay.n_rows,), float("nan"), dtype=vals.dtype, device=dev)
    y_st = torch.full((lay.n_rows,), float("nan"), dtype=vals.dtype, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    head, tail, plan = _args(lay, xd, y_ws, acc_f64, stream)
    ws = plan.workspace()
    _abi.check(L.fsp_spmv_csr(*head, ws.data_ptr(), *tail), "fsp_spmv_csr")
    head, tail, plan = _args(lay, xd, y_st, acc_f64, stream)
    _abi.check(L.fsp_spmv_csr_static(*head, plan.n_parts, *tail), "fsp_spmv_csr_static")
    torch.cuda.synchronize()
    return y_ws.cpu(), y_st.cpu(), plan


@pytest.mark.parametrize("dtype,acc_f64", [(torch.float32, True), (torch.float32, False),
                                           (torch.float64, True)])
def test_static_matches_workspace_twice(dev, dtype, acc_f64):
    L = _abi.lib()
    cap = int(L.fsp_spmv_scratch_slots())
    # first call: many rows split into chunks (thousands of partial slots); second: a smaller
    # matrix with fewer split rows, so stale slots of the first call sit past its plan
    cases = [([9000] * 300 + [7] * 500 + [30000] * 20, 60000, 1),
             ([5000] * 3 + [2] * 100, 7000, 2)]
    used = []
    for lengths, n_cols, seed in cases:
        print(f"static SpMV {dtype} acc_f64={acc_f64} rows={len(lengths)} seed={seed}", flush=True)
        vals, cols, ip, x = _matrix(lengths, n_cols, seed, dtype)
        y_ws, y_st, plan = _both(dev, vals, cols, ip, x, acc_f64)
        assert 0 < plan.n_parts <= cap
        used.append(plan.n_parts)
        assert torch.equal(y_ws, y_st)  # same kernels, same order: bit for bit
        ref = oracle.spmv_csr(ip, cols, vals, x)
        name = str(dtype).replace("torch.", "")
        assert oracle.rel_l2(y_st, ref) <= oracle.REL_L2_BOUND[name]
    assert used[1] < used[0]


def test_static_rejects_plan_larger_than_scratch(dev):
    L = _abi.lib()
    cap = int(L.fsp_spmv_scratch_slots())
    vals, cols, ip, x = _matrix([6000] * 4, 9000, 3, torch.float32)
    lay = RowBlockLayout(vals.to(dev), cols.to(dev), ip.to(dev))
    y = torch.zeros(lay.n_rows, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    head, tail, plan = _args(lay, x.to(dev), y, True, stream)
    rc = L.fsp_spmv_csr_static(*head, cap + 1, *tail)
    assert rc == -1 and b"static workspace" in L.fsp_last_error()
    torch.cuda.synchronize()
    assert np.all(y.cpu().numpy() == 0.0)  # nothing launched
