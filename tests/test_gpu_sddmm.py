"""CSR SDDMM on the GPU (sddmm_csr_kernel) against the fp64 C oracle, plus the reference's API
checks (tests/test_sddmm.py:514-557), its diagnostic variants (sddmm_csr.py:243-268) and the
benchmark case's result dictionary (:552-572).

Bars: fp64, and fp32 with float64 accumulation ("acc64"): relative L2 <= 1e-12 / 1e-5 against
the oracle.  fp32 accumulated in fp32 (the reference's baseline): the reference script's
tolerance atol 1e-4, rtol 1e-2 (tests/test_sddmm.py:41-42) and relative L2 <= 1e-5 for K <= 256.
"""

import numpy as np
import pytest
import torch

import flagsparse_amd as fs
from flagsparse_amd import sddmm_csr, synthetic
from oracle import oracle

pytestmark = pytest.mark.gpu


def _case(dev, n_rows, n_cols, nnz, K, dtype, seed, index64=False):
    data, indices, indptr = synthetic.build_random_csr(n_rows, n_cols, nnz, dtype, torch.int32,
                                                       dev, seed=seed)
    if not index64:
        indptr = indptr.to(torch.int32)
    x = synthetic.dense_uniform(n_rows, K, dtype, seed=seed + 1, device=dev)
    y = synthetic.dense_uniform(n_cols, K, dtype, seed=seed + 2, device=dev)
    return data, indices, indptr, x, y


def _check(out, indptr, indices, x, y, data, alpha, beta, acc64=False):
    ref = oracle.sddmm_csr(indptr, indices, x, y, data, alpha=alpha, beta=beta)
    assert out.shape == (ref.size,)
    if ref.size == 0:
        return
    if out.dtype == torch.float64 or acc64:
        bound = 1e-12 if x.dtype == torch.float64 else 1e-5
        assert oracle.rel_l2(out, ref) <= bound
    else:
        assert oracle.rel_l2(out, ref) <= 1e-5
        assert oracle.allclose_ratio(out, ref, 1e-4, 1e-2) <= 1.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("K", [1, 3, 8, 32, 64, 100, 128, 256, 600, 700, 1100])
def test_sddmm_random(dev, dtype, K):
    data, indices, indptr, x, y = _case(dev, 600, 500, 8000, K, dtype, seed=K)
    print(f"sddmm {dtype} K={K}", flush=True)
    out = fs.flagsparse_sddmm_csr(data=data, indices=indices, indptr=indptr, x=x, y=y,
                                  shape=(600, 500), alpha=0.75, beta=-1.5)
    assert out.dtype == dtype
    _check(out, indptr, indices, x, y, data, 0.75, -1.5)
    # no data term, a prepared pattern, an int64 indptr
    p = fs.prepare_sddmm_csr(indices, indptr.to(torch.int64), (600, 500), k_hint=K)
    out2 = fs.flagsparse_sddmm_csr(x=x, y=y, prepared=p)
    _check(out2, indptr, indices, x, y, None, 1.0, 0.0)


def test_sddmm_long_rows_and_both_schedules(dev):
    # rows far longer than the 128-entry split threshold (chunks shared by a workgroup) next to
    # empty and short rows; the row-block schedule against the one-group-per-entry schedule
    n_rows, n_cols, K = 40, 3000, 64
    lengths = torch.zeros(n_rows, dtype=torch.int64)
    lengths[3], lengths[7], lengths[20:30] = 5000, 129, 3
    indptr = torch.zeros(n_rows + 1, dtype=torch.int64)
    indptr[1:] = torch.cumsum(lengths, 0)
    nnz = int(indptr[-1])
    indices = synthetic.randint(8, 1, nnz, n_cols, "cpu").to(torch.int32)
    indptr, indices = indptr.to(dev), indices.to(dev)
    x = synthetic.dense_uniform(n_rows, K, torch.float32, seed=8, device=dev)
    y = synthetic.dense_uniform(n_cols, K, torch.float32, seed=9, device=dev)
    p = fs.prepare_sddmm_csr(indices, indptr, (n_rows, n_cols), k_hint=K)
    out = fs.flagsparse_sddmm_csr(x=x, y=y, prepared=p)
    _check(out, indptr, indices, x, y, None, 1.0, 0.0)
    # the one-group-per-entry schedule agrees (same lane split of K and reduction; the compiler
    # may contract the multiply-adds differently, so equality is up to rounding)
    flat = torch.empty_like(out)
    from flagsparse_amd import _abi
    lanes, vec = sddmm_csr._sddmm_lane_shape(K, x, y)
    _abi.check(_abi.lib().fsp_sddmm_csr(0, 0, 0, _abi.ptr(p.indices), _abi.ptr(p.row_ids), None,
                                        32, p.nnz, _abi.ptr(x), K, _abi.ptr(y), K, K, None, 1.0,
                                        0.0, _abi.ptr(flat), None, None, 0, lanes, vec,
                                        _abi.stream_handle(dev)), "fsp_sddmm_csr")
    _check(flat, indptr, indices, x, y, None, 1.0, 0.0)
    torch.testing.assert_close(out, flat, rtol=1e-6, atol=1e-6)


def test_sddmm_strided_and_unaligned_dense(dev):
    # x, y with row strides that are not multiples of 4 and an odd K: the scalar-load path
    data, indices, indptr, x, y = _case(dev, 300, 200, 3000, 37, torch.float32, seed=5)
    xs = torch.zeros((300, 41), device=dev)[:, 1:38]
    xs.copy_(x)
    out = fs.flagsparse_sddmm_csr(data=data, indices=indices, indptr=indptr, x=xs, y=y,
                                  shape=(300, 200), beta=2.0)
    _check(out, indptr, indices, x, y, data, 1.0, 2.0)


@pytest.mark.parametrize("variant", ["baseline", "acc64", "acc64_out64", "altreduce"])
def test_sddmm_diagnostic_variants(dev, variant):
    data, indices, indptr, x, y = _case(dev, 400, 300, 5000, 64, torch.float32, seed=9)
    p = fs.prepare_sddmm_csr(indices, indptr, (400, 300), k_hint=64)
    out, meta = sddmm_csr._run_sddmm_prepared(p, x, y, data, 1.0, 0.5, None, variant=variant)
    assert meta["variant"] == variant and meta["fallback_used"] is False
    want_dtype = torch.float64 if variant == "acc64_out64" else torch.float32
    assert out.dtype == want_dtype
    assert meta["acc_dtype"] == ("float64" if variant.startswith("acc64") else "float32")
    _check(out, indptr, indices, x, y, data, 1.0, 0.5, acc64=variant.startswith("acc64"))


def test_sddmm_reference_api_cases(dev):
    # tests/test_sddmm.py:520-550
    indices = torch.tensor([0, 1, 1], dtype=torch.int32, device=dev)
    indptr = torch.tensor([0, 2, 3], dtype=torch.int64, device=dev)
    shape = (2, 2)
    x = synthetic.dense_uniform(2, 8, torch.float32, seed=1, device=dev)
    y = synthetic.dense_uniform(2, 8, torch.float32, seed=2, device=dev)
    data = synthetic.uniform_values(3, 1, 3, torch.float32, dev)
    cases = [
        (lambda: fs.flagsparse_sddmm_csr(indices=indices.to(torch.int64), indptr=indptr, x=x,
                                         y=y, shape=shape), TypeError),
        (lambda: fs.flagsparse_sddmm_csr(indices=indices, indptr=indptr, x=x, y=y[:, :4],
                                         shape=shape), ValueError),
        (lambda: fs.flagsparse_sddmm_csr(data=data[:2], indices=indices, indptr=indptr, x=x,
                                         y=y, shape=shape), ValueError),
        (lambda: fs.flagsparse_sddmm_csr(indices=indices, indptr=indptr, x=x, y=y, shape=shape,
                                         beta=0.5), ValueError),
        (lambda: fs.flagsparse_sddmm_csr(data=data, indices=indices, indptr=indptr, x=x[:, :0],
                                         y=y[:, :0], shape=shape,
                                         out=torch.empty(2, dtype=torch.float32, device=dev)),
         ValueError),
        (lambda: fs.flagsparse_sddmm_csr(indices=indices, indptr=indptr, x=x.to(torch.float64),
                                         y=y, shape=shape), TypeError),
        (lambda: fs.flagsparse_sddmm_csr(
            indices=torch.tensor([0, 2, 1], dtype=torch.int32, device=dev), indptr=indptr, x=x,
            y=y, shape=shape), IndexError),
        (lambda: fs.flagsparse_sddmm_csr(
            indices=indices, indptr=torch.tensor([0, 2, 4], device=dev), x=x, y=y, shape=shape),
         ValueError),  # indptr[-1] != nnz
        (lambda: fs.flagsparse_sddmm_csr(
            indices=indices, indptr=torch.tensor([0, 4, 3], device=dev), x=x, y=y, shape=shape),
         ValueError),  # not nondecreasing
        (lambda: fs.flagsparse_sddmm_csr(indices=indices, indptr=indptr, x=x, y=y, shape=shape,
                                         out=torch.empty(3, dtype=torch.float64, device=dev)),
         TypeError),
    ]
    for fn, exc in cases:
        with pytest.raises(exc):
            fn()
    out = fs.flagsparse_sddmm_csr(data=data, indices=indices, indptr=indptr, x=x, y=y,
                                  shape=shape, alpha=1.25, beta=0.5)
    assert out.shape == (3,)
    _check(out, indptr, indices, x, y, data, 1.25, 0.5)


def test_sddmm_edges_and_return_forms(dev):
    data, indices, indptr, x, y = _case(dev, 50, 40, 300, 16, torch.float64, seed=3)
    # K = 0: only the beta term (or zeros)
    out = fs.flagsparse_sddmm_csr(data=data, indices=indices, indptr=indptr, x=x[:, :0],
                                  y=y[:, :0], shape=(50, 40), beta=3.0)
    assert torch.equal(out, data * 3.0)
    out = fs.flagsparse_sddmm_csr(indices=indices, indptr=indptr, x=x[:, :0], y=y[:, :0],
                                  shape=(50, 40))
    assert torch.count_nonzero(out) == 0
    # no entries
    e_idx = torch.empty(0, dtype=torch.int32, device=dev)
    e_ptr = torch.zeros(51, dtype=torch.int64, device=dev)
    assert fs.flagsparse_sddmm_csr(indices=e_idx, indptr=e_ptr, x=x, y=y,
                                   shape=(50, 40)).shape == (0,)
    # out=, return_time, return_meta
    buf = torch.empty(300, dtype=torch.float64, device=dev)
    r = fs.flagsparse_sddmm_csr(indices=indices, indptr=indptr, x=x, y=y, shape=(50, 40),
                                out=buf, return_time=True, return_meta=True)
    assert len(r) == 3 and r[0].data_ptr() == buf.data_ptr() and r[1] >= 0.0
    assert {"prepare_ms", "block_k", "num_warps", "fallback_used", "variant"} <= set(r[2])
    _check(buf, indptr, indices, x, y, None, 1.0, 0.0)
    out, meta = fs.flagsparse_sddmm_csr(indices=indices, indptr=indptr, x=x, y=y,
                                        shape=(50, 40), return_meta=True, allow_fallback=True)
    assert meta["fallback_used"] is False and meta["block_k"] == 32


def test_sddmm_is_deterministic(dev):
    data, indices, indptr, x, y = _case(dev, 800, 700, 20000, 96, torch.float32, seed=12)
    a = fs.flagsparse_sddmm_csr(data=data, indices=indices, indptr=indptr, x=x, y=y,
                                shape=(800, 700), beta=1.0)
    b = fs.flagsparse_sddmm_csr(data=data, indices=indices, indptr=indptr, x=x, y=y,
                                shape=(800, 700), beta=1.0)
    assert torch.equal(a, b)


def test_benchmark_sddmm_case(dev):
    r = fs.benchmark_sddmm_case(n_rows=300, n_cols=250, nnz=4000, k_dim=48, warmup=1, iters=2,
                                alpha=2.0, beta=0.5)
    assert set(r) == {"parameters", "performance", "verification", "backend_status", "samples"}
    assert set(r["parameters"]) == {"n_rows", "n_cols", "nnz", "k_dim", "value_dtype", "warmup",
                                    "iters", "alpha", "beta"}
    assert set(r["verification"]) == {"triton_match_pytorch", "triton_max_abs_error",
                                      "cusparse_match_pytorch"}
    # float32: the case compares with torch's float32 sampled dot under the float32 table
    # (_common.py:76-85, atol 1e-6), so two float32 summation orders can differ by more than
    # that near zero; the error itself stays at float32 rounding level
    assert r["verification"]["triton_max_abs_error"] < 1e-4
    r = fs.benchmark_sddmm_case(n_rows=64, n_cols=64, nnz=500, k_dim=8,
                                value_dtype=torch.float64, warmup=1, iters=2)
    assert r["verification"]["triton_match_pytorch"]
    with pytest.raises(TypeError):
        fs.benchmark_sddmm_case(value_dtype=torch.float16)
    assert np.isfinite(r["performance"]["triton_ms"])
