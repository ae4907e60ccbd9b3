"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py with
scipy fp64 products) against the oracle on the CPU, and against the gfx950 kernels on the GPU.

CPU: the oracle reproduces every fixture's expected output; the seeded generator still
produces the fixture's cfg1 arrays bit for bit.
GPU: every public entry point on the fixture inputs, to north_star's bar (relative L2 error
<= 1e-5 fp32 / 1e-12 fp64 against the fp64 expected output) and the reference scripts'
allclose ratio (tests/test_spmv_opt.py:204-207, tests/test_spmm_opt.py:202-224).
"""

import glob
import os

import numpy as np
import pytest
import torch

from oracle import oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CSR_CASES = ["cfg1_csr_f32", "poisson64_f64", "ragged_f32", "ragged_f64"]
SPMM_CASES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(HERE, "spmm_*.npz")))
COO_SPMM_CASES = ["coo_spmm_ref_f32", "coo_spmm_ref_f64", "coo_spmm_dups_f32",
                  "coo_spmm_dups_f64"]
SDDMM_CASES = ["sddmm_f32_k64", "sddmm_f64_k33"]


def _load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_fixture_inventory():
    assert len(SPMM_CASES) == 10
    for name in CSR_CASES + ["coo_dups_f32", "longrow_spmm_f32"] + COO_SPMM_CASES + SDDMM_CASES:
        assert os.path.exists(os.path.join(HERE, name + ".npz"))


@pytest.mark.parametrize("name", CSR_CASES)
def test_oracle_spmv_csr_on_fixture(name):
    g = _load(name)
    y = oracle.spmv_csr(g["indptr"], g["indices"], g["data"], g["x"])
    np.testing.assert_allclose(y, g["y"], rtol=1e-12, atol=1e-12)


def test_oracle_spmv_coo_on_fixture():
    g = _load("coo_dups_f32")
    y = oracle.spmv_coo(g["row"], g["col"], g["data"], g["x"], int(g["shape"][0]))
    np.testing.assert_allclose(y, g["y"], rtol=1e-12, atol=1e-12)
    assert np.all(y[800:] == 0.0)


@pytest.mark.parametrize("name", SPMM_CASES + ["longrow_spmm_f32"])
def test_oracle_spmm_on_fixture(name):
    g = _load(name)
    C = oracle.spmm_csr(g["indptr"], g["indices"], g["data"], g["B"])
    np.testing.assert_allclose(C, g["C"], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("name", COO_SPMM_CASES)
def test_oracle_spmm_coo_on_fixture(name):
    g = _load(name)
    C = oracle.spmm_coo(g["row"], g["col"], g["data"], g["B"], int(g["shape"][0]))
    np.testing.assert_allclose(C, g["C"], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("name", SDDMM_CASES)
def test_oracle_sddmm_on_fixture(name):
    g = _load(name)
    out = oracle.sddmm_csr(g["indptr"], g["indices"], g["x"], g["y"], g["data"],
                           alpha=float(g["alpha"]), beta=float(g["beta"]))
    np.testing.assert_allclose(out, g["out"], rtol=1e-12, atol=1e-12)


def test_generator_reproduces_cfg1_fixture():
    from flagsparse_amd import synthetic

    g = _load("cfg1_csr_f32")
    d, i, p, x, shape = synthetic.csr_uniform_rows()
    assert tuple(g["shape"]) == shape
    for key, t in (("data", d), ("indices", i), ("indptr", p), ("x", x)):
        assert np.array_equal(g[key], t.numpy()), key


# ------------------------------------------------------------------------------------------
# GPU: the HIP kernels on the fixtures
# ------------------------------------------------------------------------------------------


def _check(out, expected):
    name = "float64" if out.dtype == torch.float64 else "float32"
    err = oracle.rel_l2(out, expected)
    assert err <= oracle.REL_L2_BOUND[name], err
    atol, rtol = oracle.REF_SCRIPT_TOL[name]
    assert oracle.allclose_ratio(out, expected, atol, rtol) <= 1.0


@pytest.mark.gpu
@pytest.mark.parametrize("name", CSR_CASES)
@pytest.mark.parametrize("use_opt", [False, True])
def test_gpu_spmv_csr_fixture(dev, name, use_opt):
    import flagsparse_amd as fs

    g = _load(name)
    t = {k: torch.from_numpy(g[k]).to(dev) for k in ("data", "indices", "indptr", "x")}
    shape = tuple(int(v) for v in g["shape"])
    print(f"fixture {name} use_opt={use_opt}", flush=True)
    y = fs.flagsparse_spmv_csr(t["data"], t["indices"], t["indptr"], t["x"], shape,
                               use_opt=use_opt)
    _check(y, g["y"])
    y2 = fs.flagsparse_spmv_coo_tocsr(
        t["data"], torch.repeat_interleave(torch.arange(shape[0], device=dev),
                                           t["indptr"][1:] - t["indptr"][:-1]),
        t["indices"], t["x"], shape, use_opt=use_opt)
    _check(y2, g["y"])


@pytest.mark.gpu
@pytest.mark.parametrize("sort_by_row", [True, False])
def test_gpu_spmv_coo_fixture(dev, sort_by_row):
    import flagsparse_amd as fs

    g = _load("coo_dups_f32")
    t = {k: torch.from_numpy(g[k]).to(dev) for k in ("data", "row", "col", "x")}
    shape = tuple(int(v) for v in g["shape"])
    y = fs.flagsparse_spmv_coo(t["data"], t["row"], t["col"], t["x"], shape,
                               sort_by_row=sort_by_row)
    _check(y, g["y"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", SPMM_CASES + ["longrow_spmm_f32"])
def test_gpu_spmm_fixture(dev, name):
    import flagsparse_amd as fs

    g = _load(name)
    t = {k: torch.from_numpy(g[k]).to(dev) for k in ("data", "indices", "indptr", "B")}
    shape = tuple(int(v) for v in g["shape"])
    print(f"fixture {name}", flush=True)
    C = fs.flagsparse_spmm_csr(t["data"], t["indices"], t["indptr"], t["B"], shape)
    _check(C, g["C"])
    C = fs.flagsparse_spmm_csr_opt(t["data"], t["indices"], t["indptr"], t["B"], shape)
    _check(C, g["C"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", COO_SPMM_CASES)
@pytest.mark.parametrize("route", ["rowrun", "atomic"])
def test_gpu_spmm_coo_fixture(dev, name, route):
    from flagsparse_amd import spmm_coo

    g = _load(name)
    t = {k: torch.from_numpy(g[k]).to(dev) for k in ("data", "row", "col", "B")}
    shape = tuple(int(v) for v in g["shape"])
    print(f"fixture {name} route={route}", flush=True)
    C = spmm_coo._run_spmm_coo_route(t["data"], t["row"], t["col"], t["B"], shape, route=route)
    _check(C, g["C"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", SDDMM_CASES)
def test_gpu_sddmm_fixture(dev, name):
    import flagsparse_amd as fs

    g = _load(name)
    t = {k: torch.from_numpy(g[k]).to(dev) for k in ("data", "indices", "indptr", "x", "y")}
    shape = tuple(int(v) for v in g["shape"])
    print(f"fixture {name}", flush=True)
    out = fs.flagsparse_sddmm_csr(data=t["data"], indices=t["indices"], indptr=t["indptr"],
                                  x=t["x"], y=t["y"], shape=shape, alpha=float(g["alpha"]),
                                  beta=float(g["beta"]))
    _check(out, g["out"])
