"""``flagsparse.sparse_operations``: each submodule of the reference on the path is the
flagsparse_amd module that implements it, the same module object (so its private helpers -
``_spmm_validation_metrics``, ``_benchmark_cuda_op``, ... - are there for the reference's
scripts).  The reference's other submodules (gather_scatter, spgemm_csr, spsv) exist, and any
name taken from them raises NotImplementedError when called."""

import sys
import types

from flagsparse_amd import *  # noqa: F401,F403
from flagsparse_amd import (  # noqa: F401
    _common,
    benchmarks,
    sddmm_csr,
    spmm_coo,
    spmm_csr,
    spmv_coo,
    spmv_csr,
)

_ON_PATH = {"_common": _common, "benchmarks": benchmarks, "sddmm_csr": sddmm_csr,
            "spmm_coo": spmm_coo, "spmm_csr": spmm_csr, "spmv_coo": spmv_coo,
            "spmv_csr": spmv_csr}
for _name, _mod in _ON_PATH.items():
    sys.modules[f"{__name__}.{_name}"] = _mod


def _out_of_scope_module(qualname):
    mod = types.ModuleType(qualname, f"{qualname}: outside the MI355X build (SpMV / SpMM / SDDMM "
                                     "only); every name raises NotImplementedError when called.")

    def __getattr__(name):
        if name.startswith("__"):
            raise AttributeError(name)

        def stub(*args, **kwargs):
            raise NotImplementedError(f"{qualname}.{name} is outside the MI355X build, which "
                                      "implements CSR/COO SpMV, CSR/COO SpMM and CSR SDDMM only")

        stub.__name__ = stub.__qualname__ = name
        return stub

    mod.__getattr__ = __getattr__
    sys.modules[qualname] = mod
    return mod


gather_scatter = _out_of_scope_module(f"{__name__}.gather_scatter")
spgemm_csr = _out_of_scope_module(f"{__name__}.spgemm_csr")
spsv = _out_of_scope_module(f"{__name__}.spsv")
