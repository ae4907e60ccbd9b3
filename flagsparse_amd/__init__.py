"""flagsparse_amd - MI355X (gfx950) CSR/COO SpMV, CSR/COO SpMM and CSR SDDMM behind FlagSparse's
API.

Drop-in for the hot path of the reference package ``flagsparse`` (src/flagsparse/__init__.py):
the names below keep the reference's signatures, defaults, return values and exceptions.
Names of the reference that lie outside this path (gather/scatter, SpSV, SpGEMM and the
CuPy-backed format containers) are listed in ``__all__`` as in the reference; calling them
raises NotImplementedError.

    import flagsparse_amd as flagsparse
    p = flagsparse.prepare_spmv_csr(data, indices, indptr, shape)
    y = flagsparse.flagsparse_spmv_csr(x=x, prepared=p)
"""

__version__ = "1.0.0"

from ._common import SUPPORTED_INDEX_DTYPES, SUPPORTED_VALUE_DTYPES  # noqa: F401
from .benchmarks import benchmark_spmv_case
from .spmm_csr import (
    PreparedCsrSpmmOpt,
    benchmark_spmm_case,
    benchmark_spmm_opt_case,
    comprehensive_spmm_test,
    flagsparse_spmm_csr,
    flagsparse_spmm_csr_opt,
    prepare_spmm_csr_opt,
)
from .sddmm_csr import SDDMMPrepared, benchmark_sddmm_case, flagsparse_sddmm_csr, prepare_sddmm_csr
from .spmm_coo import flagsparse_spmm_coo
from .spmv_coo import PreparedCoo, flagsparse_spmv_coo, prepare_spmv_coo
from .spmv_csr import (
    PreparedCsrSpmv,
    flagsparse_spmv_coo_tocsr,
    flagsparse_spmv_csr,
    prepare_spmv_coo_tocsr,
    prepare_spmv_csr,
)

HOT_PATH_EXPORTS = (
    "PreparedCoo",
    "PreparedCsrSpmv",
    "PreparedCsrSpmmOpt",
    "prepare_spmv_csr",
    "prepare_spmm_csr_opt",
    "prepare_spmv_coo",
    "prepare_spmv_coo_tocsr",
    "flagsparse_spmv_csr",
    "flagsparse_spmv_coo",
    "flagsparse_spmv_coo_tocsr",
    "flagsparse_spmm_csr_opt",
    "flagsparse_spmm_csr",
    "flagsparse_spmm_coo",
    "prepare_sddmm_csr",
    "flagsparse_sddmm_csr",
    "SDDMMPrepared",
    "benchmark_sddmm_case",
    "benchmark_spmm_case",
    "benchmark_spmm_opt_case",
    "comprehensive_spmm_test",
    "benchmark_spmv_case",
)

# Reference exports outside the SpMV / SpMM path (src/flagsparse/__init__.py:5-63).
OUT_OF_SCOPE_EXPORTS = (
    "flagsparse_gather",
    "flagsparse_scatter",
    "pytorch_index_gather",
    "pytorch_index_scatter",
    "cusparse_spmv_gather",
    "cusparse_spmv_scatter",
    "benchmark_gather_case",
    "benchmark_scatter_case",
    "benchmark_performance",
    "comprehensive_gather_test",
    "comprehensive_scatter_test",
    "flagsparse_spsv_csr",
    "flagsparse_spsv_coo",
    "prepare_spgemm_csr",
    "flagsparse_spgemm_csr",
    "SpGEMMPrepared",
    "benchmark_spgemm_case",
    "create_csr_matrix",
    "create_coo_matrix",
    "create_csc_matrix",
    "create_bsr_matrix",
    "create_sell_matrix",
    "create_blocked_ell_matrix",
    "coo_to_csr",
    "coo_to_csc",
    "coo_to_bsr",
    "coo_to_sell",
    "coo_to_blocked_ell",
    "CSRMatrix",
    "COOMatrix",
    "CSCMatrix",
    "BSRMatrix",
    "SELLMatrix",
    "BLOCKEDELLMatrix",
    "generate_random_sparse_matrix",
    "read_mtx_file",
)

__all__ = list(HOT_PATH_EXPORTS) + list(OUT_OF_SCOPE_EXPORTS)


def _out_of_scope(name):
    hint = ""
    if name == "read_mtx_file":
        hint = ("; .mtx files load into torch CSR / COO tensors with "
                "flagsparse_amd.mtx.load_mtx_to_csr_torch / load_mtx_to_coo_torch")

    def stub(*args, **kwargs):
        raise NotImplementedError(
            f"flagsparse.{name} is outside the MI355X build, which implements CSR/COO SpMV, "
            f"CSR/COO SpMM and CSR SDDMM only{hint}")

    stub.__name__ = name
    stub.__qualname__ = name
    return stub


def __getattr__(name):
    if name in OUT_OF_SCOPE_EXPORTS:
        return _out_of_scope(name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


def __dir__():
    return sorted(set(globals()) | set(OUT_OF_SCOPE_EXPORTS))
