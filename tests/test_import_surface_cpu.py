"""The reference's import name works unchanged: the import statements of the reference's
test scripts resolve to this build, and every name those scripts take from the imported
modules exists (no GPU: attributes only).

The statements are the scripts' own (tests/test_spmm.py:25-26, tests/test_spmv.py:12,
tests/test_spmv_coo.py:9, tests/test_spmm_coo.py:25-26, tests/test_sddmm.py:32-33,
tests/test_spmm_opt.py:23, tests/test_spmv_opt.py:16), and the name lists are every
``<alias>.<name>`` those scripts use.
"""

import importlib

import pytest

import flagsparse_amd

# script -> (import statement, {alias: [names used through it]})
SCRIPTS = {
    "tests/test_spmm.py": (
        "import flagsparse as ast\nimport flagsparse.sparse_operations.spmm_csr as ast_ops",
        {"ast": ["benchmark_spmm_case", "flagsparse_spmm_csr"],
         "ast_ops": ["_benchmark_cuda_op", "_spmm_validation_metrics"]}),
    "tests/test_spmv.py": (
        "import flagsparse as ast",
        {"ast": ["benchmark_spmv_case", "flagsparse_spmv_csr", "prepare_spmv_csr"]}),
    "tests/test_spmv_coo.py": (
        "import flagsparse as fs",
        {"fs": ["flagsparse_spmv_coo", "prepare_spmv_coo"]}),
    "tests/test_spmv_opt.py": (
        "import flagsparse as fs",
        {"fs": ["flagsparse_spmv_csr", "prepare_spmv_csr"]}),
    "tests/test_spmm_opt.py": (
        "import flagsparse as fs",
        {"fs": ["flagsparse_spmm_csr", "flagsparse_spmm_csr_opt", "prepare_spmm_csr_opt"]}),
    "tests/test_spmm_coo.py": (
        "import flagsparse as ast\nimport flagsparse.sparse_operations.spmm_coo as ast_ops",
        {"ast": ["flagsparse_spmm_coo"],
         "ast_ops": ["_benchmark_cuda_op", "_benchmark_spmm_coo_canonical_route",
                     "_build_spmm_coo_pytorch_reference_from_canonical",
                     "_build_torch_sparse_coo", "_prepare_spmm_coo_canonical_prepared",
                     "_prepare_spmm_coo_inputs", "_spmm_coo_pairwise_summary",
                     "_spmm_validation_metrics", "benchmark_spmm_coo_case"]}),
    "tests/test_sddmm.py": (
        "import flagsparse as ast\nimport flagsparse.sparse_operations.sddmm_csr as ast_ops",
        {"ast": ["flagsparse_sddmm_csr", "prepare_sddmm_csr"],
         "ast_ops": ["_benchmark_cuda_op", "_cupy_from_torch", "_run_sddmm_prepared",
                     "_sddmm_reference", "_tolerance_for_dtype", "_torch_from_cupy", "cp",
                     "_normalize_sddmm_diagnostic_variant"]}),
}


@pytest.mark.parametrize("script", sorted(SCRIPTS))
def test_reference_script_imports_resolve(script):
    statement, used = SCRIPTS[script]
    scope = {}
    exec(statement, scope)  # the script's own import lines
    for alias, names in used.items():
        mod = scope[alias]
        for name in names:
            assert hasattr(mod, name), f"{script}: {alias}.{name}"


def test_modules_are_the_implementations():
    # the same module objects, so private helpers and state are shared
    for name in ("spmv_csr", "spmv_coo", "spmm_csr", "spmm_coo", "sddmm_csr", "benchmarks"):
        ref = importlib.import_module(f"flagsparse.sparse_operations.{name}")
        assert ref is importlib.import_module(f"flagsparse_amd.{name}")
    import flagsparse

    assert flagsparse.flagsparse_spmv_csr is flagsparse_amd.flagsparse_spmv_csr
    assert set(flagsparse_amd.__all__) <= set(dir(flagsparse))


def test_reference_scripts_see_no_cupy():
    # the scripts skip their cuSPARSE comparisons when cp is None (tests/test_sddmm.py:320)
    import flagsparse.sparse_operations.sddmm_csr as ast_ops

    assert ast_ops.cp is None
    with pytest.raises(RuntimeError):
        ast_ops._cupy_from_torch(None)


def test_out_of_scope_names_raise_when_called():
    import flagsparse
    import flagsparse.sparse_formats as formats
    import flagsparse.sparse_operations.spgemm_csr as spgemm

    for fn in (flagsparse.flagsparse_gather, spgemm.flagsparse_spgemm_csr,
               formats.create_csr_matrix):
        with pytest.raises(NotImplementedError):
            fn()


def test_spmm_coo_helpers_keep_the_reference_arity():
    # tests/test_spmm_coo.py:290 unpacks seven values, :298-311 nine
    import inspect

    import flagsparse.sparse_operations.spmm_coo as ast_ops

    assert len(inspect.signature(ast_ops._prepare_spmm_coo_inputs).parameters) == 5
    assert len(inspect.signature(ast_ops._prepare_spmm_coo_canonical_prepared).parameters) == 7
    assert len(inspect.signature(ast_ops._benchmark_spmm_coo_canonical_route).parameters) == 12
