"""``flagsparse.sparse_formats``: the reference's CuPy-backed format containers
(src/flagsparse/sparse_formats.py) are outside the MI355X build; every name raises
NotImplementedError when called, as the top-level ``create_*_matrix`` / ``coo_to_*`` names do.
Matrix Market files load into torch CSR / COO tensors with flagsparse_amd.mtx."""


def __getattr__(name):
    if name.startswith("__"):
        raise AttributeError(name)

    def stub(*args, **kwargs):
        raise NotImplementedError(f"flagsparse.sparse_formats.{name} is outside the MI355X "
                                  "build (CuPy format containers)")

    stub.__name__ = stub.__qualname__ = name
    return stub
