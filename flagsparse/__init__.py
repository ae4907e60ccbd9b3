"""The reference package's import name, ``flagsparse``, resolved to the MI355X build.

Scripts written against the reference - ``import flagsparse``,
``import flagsparse.sparse_operations.spmm_csr as ast_ops`` - run unchanged: the top-level
names are flagsparse_amd's (the reference exports them at src/flagsparse/__init__.py:5-63,
lazily at :65-136), and ``flagsparse.sparse_operations.<module>`` is the flagsparse_amd module
that implements that reference module.  Names outside the SpMV / SpMM / SDDMM path raise
NotImplementedError when called, as ``flagsparse_amd``'s do.
"""

import flagsparse_amd as _impl
from flagsparse_amd import *  # noqa: F401,F403  (the reference's exports)
from flagsparse_amd import HOT_PATH_EXPORTS, OUT_OF_SCOPE_EXPORTS, __all__, __version__  # noqa: F401

from . import sparse_formats, sparse_operations  # noqa: F401,E402


def __getattr__(name):
    return getattr(_impl, name)


def __dir__():
    return sorted(set(globals()) | set(OUT_OF_SCOPE_EXPORTS))
