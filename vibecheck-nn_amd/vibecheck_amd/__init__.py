"""vibecheck_amd -- MI355X-native batched linear-bound-propagation engine.

Drop-in GPU implementations of the reference's bound primitives
(``verify_zono_bnb``) and input-split BaB step (``verify_graph``), computed
by hand-written HIP kernels for gfx950 in libvibecheck_amd.so (C ABI:
include/vibecheck_amd.h).
"""
from . import _lib, spec, workloads  # noqa: F401

__version__ = '0.1.0'


def library_path():
    return _lib.LIB_PATH


def load_library():
    """Load the HIP library; raises if it has not been built."""
    return _lib.load()
