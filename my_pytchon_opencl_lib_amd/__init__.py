"""MI355X (gfx950) native fp32 matrix-multiplication path of my_pytchon_opencl_lib.

The compute lives in libmigemm.so (hand-written HIP kernels behind the C ABI of
include/migemm.h); this package is the Python host side: ctypes bindings (_native), the
operator dispatcher mirroring the reference's NnClGlob (nncl_glob) and the gradient nodes
(autograd).
"""
from . import _native
from .nncl_glob import NnClGlob, ShapeError
from ._native import MigemmArgumentError, MigemmRuntimeError

__all__ = ["NnClGlob", "ShapeError", "MigemmArgumentError", "MigemmRuntimeError", "_native",
           "autograd"]


def __getattr__(name):
    if name == "autograd":
        from . import autograd
        return autograd
    raise AttributeError(name)
