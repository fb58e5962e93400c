"""decisive_amd: MI355X (gfx950) quantized matrix-product path of decisive.

The product is libdecisive_rocm.so (HIP kernels + C ABI, include/decisive_rocm.h);
`decisive_amd.rocm` binds it with ctypes and `decisive_amd.inference` mirrors the
reference's Backend / Model<B> interface over it.
"""
from . import rocm  # noqa: F401

__all__ = ["rocm"]
