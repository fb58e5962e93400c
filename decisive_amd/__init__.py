"""decisive_amd: MI355X (gfx950) quantized matrix-product path of decisive.

The product is libdecisive_rocm.so (HIP kernels + C ABI, include/decisive_rocm.h).
`decisive_amd.rocm` binds it with ctypes. The reference's Backend / Model<B> /
Cache interface over that library is C++, in decisive_amd/host/
(inference.hpp, rocm_backend.hpp, pplx_backend.hpp).
"""
from . import rocm  # noqa: F401

__all__ = ["rocm"]
