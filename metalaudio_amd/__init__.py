"""MI355X-native MetalNN inference layers (gfx950 HIP kernels behind a C ABI).

The compute lives in libmnn.so (built by `python -m metalaudio_amd.build`); `metalaudio_amd.nn`
mirrors the reference's layer API over it.
"""
from ._lib import LIB_PATH, MNNError  # noqa: F401

__version__ = "0.1.0"
