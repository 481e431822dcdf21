"""nanoserve_amd: MI355X-native (gfx950) W4A16 linear-layer engine.

Drop-in for the W4 path of Uttaprexa/nanoserve: the C ABI ``ns_w4_linear`` / ``ns_w4_quantize``
(include/nanoserve_w4.h, built as ``libnanoserve_amd.so``) and the Python ``Kernels`` class with
``w4_linear`` / ``w4_quantize`` (reference python/nanoserve/ops.py:76-97).
"""
from .ops import Kernels, LIB_PATH  # noqa: F401

__all__ = ["Kernels", "LIB_PATH"]
