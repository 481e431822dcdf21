"""ctypes bindings to libnanoserve_amd.so: the W4A16 part of the reference's ``Kernels`` class
(Uttaprexa/nanoserve python/nanoserve/ops.py:15-39, 76-97), same method names, argument
meaning, return values and exceptions.

The library is loaded with ctypes exactly as the reference loads build/libnanoserve.so; loading
needs no GPU. There is no CPU fallback: a missing library raises at construction, and tensors
that are not on the GPU raise before any native call.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnanoserve_amd.so")

# Exported symbols and their ctypes signatures (include/nanoserve_w4.h).
_VP, _I32 = ctypes.c_void_p, ctypes.c_int
SIGNATURES = {
    "ns_w4_quantize": [_VP, _VP, _VP, _I32, _I32, _I32, _VP],
    "ns_w4_linear": [_VP, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP],
}


def _require_gpu_tensor(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got device {t.device})")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")


class Kernels:
    """W4A16 kernels through the C ABI. ``path`` defaults to the in-tree library."""

    def __init__(self, path: str = LIB_PATH):
        path = os.path.abspath(path)
        if not os.path.exists(path):
            raise OSError(f"{path} not found: build it with `python -m nanoserve_amd.build` "
                          "(there is no CPU fallback)")
        self.lib = ctypes.CDLL(path)
        for name, args in SIGNATURES.items():
            fn = getattr(self.lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int

    # reference ops.py:32-34: the current torch stream (a hipStream_t on ROCm)
    @staticmethod
    def _stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    # reference ops.py:36-39
    @staticmethod
    def _check(rc: int, name: str):
        if rc != 0:
            raise RuntimeError(f"{name} failed with code {rc}")

    def w4_quantize(self, W, group=128):
        """W [N, K] bf16 -> (Wq int32 [N, K // 8], S bf16 [N, K // group]). Reference
        ops.py:76-83 (kernel: kernels/quant/w4a16.cuh:272-301)."""
        _require_gpu_tensor(W, "W", torch.bfloat16)
        N, K = W.shape
        Wq = torch.empty((N, K // 8), dtype=torch.int32, device=W.device)
        S = torch.empty((N, K // group), dtype=torch.bfloat16, device=W.device)
        W = W.contiguous()
        rc = self.lib.ns_w4_quantize(W.data_ptr(), Wq.data_ptr(), S.data_ptr(), N, K, group,
                                     self._stream())
        self._check(rc, "ns_w4_quantize")
        return Wq, S

    def w4_linear(self, x, Wq, S, group=128):
        """x [M, K] bf16 -> y [M, N] bf16 = x @ deq(Wq, S)^T. Reference ops.py:85-97.

        M <= 8 runs natively (the reference pads 3 -> 4 and 5..7 -> 8 with zero rows, which
        does not change any output row); larger M is padded with zero rows up to a multiple
        of 128, as the reference does."""
        _require_gpu_tensor(x, "x", torch.bfloat16)
        _require_gpu_tensor(Wq, "Wq", torch.int32)
        _require_gpu_tensor(S, "S", torch.bfloat16)
        M, K = x.shape
        N = Wq.shape[0]
        Mp = M if M <= 8 else ((M + 127) // 128) * 128
        if M == 0:
            Mp = 1
        if Mp != M:
            x = torch.cat([x, x.new_zeros(Mp - M, K)])
        x = x.contiguous()
        Wq = Wq.contiguous()
        S = S.contiguous()
        y = torch.empty((Mp, N), dtype=torch.bfloat16, device=x.device)
        rc = self.lib.ns_w4_linear(x.data_ptr(), Wq.data_ptr(), S.data_ptr(), y.data_ptr(), Mp, N,
                                   K, group, self._stream())
        self._check(rc, "ns_w4_linear")
        return y[:M]
