"""CPU-only checks of the C-ABI boundary (no GPU): the library loads without a GPU, exports
exactly what include/nanoserve_w4.h declares, and rejects every invalid argument with the
reference's return codes (csrc/nanoserve_ops.cu:65-90) before touching HIP."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

from nanoserve_amd import LIB_PATH, Kernels
from nanoserve_amd.ops import SIGNATURES

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nanoserve_w4.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\bint\s+(ns_\w+)\s*\(", text)))


def test_header_declares_the_reference_entry_points():
    assert declared_symbols() == ["ns_w4_linear", "ns_w4_quantize"]


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB_PATH), "build with python -m nanoserve_amd.build"
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT\s+(ns_\w+)$", out, flags=re.M))
    assert set(declared_symbols()) <= exported
    assert set(SIGNATURES) == set(declared_symbols())
    lib = ctypes.CDLL(LIB_PATH)
    for name in declared_symbols():
        assert callable(getattr(lib, name))


@pytest.fixture(scope="module")
def k():
    return Kernels()


P = 0x10000  # a 64 KiB-aligned non-null address: never dereferenced on these paths


@pytest.mark.parametrize("M,N,K,G", [
    (0, 128, 128, 128), (-1, 128, 128, 128), (1, 0, 128, 128), (1, 128, 0, 128),
    (1, 128, 128, 0), (9, 128, 128, 128), (127, 128, 128, 128), (129, 128, 128, 128),
    (128, 64, 128, 128), (128, 128, 96, 64), (1, 128, 100, 128), (1, 128, 128, 48),
    (2, 128, 256, 96), (4, 128, 192, 128), (256, 128, 192, 128),
])
def test_linear_rejects_unsupported_shapes(k, M, N, K, G):
    assert k.lib.ns_w4_linear(P, P, P, P, M, N, K, G, None) == -2


def test_linear_rejects_null_and_misaligned(k):
    assert k.lib.ns_w4_linear(None, P, P, P, 1, 128, 128, 128, None) == -2
    assert k.lib.ns_w4_linear(P, None, P, P, 1, 128, 128, 128, None) == -2
    assert k.lib.ns_w4_linear(P, P, None, P, 1, 128, 128, 128, None) == -2
    assert k.lib.ns_w4_linear(P, P, P, None, 1, 128, 128, 128, None) == -2
    assert k.lib.ns_w4_linear(P + 8, P, P, P, 1, 128, 128, 128, None) == -2
    assert k.lib.ns_w4_linear(P, P + 4, P, P, 1, 128, 128, 128, None) == -2
    assert k.lib.ns_w4_linear(P, P, P + 1, P, 1, 128, 128, 128, None) == -2
    assert k.lib.ns_w4_linear(P, P, P, P + 1, 1, 128, 128, 128, None) == -2


@pytest.mark.parametrize("N,K,G", [(16, 100, 128), (16, 256, 48), (16, 256, 0), (-1, 128, 128),
                                   (16, -128, 128), (16, 192, 128)])
def test_quantize_rejects_bad_arguments(k, N, K, G):
    assert k.lib.ns_w4_quantize(P, P, P, N, K, G, None) == -1


def test_quantize_empty_is_noop(k):
    assert k.lib.ns_w4_quantize(None, None, None, 0, 128, 128, None) == 0
    assert k.lib.ns_w4_quantize(None, None, None, 16, 0, 128, None) == 0


def test_quantize_rejects_null_and_misaligned(k):
    assert k.lib.ns_w4_quantize(None, P, P, 16, 128, 128, None) == -1
    assert k.lib.ns_w4_quantize(P + 2, P, P, 16, 128, 128, None) == -1


def test_python_wrapper_refuses_cpu_tensors(k):
    x = torch.zeros(1, 128, dtype=torch.bfloat16)
    Wq = torch.zeros(16, 16, dtype=torch.int32)
    S = torch.zeros(16, 1, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        k.w4_linear(x, Wq, S)
    with pytest.raises(ValueError):
        k.w4_quantize(torch.zeros(16, 128, dtype=torch.bfloat16))


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(OSError):
        Kernels(str(tmp_path / "missing.so"))
