"""CPU oracle for the W4A16 linear-layer path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module, and only as the checker (or, for ``cpu_baseline``, as the timed CPU comparison).
The product package ``nanoserve_amd`` never imports it and has no CPU fallback.

Two layers:
  * ``libw4oracle.so`` (``w4_oracle.c``): exact C restatements of the reference's arithmetic,
    each citing the reference file:line it follows.
  * numpy/torch helpers below: the reference's error metrics and the PyTorch CPU
    dequant+matmul baseline.

Reference citations are paths inside Uttaprexa/nanoserve.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libw4oracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile ``libw4oracle.so`` with the Makefile beside this file."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, i32, u32, sz, f32 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_size_t,
                                 ctypes.c_float)
        sigs = {
            "orc_bf16_rne": ([f32], ctypes.c_uint16),
            "orc_bf16_rne_array": ([vp, vp, sz], None),
            "orc_hash_fill": ([vp, sz, u32, f32], None),
            "orc_quantize": ([vp, vp, vp, i32, i32, i32], ctypes.c_int),
            "orc_dequant_f32": ([vp, vp, vp, i32, i32, i32], None),
            "orc_dequant_bf16": ([vp, vp, vp, i32, i32, i32], None),
            "orc_linear_f64": ([vp, vp, vp, i32, i32, i32], None),
            "orc_linear_w4_f64": ([vp, vp, vp, vp, i32, i32, i32, i32, i32], None),
            "orc_gemv_ref_order": ([vp, vp, vp, vp, i32, i32, i32, i32], None),
            "orc_gptq": ([vp, vp, vp, vp, i32, i32, i32], ctypes.c_int),
        }
        for name, (args, res) in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------- bf16 bit helpers (uint16)
def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """Round to nearest even through the C restatement (vec.cuh:14-19)."""
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    lib().orc_bf16_rne_array(_p(f), _p(out), f.size)
    return out


# ----------------------------------------------------------------- restated reference functions
def hash_fill(n: int, seed: int, scale: float) -> np.ndarray:
    """bench/bench_w4a16.cu:32-40 (fill_kernel): n bf16 values (uint16 bit patterns)."""
    out = np.empty(n, dtype=np.uint16)
    lib().orc_hash_fill(_p(out), n, seed, scale)
    return out


def quantize(W: np.ndarray, G: int = 128):
    """kernels/quant/w4a16.cuh:272-297. W: uint16 bf16 bits [N, K] -> (Wq uint32 [N, K/8],
    S uint16 [N, K/G])."""
    W = np.ascontiguousarray(W, dtype=np.uint16)
    N, K = W.shape
    Wq = np.empty((N, K // 8), dtype=np.uint32)
    S = np.empty((N, max(K // G, 1)), dtype=np.uint16)
    rc = lib().orc_quantize(_p(W), _p(Wq), _p(S), N, K, G)
    if rc != 0:
        raise ValueError(f"orc_quantize rejected K={K}, G={G}")
    return Wq, S


def gptq(W: np.ndarray, U: np.ndarray, G: int = 128):
    """GPTQ restatement (orc_gptq in w4_oracle.c). W [N, K] float32 weights, U [K, K] float32
    upper Cholesky factor of the damped inverse Hessian -> (Wq uint32 [N, K/8], S uint16
    [N, K/G], Wpre float32 [N, K]: the value each column had when it was quantized)."""
    Wpre = np.array(W, dtype=np.float32, order="C", copy=True)
    U = np.ascontiguousarray(U, dtype=np.float32)
    N, K = Wpre.shape
    assert U.shape == (K, K)
    Wq = np.empty((N, K // 8), dtype=np.uint32)
    S = np.empty((N, max(K // G, 1)), dtype=np.uint16)
    rc = lib().orc_gptq(_p(Wpre), _p(U), _p(Wq), _p(S), N, K, G)
    if rc != 0:
        raise ValueError(f"orc_gptq rejected K={K}, G={G}")
    return Wq, S, Wpre


def dequant_f32(Wq: np.ndarray, S: np.ndarray, G: int = 128) -> np.ndarray:
    """kernels/quant/w4a16.cuh:28-32; bench/bench_w4a16.cu:156-162 (exact fp32)."""
    Wq = np.ascontiguousarray(Wq, dtype=np.uint32)
    S = np.ascontiguousarray(S, dtype=np.uint16)
    N, K = Wq.shape[0], Wq.shape[1] * 8
    out = np.empty((N, K), dtype=np.float32)
    lib().orc_dequant_f32(_p(Wq), _p(S), _p(out), N, K, G)
    return out


def dequant_bf16(Wq: np.ndarray, S: np.ndarray, G: int = 128) -> np.ndarray:
    """kernels/quant/w4a16.cuh:190-198: GEMM staging, bf16_rne((q - 8) * s), uint16 bits."""
    Wq = np.ascontiguousarray(Wq, dtype=np.uint32)
    S = np.ascontiguousarray(S, dtype=np.uint16)
    N, K = Wq.shape[0], Wq.shape[1] * 8
    out = np.empty((N, K), dtype=np.uint16)
    lib().orc_dequant_bf16(_p(Wq), _p(S), _p(out), N, K, G)
    return out


def linear_f64(X: np.ndarray, Wq: np.ndarray, S: np.ndarray, G: int = 128,
               bf16_weights: bool = False) -> np.ndarray:
    """bench/bench_w4a16.cu:163-173: Y = X @ deq(Wq, S)^T accumulated in double.
    X: uint16 bf16 bits [M, K]. Returns float64 [M, N]."""
    X = np.ascontiguousarray(X, dtype=np.uint16)
    Wq = np.ascontiguousarray(Wq, dtype=np.uint32)
    S = np.ascontiguousarray(S, dtype=np.uint16)
    M, K = X.shape
    N = Wq.shape[0]
    assert Wq.shape[1] * 8 == K
    Y = np.empty((M, N), dtype=np.float64)
    lib().orc_linear_w4_f64(_p(X), _p(Wq), _p(S), _p(Y), M, N, K, G, int(bf16_weights))
    return Y


def linear_dense_f64(X: np.ndarray, Wd: np.ndarray) -> np.ndarray:
    """bench/bench_w4a16.cu:163-173 on an explicit fp32 weight matrix Wd [N, K]."""
    X = np.ascontiguousarray(X, dtype=np.uint16)
    Wd = np.ascontiguousarray(Wd, dtype=np.float32)
    M, K = X.shape
    N = Wd.shape[0]
    Y = np.empty((M, N), dtype=np.float64)
    lib().orc_linear_f64(_p(X), _p(Wd), _p(Y), M, N, K)
    return Y


def gemv_ref_order(X: np.ndarray, Wq: np.ndarray, S: np.ndarray, G: int = 128) -> np.ndarray:
    """kernels/quant/w4a16.cuh:42-95 (R = 1, fp32 out): the reference GEMV's exact fp32
    rounding sequence."""
    X = np.ascontiguousarray(X, dtype=np.uint16)
    Wq = np.ascontiguousarray(Wq, dtype=np.uint32)
    S = np.ascontiguousarray(S, dtype=np.uint16)
    M, K = X.shape
    N = Wq.shape[0]
    Y = np.empty((M, N), dtype=np.float32)
    lib().orc_gemv_ref_order(_p(X), _p(Wq), _p(S), _p(Y), M, N, K, G)
    return Y


# ----------------------------------------------------------------- reference error metrics
def max_rel_err(a: np.ndarray, ref: np.ndarray) -> float:
    """bench/bench_w4a16.cu:94-103: max |a - ref| / (max |ref| + 1e-6); inf if a is not finite."""
    a = np.asarray(a, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if not np.all(np.isfinite(a)):
        return float("inf")
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - ref)) / (scale + 1e-6))


def rel_fro(a: np.ndarray, ref: np.ndarray) -> float:
    """bench/bench_w4a16.cu:104-111: ||a - ref||_F / ||ref||_F."""
    a = np.asarray(a, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.sqrt(np.sum((a - ref) ** 2) / np.sum(ref ** 2)))


# ----------------------------------------------------------------- PyTorch CPU baseline
def torch_cpu_linear(x, Wq, S, G: int = 128):
    """The PyTorch-CPU restatement of the reference's CPU dequant+matmul loop
    (bench/bench_w4a16.cu:156-173): unpack nibbles low-first from the int32 words, dequantize
    (q - 8) * s in fp32, then an fp32 matmul. Dequantization is part of the work.
    x: bf16 [M, K]; Wq: int32 [N, K/8]; S: bf16 [N, K/G]. Returns fp32 [M, N]."""
    import torch

    N = Wq.shape[0]
    K = Wq.shape[1] * 8
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    q = (Wq.unsqueeze(-1) >> shifts) & 0xF                         # [N, K/8, 8], low nibble first
    w = (q.reshape(N, K).to(torch.float32) - 8.0)
    w = w.view(N, K // G, G) * S.to(torch.float32).unsqueeze(-1)
    return x.to(torch.float32) @ w.view(N, K).t()


# ----------------------------------------------------------------- packed tile format
def pack_word_nibbles(w: np.ndarray) -> np.ndarray:
    """Element e of a natural-order word (nibble e) -> nibble position e//2 + 4*(e%2): the
    packed order e0 e2 e4 e6 e1 e3 e5 e7 of ns_w4_repack (include/nanoserve_w4.h)."""
    w = np.asarray(w, dtype=np.uint32)
    out = np.zeros_like(w)
    for e in range(8):
        p = e // 2 + 4 * (e % 2)
        out |= ((w >> np.uint32(4 * e)) & np.uint32(0xF)) << np.uint32(4 * p)
    return out


def unpack_word_nibbles(w: np.ndarray) -> np.ndarray:
    """Inverse of pack_word_nibbles."""
    w = np.asarray(w, dtype=np.uint32)
    out = np.zeros_like(w)
    for e in range(8):
        p = e // 2 + 4 * (e % 2)
        out |= ((w >> np.uint32(4 * p)) & np.uint32(0xF)) << np.uint32(4 * e)
    return out


def repack_tiles(Wq: np.ndarray, S: np.ndarray):
    """The packed tile format of ns_w4_repack, restated with numpy (G = 128): tile (t, c) =
    rows 16t..16t+15 x k 128c..128c+127; within a tile, lane l = 16 kg + j holds four words
    s = 0..3 of row 16t + j at word index 16c + 4s + kg of the row; tiles t-major; rows past N
    are zero. Returns (Wp uint32 [NT*C*256], Sp uint16 [NT*C*16])."""
    Wq = np.asarray(Wq, dtype=np.uint32)
    S = np.asarray(S, dtype=np.uint16)
    N, KW = Wq.shape
    C = KW // 16
    NT = (N + 15) // 16
    Wpad = np.zeros((NT * 16, KW), dtype=np.uint32)
    Wpad[:N] = Wq
    Spad = np.zeros((NT * 16, C), dtype=np.uint16)
    Spad[:N] = S
    tiles = Wpad.reshape(NT, 16, C, 4, 4).transpose(0, 2, 4, 1, 3)  # [t][c][kg][j][s]
    Wp = pack_word_nibbles(tiles.reshape(-1))
    Sp = Spad.reshape(NT, 16, C).transpose(0, 2, 1).reshape(-1)
    return np.ascontiguousarray(Wp), np.ascontiguousarray(Sp)
