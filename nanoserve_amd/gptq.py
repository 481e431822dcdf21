"""Calibrated W4 quantization (GPTQ) into the reference's W4 format.

The reference quantizes weights by symmetric round to nearest only (``Kernels.w4_quantize``,
python/nanoserve/ops.py:76-83, kernel kernels/quant/w4a16.cuh:272-297) and names calibrated
methods as its next step (README.md:233-235). GPTQ (Frantar et al., "GPTQ: Accurate Post-Training
Quantization for Generative Pre-trained Transformers", 2022) chooses the same codes and scales
format but quantizes the columns of each row one after another, pushing each column's rounding
error onto the columns not yet quantized through the inverse Hessian of the layer's
reconstruction error ``||(W - W_q) X^T||^2`` over calibration activations X.

Split of the work:
  * ``hessian`` and ``hessian_factor`` (library calls: one GEMM, two Cholesky factorisations and
    a triangular inverse, in float64) produce U, the upper Cholesky factor of the damped inverse
    Hessian;
  * ``Kernels.w4_gptq`` (HIP, ns_w4_gptq) runs the sequential quantize-and-propagate loop and the
    rank-128 updates between groups, and writes (Wq, S) in ``w4_quantize``'s format, so every
    consumer of that format (``w4_linear``, ``w4_repack``, the decode runner) reads it unchanged.
"""
from __future__ import annotations

import torch

from .ops import Kernels

DEFAULT_DAMP = 0.01  # fraction of the mean Hessian diagonal added to the diagonal (GPTQ's 1%)


def hessian(X: torch.Tensor) -> torch.Tensor:
    """H = 2 X^T X / T (float64) of calibration activations X [..., K] (T rows after flattening):
    the Hessian of the layer's squared reconstruction error in its weights."""
    X = X.reshape(-1, X.shape[-1]).to(torch.float64)
    if X.shape[0] == 0:
        raise ValueError("no calibration rows")
    return (2.0 / X.shape[0]) * (X.t() @ X)


def hessian_factor(H: torch.Tensor, damp: float = DEFAULT_DAMP):
    """(U, dead) for a Hessian H [K, K]: input columns whose diagonal is zero (never active in
    the calibration data) get diagonal 1 and are reported in ``dead`` (bool [K]); then
    damp * mean(diag H) is added to the diagonal and U (float32 [K, K], upper triangular) is the
    Cholesky factor with U^T U = H^-1."""
    if H.ndim != 2 or H.shape[0] != H.shape[1]:
        raise ValueError(f"H must be square, got {tuple(H.shape)}")
    if damp <= 0:
        raise ValueError("damp must be positive")
    H = H.to(torch.float64).clone()
    diag = H.diagonal()
    dead = diag == 0
    diag[dead] = 1.0
    diag += damp * diag.mean()
    L = torch.linalg.cholesky(H)
    Hinv = torch.cholesky_inverse(L)
    U = torch.linalg.cholesky(Hinv, upper=True)
    return U.to(torch.float32).contiguous(), dead


def quantize_layer(kernels: Kernels, W: torch.Tensor, X: torch.Tensor | None = None,
                   H: torch.Tensor | None = None, group: int = 128, damp: float = DEFAULT_DAMP):
    """GPTQ-quantize one linear layer's weights W [N, K] (GPU tensor) for calibration activations
    X [..., K] of its input (or a precomputed Hessian H [K, K]) -> (Wq int32 [N, K // 8],
    S bf16 [N, K // group]), the format of ``Kernels.w4_quantize``. Weights of dead input
    columns are zeroed first (their products are zero on the calibration data)."""
    if (X is None) == (H is None):
        raise ValueError("pass exactly one of X and H")
    if H is None:
        H = hessian(X.to(W.device))
    U, dead = hessian_factor(H.to(W.device), damp)
    Wf = W.to(torch.float32).clone()
    Wf[:, dead] = 0.0
    return kernels.w4_gptq(Wf, U, group)
