"""GPU parity of the calibrated quantizer ns_w4_gptq (nanoserve_amd/csrc/w4_gptq.hip) against
its CPU restatement orc_gptq (oracle/w4_oracle.c, pinned in tests/test_gptq_oracle.py).

The kernels fix their arithmetic (fp32, one fused multiply-add per update, each weight's updates
in column order, IEEE division), so codes and scales must equal the restatement's bit for bit,
given the same factor U. At full layer sizes the rows are checked on a sample (rows are
independent in the algorithm), and the whole matrix through size-independent properties: a
diagonal factor reproduces ns_w4_quantize exactly, and two runs are identical.
"""
import numpy as np
import pytest
import torch

from nanoserve_amd import Kernels
from nanoserve_amd import gptq as gq
from oracle import w4_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def k():
    return Kernels()


def _calib(T, K, seed):
    """Correlated activations (rank-32 component plus noise), channel scales over a decade."""
    g = torch.Generator().manual_seed(seed)
    Z = torch.randn(T, 32, generator=g) @ torch.randn(32, K, generator=g) / 32 ** 0.5
    Z = Z + 0.3 * torch.randn(T, K, generator=g)
    scale = torch.exp(torch.empty(K).uniform_(np.log(0.3), np.log(3.0), generator=g))
    return Z * scale


def _weights(N, K, seed, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, K, generator=g) * scale).to(torch.bfloat16)


def _np_bits(t):
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy().view(np.uint32)


def _run(k, W, U):
    Wq, S = k.w4_gptq(W.to(DEV), U.to(DEV))
    torch.cuda.synchronize()
    return _np_bits(Wq), _np_bits(S)


@pytest.mark.parametrize("N,K,seed", [(1, 128, 1), (63, 384, 2), (200, 512, 3), (256, 1024, 4),
                                      (130, 256, 5)])
def test_gptq_matches_oracle(k, N, K, seed):
    W = _weights(N, K, seed)
    W[0, 128 * (K // 256):128 * (K // 256) + 128] = 0  # an all-zero group (scale 1)
    X = _calib(2 * K, K, seed)
    X[:, 7] = 0  # a dead input column
    H = gq.hessian(X)
    U, dead = gq.hessian_factor(H)
    Wf = W.float()
    Wf[:, dead] = 0
    Wq, S = _run(k, Wf, U)
    Wq_o, S_o, _ = O.gptq(Wf.numpy(), U.numpy(), 128)
    assert np.array_equal(S, S_o)
    assert np.array_equal(Wq, Wq_o)


@pytest.mark.parametrize("N,K", [(4608, 3584), (100, 256)])
def test_gptq_diagonal_factor_equals_w4_quantize(k, N, K):
    W = _weights(N, K, 11)
    g = torch.Generator().manual_seed(12)
    U = torch.diag(torch.empty(K).uniform_(0.5, 2.0, generator=g))
    Wq, S = _run(k, W, U)
    Wq_r, S_r = k.w4_quantize(W.to(DEV), 128)
    torch.cuda.synchronize()
    assert np.array_equal(Wq, _np_bits(Wq_r)) and np.array_equal(S, _np_bits(S_r))


def test_gptq_full_size_sampled_rows(k):
    """Qwen2.5-7B's up projection shape (18944 x 3584): 24 sampled rows bit-exact against the
    restatement, and a second run identical to the first."""
    N, K = 18944, 3584
    W = _weights(N, K, 21)
    U, _ = gq.hessian_factor(gq.hessian(_calib(1024, K, 22)))
    Wq, S = _run(k, W, U)
    rows = np.random.default_rng(23).choice(N, 24, replace=False)
    rows[0], rows[1] = 0, N - 1
    Wq_o, S_o, _ = O.gptq(W[rows].float().numpy(), U.numpy(), 128)
    assert np.array_equal(S[rows], S_o)
    assert np.array_equal(Wq[rows], Wq_o)
    Wq2, S2 = _run(k, W, U)
    assert np.array_equal(Wq, Wq2) and np.array_equal(S, S2)


def test_gptq_long_rows_sampled(k):
    """Qwen2.5-7B's down projection row length (K = 18944), factor computed on the GPU
    (float64 Cholesky): 6 sampled rows bit-exact against the restatement."""
    N, K = 192, 18944
    W = _weights(N, K, 31)
    U, _ = gq.hessian_factor(gq.hessian(_calib(512, K, 32).to(DEV)))
    Wq, S = _run(k, W, U)
    rows = np.array([0, 5, 64, 100, 150, N - 1])
    Wq_o, S_o, _ = O.gptq(W[rows].float().numpy(), U.cpu().numpy(), 128)
    assert np.array_equal(S[rows], S_o)
    assert np.array_equal(Wq[rows], Wq_o)


def test_quantize_layer_beats_round_to_nearest(k):
    """End to end on the GPU (Hessian, factor, kernels): the layer's output error on the
    calibration data is well below round to nearest's, through ns_w4_linear."""
    N, K, T = 512, 1024, 2048
    W = _weights(N, K, 41).to(DEV)
    X = _calib(T, K, 42).to(DEV)
    Wq, S = gq.quantize_layer(k, W, X=X)
    Wq_r, S_r = k.w4_quantize(W, 128)
    xb = X[:256].to(torch.bfloat16)
    ref = xb.float() @ W.float().t()
    e_g = (k.w4_linear(xb, Wq, S).float() - ref).norm()
    e_r = (k.w4_linear(xb, Wq_r, S_r).float() - ref).norm()
    torch.cuda.synchronize()
    assert e_g < 0.5 * e_r, (float(e_g), float(e_r))


def test_gptq_rejects(k):
    W = torch.zeros(4, 256, device=DEV)
    with pytest.raises(ValueError):
        k.w4_gptq(W, torch.eye(128, device=DEV))
    with pytest.raises(RuntimeError):
        k.w4_gptq(W, torch.eye(256, device=DEV), group=64)
    with pytest.raises(RuntimeError):
        k.w4_gptq(torch.zeros(4, 200, device=DEV), torch.eye(200, device=DEV))
