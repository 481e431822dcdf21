"""Seeded random shapes through ns_w4_linear (M = 1, M = 2..8 and the GEMM, group sizes 32..256),
the packed tile format and the one-token decode GEMV, against the oracle's float64 product: the
planners' choices on shapes nobody picked by hand (odd N, odd chunk counts, N tails, small and
long rows). Shapes are bounded so the oracle finishes each case in well under a second."""
import random

import numpy as np
import pytest
import torch

from nanoserve_amd import synth
from tests.conftest import to_dev, to_host_bits

pytestmark = pytest.mark.gpu


def _cases(n=48, seed=20261202):
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        M = rng.choice([1, 1, 1, 2, 3, 4, 5, 6, 7, 8, 17, 40, 130, 256])
        G = 128 if M > 8 or rng.random() < 0.7 else rng.choice([32, 64, 256])
        K = G * rng.randint(1, max(1, 12288 // G))
        N = rng.choice([rng.randint(1, 64), rng.randint(65, 1500), rng.randint(1500, 9000)])
        if M > 8:
            N = max(128, N // 128 * 128)  # the standard GEMM's contract (N % 128 == 0)
        if M * N * K > 300_000_000 or N * K > 60_000_000:
            continue
        out.append((M, N, K, G))
    return out


CASES = _cases()


def _faithful(y, ref, rel_slack=2e-5):
    """y is bf16(RNE) of a value within rel_slack * ||ref||_inf of ref."""
    bound = np.abs(ref) * 2.0 ** -8 + rel_slack * np.max(np.abs(ref))
    assert np.all(np.abs(y - ref) <= bound), float(np.max(np.abs(y - ref) - bound))


def _host(y):
    return synth.bf16_bits_to_f32(to_host_bits(y)).astype(np.float64)


@pytest.mark.parametrize("M,N,K,G", CASES)
def test_w4_linear_random_shapes(kernels, oracle, M, N, K, G):
    """ns_w4_linear within half a bf16 ulp (+2e-5 ||ref||) of the oracle: the exact dequant for
    M <= 8, the bf16-staged weights of the reference GEMM for M > 8; the packed format (group
    128) on the same inputs for M >= 2."""
    print(f"random shape M={M} N={N} K={K} G={G}", flush=True)
    Wq, S = synth.weights(N, K, G, seed=N * 7 + K + M)
    X = synth.activations(M, K, seed=M * 13 + N, per_row_seed=True)
    xd, wd, sd = to_dev(X, torch.bfloat16), to_dev(Wq, torch.int32), to_dev(S, torch.bfloat16)
    y = kernels.w4_linear(xd, wd, sd, G)
    torch.cuda.synchronize()
    staged = M > 8
    _faithful(_host(y), oracle.linear_f64(X, Wq, S, G, bf16_weights=staged))
    if M >= 2 and G == 128 and K <= 20480:
        wp, sp = kernels.w4_repack(wd, sd)
        yp = kernels.w4_linear_packed(xd, wp, sp, N)
        torch.cuda.synchronize()
        _faithful(_host(yp), oracle.linear_f64(X, Wq, S, G, bf16_weights=M > 16))


@pytest.mark.parametrize("M,N,K,G", [c for c in CASES if c[0] == 1 and c[3] == 128 and c[2] <= 16384])
def test_gemv_decode_random_shapes(kernels, oracle, M, N, K, G):
    """The one-token decode GEMV entry (plain activation) on the same M = 1 shapes: the same
    layout as ns_w4_linear, so the same bits."""
    Wq, S = synth.weights(N, K, G, seed=N * 7 + K + M)
    X = synth.activations(1, K, seed=M * 13 + N)
    xd, wd, sd = to_dev(X, torch.bfloat16), to_dev(Wq, torch.int32), to_dev(S, torch.bfloat16)
    y = kernels.w4_linear(xd, wd, sd, G)
    yd = kernels.gemv_decode(wd, sd, G, x=xd.reshape(-1))
    torch.cuda.synchronize()
    assert torch.equal(y.reshape(-1), yd.reshape(-1))
    _faithful(_host(yd).reshape(1, -1), oracle.linear_f64(X, Wq, S, G))


def _decode_cases(n=16, seed=7):
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        K = 128 * rng.choice([1, 2, 3, 7, 8, 12, 14, 20, 28, 40, 56, 64, 100, 128])
        N = 16 * rng.randint(1, rng.choice([8, 200, 2500]))
        if N * K > 60_000_000:
            continue
        out.append((N, K, rng.choice(["norm_add", "swiglu_norm"])))
    return out


@pytest.mark.parametrize("N,K,mode", _decode_cases())
def test_gemv_decode_fused_random_shapes(kernels, N, K, mode):
    """The fused decode GEMV (add + RMSNorm in; SwiGLU out for gate/up rows interleaved in
    blocks of 8) on random shapes: the new residual stream bit-exact against the oracle, the
    output against the oracle-normalised activation's float64 product
    and, for K <= 8192, against the unfused kernels (ns_rmsnorm, ns_w4_linear, ns_swiglu) to one
    bf16 ulp."""
    from oracle import decode_ref as R
    from oracle import w4_oracle as O

    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(N + K)
    Wd = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    Wq, S = kernels.w4_quantize(Wd, 128)
    del Wd
    res = (torch.randn(K, generator=g) * 3.0).to(torch.bfloat16).to(dev)
    r = torch.randn(K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(K, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    res_out = torch.empty(K, dtype=torch.bfloat16, device=dev)
    sw = mode == "swiglu_norm"
    y = kernels.gemv_decode(Wq, S, 128, res=res, r=r, norm_w=w, eps=1e-6, res_out=res_out,
                            swiglu=sw)
    torch.cuda.synchronize()
    v_ref, h_ref = R.rmsnorm(res.reshape(1, -1), r.reshape(1, -1), w, 1e-6)
    assert torch.equal(res_out.double().cpu(), v_ref.reshape(-1))
    hb = R.bf16_round(h_ref).to(torch.bfloat16).reshape(1, -1)
    ref = torch.from_numpy(O.linear_f64(hb.view(torch.int16).numpy().view("uint16"),
                                        Wq.cpu().numpy().view("uint32"),
                                        S.cpu().view(torch.int16).numpy().view("uint16"), 128))
    if sw:
        g4 = ref.view(N // 16, 2, 8)
        gate, up = R.bf16_round(g4[:, 0].reshape(-1)), R.bf16_round(g4[:, 1].reshape(-1))
        ref = (gate / (1.0 + torch.exp(-gate)) * up).reshape(1, -1)
    err = (y.double().cpu() - ref).abs().max().item()
    assert err <= 1e-2 * ref.abs().max().item(), err
    if K <= 8192:  # ns_rmsnorm's own limit (the reference's: H <= 8192)
        h = kernels.rmsnorm(res.clone().reshape(1, -1), r.reshape(1, -1), w, 1e-6)
        gu = kernels.w4_linear(h, Wq, S, 128)
        if sw:
            u4 = gu.view(N // 16, 2, 8)
            gu = kernels.swiglu(u4[:, 0].reshape(1, -1).contiguous(),
                                u4[:, 1].reshape(1, -1).contiguous())
        torch.cuda.synchronize()
        torch.testing.assert_close(y.double().cpu(), gu.double().cpu(), rtol=2 ** -7,
                                   atol=1e-3 * gu.abs().max().item())
