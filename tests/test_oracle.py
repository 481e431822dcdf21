"""Pins the CPU oracle (oracle/w4_oracle.c) against what fixes it independently:

* the reference's own recorded outputs for its correctness case (N=256, K=512, hash-filled
  inputs seeds 11/12): quantization error 7.05% (README.md:154, results/ncu/w4_gemv_m8.txt:11),
  GEMV max-rel-err 5.8e-08 (M=1) and 1.1e-07 (M=8), GEMM 2.2e-03 (w4_gemv_m8.txt:7-10);
* closed forms of the weight format (kernels/quant/w4a16.cuh:5-9), exhaustively;
* library routines: torch's bf16 rounding, numpy float64 matmul;
* invariants of the quantizer (w4a16.cuh:272-297).
"""
import numpy as np
import pytest
import torch

from nanoserve_amd import synth


# ----------------------------------------------------------------- reference known answers
@pytest.fixture(scope="module")
def ref_case(oracle):
    N, K, G, Mmax = 256, 512, 128, 128
    W = oracle.hash_fill(N * K, 11, 0.05).reshape(N, K)          # bench_w4a16.cu:143, 63
    X = oracle.hash_fill(Mmax * K, 12, 1.0).reshape(Mmax, K)     # bench_w4a16.cu:148
    Wq, S = oracle.quantize(W, G)                                # bench_w4a16.cu:64
    ref = oracle.linear_f64(X, Wq, S, G).astype(np.float32)      # bench_w4a16.cu:163-173
    return dict(N=N, K=K, G=G, W=W, X=X, Wq=Wq, S=S, ref=ref)


def test_kat_quantization_error_7_05(oracle, ref_case):
    c = ref_case
    y_bf16 = oracle.linear_dense_f64(c["X"], oracle.bf16_to_f32(c["W"]))
    err = 100 * oracle.rel_fro(c["ref"], y_bf16)
    assert f"{err:.2f}" == "7.05", err


@pytest.mark.parametrize("M,expected", [(1, "5.8e-08"), (8, "1.1e-07")])
def test_kat_reference_gemv_error(oracle, ref_case, M, expected):
    c = ref_case
    y = oracle.gemv_ref_order(c["X"][:M], c["Wq"], c["S"], c["G"])
    assert f"{oracle.max_rel_err(y, c['ref'][:M]):.1e}" == expected


def test_kat_reference_gemm_bf16_staging_error(oracle, ref_case):
    c = ref_case
    y = oracle.linear_f64(c["X"], c["Wq"], c["S"], c["G"], bf16_weights=True).astype(np.float32)
    assert f"{oracle.max_rel_err(y, c['ref']):.1e}" == "2.2e-03"


# ----------------------------------------------------------------- format closed forms
def test_nibble_order_exhaustive(oracle):
    """Every (position i, value q): k = 8j + i lives in bits 4i..4i+3 (w4a16.cuh:6-8)."""
    G = 32
    N, K = 16 * 8, 32
    Wq = np.full((N, K // 8), 0x88888888, dtype=np.uint32)       # q = 8 -> weight 0 elsewhere
    S = np.full((N, 1), 0x3F80, dtype=np.uint16)                 # scale 1.0
    for q in range(16):
        for i in range(8):
            n = q * 8 + i
            Wq[n, 1] = (0x88888888 & ~(0xF << (4 * i))) | (q << (4 * i))
    Wd = oracle.dequant_f32(Wq, S, G)
    for q in range(16):
        for i in range(8):
            row = Wd[q * 8 + i]
            expect = np.zeros(K, dtype=np.float32)
            expect[8 + i] = q - 8
            np.testing.assert_array_equal(row, expect)


def test_dequant_is_exact_product(oracle):
    Wq, S = synth.weights(64, 512, 128, seed=3)
    Wd = oracle.dequant_f32(Wq, S, 128).astype(np.float64)
    q = ((Wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(64, 512)
    s = synth.bf16_bits_to_f32(S).astype(np.float64)
    exact = (q.astype(np.float64) - 8.0) * np.repeat(s, 128, axis=1)
    np.testing.assert_array_equal(Wd, exact)


def test_bf16_rne_matches_torch(oracle):
    rng = np.random.default_rng(5)
    f = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 65504.0, 3.0e38, -3.0e38, 1e-40,
                  -1e-45, np.inf, -np.inf], dtype=np.float32),
        # exact ties: low 16 bits 0x8000 with even and odd bf16 lsb
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ]).astype(np.float32)
    ours = oracle.f32_to_bf16(f)
    theirs = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)
    np.testing.assert_array_equal(synth.bf16_rne_bits(f[np.isfinite(f)]), theirs[np.isfinite(f)])


def test_gemm_staging_is_rne_of_exact(oracle):
    Wq, S = synth.weights(32, 1024, 128, seed=9)
    staged = oracle.dequant_bf16(Wq, S, 128)
    exact = oracle.dequant_f32(Wq, S, 128)
    theirs = torch.from_numpy(exact).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(staged, theirs)
    # the staging really rounds: some (q - 8) * s need more than 8 significant bits
    assert np.any(oracle.bf16_to_f32(staged) != exact)


# ----------------------------------------------------------------- accumulation
@pytest.mark.parametrize("M,N,K,G", [(1, 64, 256, 128), (3, 33, 96, 32), (8, 16, 1024, 256)])
def test_linear_matches_numpy_f64(oracle, M, N, K, G):
    Wq, S = synth.weights(N, K, G, seed=M + N)
    X = synth.activations(M, K, seed=K)
    Wd = oracle.dequant_f32(Wq, S, G).astype(np.float64)
    ref = synth.bf16_bits_to_f32(X).astype(np.float64) @ Wd.T
    got = oracle.linear_f64(X, Wq, S, G)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.linear_dense_f64(X, Wd.astype(np.float32)), ref,
                               rtol=1e-12, atol=1e-12)


def test_torch_cpu_baseline_matches_oracle(oracle):
    M, N, K, G = 4, 96, 512, 128
    Wq, S = synth.weights(N, K, G, seed=4)
    X = synth.activations(M, K, seed=6)
    x = torch.from_numpy(X.view(np.int16).copy()).view(torch.bfloat16)
    wq = torch.from_numpy(Wq.view(np.int32).copy())
    s = torch.from_numpy(S.view(np.int16).copy()).view(torch.bfloat16)
    y = oracle.torch_cpu_linear(x, wq, s, G).numpy()
    assert oracle.max_rel_err(y, oracle.linear_f64(X, Wq, S, G)) < 1e-5


# ----------------------------------------------------------------- quantizer invariants
def test_quantizer_invariants(oracle):
    W = oracle.hash_fill(64 * 512, 77, 0.3).reshape(64, 512)
    Wq, S = oracle.quantize(W, 128)
    w = oracle.bf16_to_f32(W).reshape(64, 4, 128)
    s = oracle.bf16_to_f32(S)
    mx = np.abs(w).max(axis=2)
    np.testing.assert_array_equal(S, oracle.f32_to_bf16((mx / np.float32(7)).astype(np.float32)))
    q = ((Wq[:, :, None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(64, 4, 128)
    expect = np.clip(np.rint(w / s[:, :, None]).astype(np.int64) + 8, 0, 15)
    np.testing.assert_array_equal(q, expect)
    deq = (q.astype(np.float64) - 8) * s[:, :, None]
    unclipped = (expect > 0) & (expect < 15)
    assert np.all(np.abs(deq - w)[unclipped] <= 0.5 * np.broadcast_to(s[:, :, None], w.shape)[unclipped] * (1 + 1e-6))


def test_quantizer_special_groups(oracle):
    K, G = 64, 32
    W = np.zeros((4, K), dtype=np.float32)
    W[1, 5] = -3.0                        # single nonzero: q = 1 there (-7 * s), 8 elsewhere
    W[2, :32] = np.linspace(-1, 1, 32)    # ties and both signs
    W[3, 32:] = 1e-39                     # fp32-subnormal magnitudes
    Wb = oracle.f32_to_bf16(W)
    Wq, S = oracle.quantize(Wb, G)
    assert S[0, 0] == 0x3F80 and S[0, 1] == 0x3F80          # all-zero group -> scale 1.0
    assert Wq[0, 0] == 0x88888888
    assert ((Wq[1, 0] >> 20) & 0xF) == 1
    with pytest.raises(ValueError):
        oracle.quantize(Wb, 48)                                # G % 32 != 0 -> rejected


# ----------------------------------------------------------------- packed tile format
def test_pack_word_nibbles_closed_form():
    # nibbles 0..7 in natural order -> positions 0,4,1,5,2,6,3,7: 0x75316420
    from oracle.w4_oracle import pack_word_nibbles, unpack_word_nibbles
    w = np.array([0x76543210], dtype=np.uint32)
    assert pack_word_nibbles(w)[0] == 0x75316420
    # (packed >> 4i) & 0x000F000F holds elements 2i and 2i+1 in its two halves
    p = int(pack_word_nibbles(w)[0])
    for i in range(4):
        v = (p >> (4 * i)) & 0x000F000F
        assert (v & 0xF, v >> 16) == (2 * i, 2 * i + 1)
    rng = np.random.default_rng(5)
    r = rng.integers(0, 2 ** 32, size=1000, dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(unpack_word_nibbles(pack_word_nibbles(r)), r)


def test_repack_tiles_places_every_word_once():
    from oracle.w4_oracle import repack_tiles, unpack_word_nibbles
    N, K = 40, 384  # N not a multiple of 16
    rng = np.random.default_rng(6)
    Wq = rng.integers(0, 2 ** 32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    S = rng.integers(0, 2 ** 16, size=(N, K // 128), dtype=np.uint64).astype(np.uint16)
    Wp, Sp = repack_tiles(Wq, S)
    C, NT = K // 128, (N + 15) // 16
    assert Wp.size == NT * C * 256 and Sp.size == NT * C * 16
    words = unpack_word_nibbles(Wp).reshape(NT, C, 64, 4)
    for t in range(NT):
        for c in range(C):
            for lane in range(64):
                j, kg = lane % 16, lane // 16
                row = 16 * t + j
                for s in range(4):
                    want = Wq[row, 16 * c + 4 * s + kg] if row < N else 0
                    assert words[t, c, lane, s] == want
                if s == 3 and lane < 16:
                    assert Sp[(t * C + c) * 16 + j] == (S[row, c] if row < N else 0)
