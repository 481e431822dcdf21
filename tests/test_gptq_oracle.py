"""CPU checks that pin the GPTQ restatement (orc_gptq in oracle/w4_oracle.c, the checker of
ns_w4_gptq) and the host-side Hessian factor (nanoserve_amd/gptq.py), independently of the
restatement itself:

  * with a diagonal factor the algorithm must reduce to the round-to-nearest quantizer,
    bit for bit (orc_quantize, itself pinned against the reference's golden vectors);
  * the optimal-brain-quantizer formulation (OBQ: Frantar & Alistarh 2022, the form GPTQ is
    derived from), which never forms a Cholesky factor: after quantizing column i, every later
    column moves by -(w_i - q_i) / Hinv[i, i] * Hinv[i, :], and Hinv is downdated by the
    Gaussian elimination of row and column i. Computed here in float64; the restatement must
    agree with it, and each plausible mistake planted in a float64 copy of the restatement
    (transposed factor, dropped division, flipped sign, scales fixed before the updates) must
    disagree;
  * the published effect: on correlated calibration data GPTQ lowers the layer's reconstruction
    error ||(W - W_q) X^T|| well below round to nearest.
"""
import numpy as np
import pytest
import torch

from nanoserve_amd import gptq as gq
from oracle import w4_oracle as O


def _bf16_vals(a):
    return O.bf16_to_f32(O.f32_to_bf16(np.asarray(a, np.float32)))


def _calib(T, K, seed, outliers=4):
    """Calibration-like activations: correlated channels (a rank-32 component plus noise, as
    transformer activations are), per-channel scales spread over a decade, a few outlier
    channels."""
    rng = np.random.default_rng(seed)
    Z = rng.standard_normal((T, 32)) @ rng.standard_normal((32, K)) / np.sqrt(32.0)
    Z = Z + 0.3 * rng.standard_normal((T, K))
    scale = np.exp(rng.uniform(np.log(0.3), np.log(3.0), K))
    scale[rng.choice(K, outliers, replace=False)] *= 8.0
    return (Z * scale).astype(np.float32)


def _factor(X, damp=0.01):
    U, dead = gq.hessian_factor(gq.hessian(torch.from_numpy(X)), damp)
    return U.numpy(), dead.numpy()


def _codes(Wq):
    """Wq [N, K/8] uint32 -> codes [N, K] (k = 8j + i in bits 4i of word j)."""
    Wq = np.asarray(Wq, np.uint32)
    sh = (4 * np.arange(8, dtype=np.uint32))[None, None, :]
    return ((Wq[:, :, None] >> sh) & np.uint32(15)).reshape(Wq.shape[0], -1).astype(np.int64)


def _obq_f64(W, H, G, damp=0.01):
    """OBQ in float64, natural order, the scale rule of orc_quantize fixed at each group's start.
    Returns (codes [N, K], scales bf16 bits [N, K/G], values at quantization time [N, K])."""
    W = np.array(W, np.float64)
    N, K = W.shape
    H = np.array(H, np.float64)
    d = np.diag(H).copy()
    H[np.arange(K), np.arange(K)] += damp * d.mean()
    Hinv = np.linalg.inv(H)
    codes = np.zeros((N, K), np.int64)
    scales = np.zeros((N, K // G), np.uint16)
    pre = np.zeros((N, K))
    for i in range(K):
        if i % G == 0:
            mx = np.abs(W[:, i:i + G]).max(axis=1).astype(np.float32)
            sb = O.f32_to_bf16(np.where(mx > 0, mx / np.float32(7), np.float32(1)).astype(np.float32))
            scales[:, i // G] = sb
            sf = O.bf16_to_f32(sb).astype(np.float64)
        pre[:, i] = W[:, i]
        q = np.clip(np.rint(W[:, i] / sf) + 8, 0, 15)
        codes[:, i] = q
        err = (W[:, i] - (q - 8) * sf) / Hinv[i, i]
        W[:, i + 1:] -= np.outer(err, Hinv[i, i + 1:])
        Hinv = Hinv - np.outer(Hinv[:, i], Hinv[i, :]) / Hinv[i, i]
    return codes, scales, pre


def _gptq_f64(W, U, G, mistake=None):
    """The restatement's algorithm in float64, with an optional planted mistake."""
    W = np.array(W, np.float64)
    U = np.array(U, np.float64)
    if mistake == "transposed":
        U = U.T.copy()
    N, K = W.shape
    W0 = W.copy()
    codes = np.zeros((N, K), np.int64)
    scales = np.zeros((N, K // G), np.uint16)
    pre = np.zeros((N, K))
    for i in range(K):
        if i % G == 0:
            src = W0 if mistake == "static_scales" else W
            mx = np.abs(src[:, i:i + G]).max(axis=1).astype(np.float32)
            sb = O.f32_to_bf16(np.where(mx > 0, mx / np.float32(7), np.float32(1)).astype(np.float32))
            scales[:, i // G] = sb
            sf = O.bf16_to_f32(sb).astype(np.float64)
        pre[:, i] = W[:, i]
        q = np.clip(np.rint(W[:, i] / sf) + 8, 0, 15)
        codes[:, i] = q
        err = W[:, i] - (q - 8) * sf
        if mistake != "no_diag_division":
            err = err / U[i, i]
        if mistake == "flipped_sign":
            err = -err
        W[:, i + 1:] -= np.outer(err, U[i, i + 1:])
    return codes, scales, pre


def _agreement(a, b):
    """(fraction of equal codes, fraction of rows whose codes all agree)."""
    eq = a == b
    return eq.mean(), eq.all(axis=1).mean()


def _assert_same_run(got, ref, G, rtol, tie, min_rows=0.75):
    """Two runs of the algorithm agree: in every row, up to the first column whose code or group
    scale differs, the values at quantization time agree to rtol (relative to the row's largest),
    and that first difference sits at a rounding tie of the reference run (|w / s| within `tie`
    of a half-integer, or max|w| / 7 within `tie` of a bf16 rounding boundary), where the
    arithmetic of the two runs may legitimately round differently. At least min_rows of the rows
    agree completely."""
    codes, S, pre = got
    codes_o, S_o, pre_o = ref
    N, K = codes.shape
    full = 0
    for r in range(N):
        scale_bad = np.repeat(S[r] != S_o[r], G)
        bad = np.flatnonzero((codes[r] != codes_o[r]) | scale_bad)
        c = bad[0] if bad.size else K
        lim = rtol * np.abs(pre_o[r]).max()
        assert np.abs(pre[r, :c] - pre_o[r, :c]).max(initial=0.0) <= lim, (r, c)
        if c == K:
            full += 1
            continue
        g = c // G
        if scale_bad[c]:
            m = np.float32(np.abs(pre_o[r, g * G:(g + 1) * G]).max()) / np.float32(7)
            lo = O.bf16_to_f32(O.f32_to_bf16(np.array([m], np.float32)))[0]
            ulp = 2.0 ** (np.floor(np.log2(m)) - 7)
            d = abs(abs(m - lo) - ulp / 2) / ulp
            assert d < tie, (r, c, "scale not at a tie", d)
        else:
            sf = float(O.bf16_to_f32(np.array([S_o[r, g]], np.uint16))[0])
            t = pre_o[r, c] / sf
            assert abs(abs(t - np.floor(t)) - 0.5) < tie, (r, c, "code not at a tie", t)
    assert full >= min_rows * N, (full, N)


def test_diagonal_factor_is_round_to_nearest():
    """U diagonal: no error is propagated, so GPTQ must give orc_quantize's codes and scales
    bit for bit (including an all-zero group, exact .5 ties and clamped values)."""
    rng = np.random.default_rng(0)
    N, K = 37, 512
    W = _bf16_vals(rng.standard_normal((N, K)) * 0.05)
    W[3, 128:256] = 0.0
    W[5, :8] = _bf16_vals(np.array([0.5, -0.5, 1.5, -2.5, 7.0, -8.0, 3.5, -3.5], np.float32))
    W[5, 8] = 7.0  # scale 1: the row above rounds ties to even
    U = np.diag(rng.uniform(0.5, 2.0, K)).astype(np.float32)
    Wq, S, _ = O.gptq(W, U, 128)
    Wq_r, S_r = O.quantize(O.f32_to_bf16(W), 128)
    assert np.array_equal(Wq, Wq_r) and np.array_equal(S, S_r)


@pytest.mark.parametrize("N,K,seed", [(24, 256, 1), (16, 384, 2), (8, 1024, 3)])
def test_restatement_matches_obq_f64(N, K, seed):
    rng = np.random.default_rng(seed)
    X = _calib(4 * K, K, seed)
    W = _bf16_vals(rng.standard_normal((N, K)) * 0.05)
    U, _ = _factor(X)
    Hn = gq.hessian(torch.from_numpy(X)).numpy()
    ref = _obq_f64(W, Hn, 128)
    Wq, S, pre = O.gptq(W, U, 128)
    _assert_same_run((_codes(Wq), S, pre), ref, 128, rtol=2e-4, tie=2e-3)


@pytest.mark.parametrize("mistake", ["transposed", "no_diag_division", "flipped_sign",
                                     "static_scales"])
def test_obq_rejects_planted_mistakes(mistake):
    N, K, seed = 24, 256, 1
    rng = np.random.default_rng(seed)
    X = _calib(4 * K, K, seed)
    W = _bf16_vals(rng.standard_normal((N, K)) * 0.05)
    U, _ = _factor(X)
    Hn = gq.hessian(torch.from_numpy(X)).numpy()
    ref = _obq_f64(W, Hn, 128)
    good = _gptq_f64(W, U, 128)
    _assert_same_run(good, ref, 128, rtol=1e-5, tie=1e-4)
    with pytest.raises(AssertionError):
        _assert_same_run(_gptq_f64(W, U, 128, mistake), ref, 128, rtol=1e-3, tie=1e-2)


def test_restatement_matches_float64_copy():
    """The C restatement (fp32, fused multiply-adds) and its float64 copy differ only where fp32
    rounding flips a code near a tie."""
    N, K, seed = 32, 384, 5
    rng = np.random.default_rng(seed)
    X = _calib(2 * K, K, seed)
    W = _bf16_vals(rng.standard_normal((N, K)) * 0.05)
    U, _ = _factor(X)
    Wq, S, pre = O.gptq(W, U, 128)
    _assert_same_run((_codes(Wq), S, pre), _gptq_f64(W, U, 128), 128, rtol=2e-4, tie=2e-3)


def test_gptq_lowers_reconstruction_error():
    N, K, seed = 64, 512, 7
    rng = np.random.default_rng(seed)
    X = _calib(4 * K, K, seed)
    W = _bf16_vals(rng.standard_normal((N, K)) * 0.05)
    U, _ = _factor(X)
    Wq, S, _ = O.gptq(W, U, 128)
    Wq_r, S_r = O.quantize(O.f32_to_bf16(W), 128)
    Xd = X.astype(np.float64)
    e_g = np.linalg.norm((W - O.dequant_f32(Wq, S, 128)) @ Xd.T)
    e_r = np.linalg.norm((W - O.dequant_f32(Wq_r, S_r, 128)) @ Xd.T)
    assert e_g < 0.5 * e_r, (e_g, e_r)


def test_hessian_factor():
    """U^T U = (H + damp * mean(diag H) I)^-1 with dead columns given diagonal 1 first; U upper."""
    K = 64
    X = _calib(256, K, 3)
    X[:, [5, 40]] = 0.0
    H = gq.hessian(torch.from_numpy(X))
    Hn = 2.0 * X.astype(np.float64).T @ X.astype(np.float64) / X.shape[0]
    np.testing.assert_allclose(H.numpy(), Hn, rtol=1e-10, atol=1e-9)
    U, dead = gq.hessian_factor(H, 0.01)
    assert dead.numpy().tolist() == [i in (5, 40) for i in range(K)]
    Hd = Hn.copy()
    Hd[[5, 40], [5, 40]] = 1.0
    Hd[np.arange(K), np.arange(K)] += 0.01 * np.diag(Hd).mean()
    U = U.numpy().astype(np.float64)
    assert np.array_equal(U, np.triu(U)) and (np.diag(U) > 0).all()
    np.testing.assert_allclose(U.T @ U @ Hd, np.eye(K), atol=2e-4)


def test_hessian_factor_rejects():
    with pytest.raises(ValueError):
        gq.hessian_factor(torch.eye(3)[:2])
    with pytest.raises(ValueError):
        gq.hessian_factor(torch.eye(3), damp=0.0)
    with pytest.raises(ValueError):
        gq.hessian(torch.zeros(0, 8))
