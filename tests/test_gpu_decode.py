"""GPU parity of the decoder-step kernels (nanoserve_amd/csrc/decode_ops.hip) against the CPU
oracle (oracle/decode_ref.py, pinned in tests/test_decode_oracle.py), and of the W4A16 Qwen2
runner (nanoserve_amd/qwen.py) against Hugging Face transformers' Qwen2ForCausalLM evaluated
in float32 on the CPU with the same (dequantized) weights.

Tolerances, all stated against a float64 / float32 reference:
  * bit-exact: residual-stream adds, bias adds, cache rows not written, v rows;
  * bf16 outputs of fp32 arithmetic: rtol 2^-8 (half a bf16 ulp of rounding plus fp32 error)
    with a small absolute floor;
  * the whole runner: max |logits - ref| <= 3e-2 * max |ref| and cosine similarity >= 0.999
    (bf16 activations between kernels, as the reference's runner; measured bf16-vs-fp32 gap
    of the same models on the CPU: about 1e-2 * max |ref|);
  * a replayed HIP graph equals the eager step bit for bit.
"""
import copy
import dataclasses

import pytest
import torch

from nanoserve_amd import Kernels
from nanoserve_amd.qwen import Qwen2Runner, Qwen2Shape
from oracle import decode_ref as R
from oracle import w4_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def k():
    return Kernels()


def rnd(*shape, seed, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype).to(DEV)


def close(out, ref, rtol=2 ** -8, atol=1e-6):
    torch.testing.assert_close(out.detach().double().cpu(), ref.double().cpu(), rtol=rtol,
                               atol=atol)


# ------------------------------------------------------------------ ns_rmsnorm
@pytest.mark.parametrize("T,H", [(1, 3584), (4, 896), (33, 8), (2, 8192), (3, 4096)])
@pytest.mark.parametrize("with_r", [False, True])
def test_rmsnorm(k, T, H, with_r):
    print(f"rmsnorm T={T} H={H} r={with_r}", flush=True)
    x, r, w = rnd(T, H, seed=1, scale=3.0), rnd(T, H, seed=2), rnd(H, seed=3, scale=0.5)
    x0 = x.clone()
    y = k.rmsnorm(x, r if with_r else None, w, 1e-6)
    torch.cuda.synchronize()
    v_ref, y_ref = R.rmsnorm(x0, r if with_r else None, w, 1e-6)
    assert torch.equal(x.double().cpu(), v_ref)  # residual stream: bit-exact
    close(y, y_ref)


def test_rmsnorm_rejects(k):
    x = torch.empty(2, 12, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError):
        k.rmsnorm(x, None, torch.empty(12, dtype=torch.bfloat16, device=DEV), 1e-6)


# ------------------------------------------------------------------ ns_rope
@pytest.mark.parametrize("T", [1, 5])
@pytest.mark.parametrize("pos0", [0, 1023, 32000])
def test_rope_in_fused_buffer(k, T, pos0):
    print(f"rope T={T} pos0={pos0}", flush=True)
    Hq, Hk, D = 28, 4, 128
    qn, kn = Hq * D, Hk * D
    qkv = rnd(T, qn + 2 * kn, seed=4, scale=2.0)
    ref_in = qkv.clone()
    freq = R.inv_freq(D, 1000000.0)
    k.rope(qkv[:, :qn], qkv[:, qn:qn + kn], freq.to(DEV), Hq, Hk, D, pos0)
    torch.cuda.synchronize()
    pos = torch.arange(pos0, pos0 + T)
    q_ref = R.rope(ref_in[:, :qn], Hq, D, pos, freq)
    k_ref = R.rope(ref_in[:, qn:qn + kn], Hk, D, pos, freq)
    close(qkv[:, :qn], q_ref, atol=1e-4)
    close(qkv[:, qn:qn + kn], k_ref, atol=1e-4)
    assert torch.equal(qkv[:, qn + kn:], ref_in[:, qn + kn:])  # v untouched


# ------------------------------------------------------------------ ns_swiglu
@pytest.mark.parametrize("T,I", [(1, 18944), (3, 1024), (1, 8), (7, 264)])
def test_swiglu(k, T, I):
    print(f"swiglu T={T} I={I}", flush=True)
    g, u = rnd(T, I, seed=5, scale=4.0), rnd(T, I, seed=6)
    out = k.swiglu(g, u)
    torch.cuda.synchronize()
    close(out, R.swiglu(g, u), atol=1e-6)


# ------------------------------------------------------------------ ns_decode_qkv
@pytest.mark.parametrize("pos", [0, 17, 63, 64, -1])
@pytest.mark.parametrize("with_bias", [True, False])
def test_decode_qkv(k, pos, with_bias):
    print(f"decode_qkv pos={pos} bias={with_bias}", flush=True)
    Hq, Hk, D, max_len = 28, 4, 128, 64
    qn, kn = Hq * D, Hk * D
    qkv = rnd(qn + 2 * kn, seed=7, scale=2.0)
    bias = rnd(qn + 2 * kn, seed=8, scale=0.5) if with_bias else None
    kc, vc = rnd(Hk, max_len, D, seed=9), rnd(Hk, max_len, D, seed=10)
    qkv0, kc0, vc0 = qkv.clone(), kc.clone(), vc.clone()
    freq = R.inv_freq(D, 1000000.0)
    p = torch.tensor([pos], dtype=torch.int32, device=DEV)
    k.decode_qkv(qkv, bias, freq.to(DEV), p, kc, vc, Hq, Hk, D)
    torch.cuda.synchronize()
    q_ref, k_ref, v_ref = R.decode_qkv(qkv0, bias, Hq, Hk, D, pos, freq)
    close(qkv[:qn], q_ref.reshape(-1), rtol=2 ** -7, atol=1e-4)
    close(qkv[qn:qn + kn], k_ref.reshape(-1), rtol=2 ** -7, atol=1e-4)
    assert torch.equal(qkv[qn + kn:].double().cpu(), v_ref.reshape(-1))
    written = 0 <= pos < max_len
    rows = torch.ones(max_len, dtype=torch.bool)
    if written:
        rows[pos] = False
        assert torch.equal(kc[:, pos].reshape(-1), qkv[qn:qn + kn])
        assert torch.equal(vc[:, pos].reshape(-1), qkv[qn + kn:])
    assert torch.equal(kc[:, rows.to(DEV)], kc0[:, rows.to(DEV)])  # other rows untouched
    assert torch.equal(vc[:, rows.to(DEV)], vc0[:, rows.to(DEV)])


# ------------------------------------------------------------------ ns_decode_attention
@pytest.mark.parametrize("Hq,Hk", [(28, 4), (7, 1), (4, 4), (8, 1), (16, 4)])
@pytest.mark.parametrize("max_len,n", [(64, 1), (64, 64), (1024, 63), (1024, 65), (1024, 1024),
                                       (1100, 1000), (1100, 1100), (4096, 4000), (16384, 16384)])
def test_decode_attention(k, Hq, Hk, max_len, n):
    print(f"decode_attention Hq={Hq} Hk={Hk} max_len={max_len} n={n}", flush=True)
    D = 128
    q = rnd(Hq * D, seed=11)
    kc, vc = rnd(Hk, max_len, D, seed=12), rnd(Hk, max_len, D, seed=13)
    work = k.decode_attention_workspace(Hq, Hk, D, max_len)
    p = torch.tensor([n - 1], dtype=torch.int32, device=DEV)
    out = k.decode_attention(q, kc, vc, p, Hq, Hk, D, work)
    torch.cuda.synchronize()
    close(out.reshape(-1), R.decode_attention(q, kc, vc, n, Hq, Hk), atol=1e-5)


def test_decode_attention_peaked_and_empty(k):
    Hq, Hk, D, max_len = 28, 4, 128, 300
    q = rnd(Hq * D, seed=14, scale=8.0)  # large logits: a few rows dominate each softmax
    kc, vc = rnd(Hk, max_len, D, seed=15), rnd(Hk, max_len, D, seed=16)
    work = k.decode_attention_workspace(Hq, Hk, D, max_len)
    p = torch.tensor([250], dtype=torch.int32, device=DEV)
    out = k.decode_attention(q, kc, vc, p, Hq, Hk, D, work)
    torch.cuda.synchronize()
    close(out.reshape(-1), R.decode_attention(q, kc, vc, 251, Hq, Hk), atol=1e-5)
    p.fill_(-1)  # no rows: zeros
    out = k.decode_attention(q, kc, vc, p, Hq, Hk, D, work)
    torch.cuda.synchronize()
    assert not out.any()


# ------------------------------------------------------------------ ns_decode_qkv_attention
@pytest.mark.parametrize("Hq,Hk", [(28, 4), (7, 1), (16, 4)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_decode_qkv_attention(k, Hq, Hk, with_bias):
    """The fused launch against the oracle's bias + RoPE followed by attention over the cache
    with the new row appended, at positions inside, at the end of and across 128-row splits, at
    the cache's last row, beyond it (no append, attention over the whole cache) and before row
    0 (zeros); one workspace serves every launch in turn."""
    D, max_len = 128, 600
    qn, kn = Hq * D, Hk * D
    work = k.decode_attention_workspace(Hq, Hk, D, max_len)
    freq = R.inv_freq(D, 1000000.0)
    kc, vc = rnd(Hk, max_len, D, seed=20), rnd(Hk, max_len, D, seed=21)
    for i, pos in enumerate([0, 1, 255, 256, 257, 300, 511, 512, 599, 600, 900, -1]):
        print(f"decode_qkv_attention Hq={Hq} Hk={Hk} bias={with_bias} pos={pos}", flush=True)
        # moderate q so that the oracle's and the kernel's q roundings, which may differ by one
        # bf16 ulp in rare elements, move the output by well under the tolerance
        qkv = rnd(qn + 2 * kn, seed=30 + i, scale=0.5)
        bias = rnd(qn + 2 * kn, seed=60 + i, scale=0.25) if with_bias else None
        qkv0, kc0, vc0 = qkv.clone(), kc.clone(), vc.clone()
        p = torch.tensor([pos], dtype=torch.int32, device=DEV)
        out = k.decode_qkv_attention(qkv, bias, freq.to(DEV), p, kc, vc, Hq, Hk, D, work)
        torch.cuda.synchronize()
        assert torch.equal(qkv, qkv0)  # qkv is not modified
        q_ref, k_ref, v_ref = R.decode_qkv(qkv0, bias, Hq, Hk, D, pos, freq)
        kc_ref, vc_ref = kc0.double().cpu(), vc0.double().cpu()
        if 0 <= pos < max_len:
            kc_ref[:, pos] = k_ref.reshape(Hk, D)
            vc_ref[:, pos] = v_ref.reshape(Hk, D)
            # the appended rows within a bf16 ulp of the oracle's, all other rows untouched
            close(kc[:, pos], kc_ref[:, pos], rtol=2 ** -7, atol=1e-4)
            assert torch.equal(vc[:, pos].double().cpu(), vc_ref[:, pos])
            kc_ref[:, pos] = kc[:, pos].double().cpu()  # attend over what the kernel stored
        assert torch.equal(kc.double().cpu(), kc_ref) and torch.equal(vc.double().cpu(), vc_ref)
        n = min(pos + 1, max_len)
        if n <= 0:
            assert not out.any()
            continue
        qr = q_ref.reshape(-1).to(torch.bfloat16)
        close(out.reshape(-1), R.decode_attention(qr, kc_ref.to(torch.bfloat16),
                                                  vc_ref.to(torch.bfloat16), n, Hq, Hk),
              atol=2e-3)


@pytest.mark.parametrize("H,vocab,D", [(3584, 152064, 128), (896, 1000, 64), (8, 3, 16)])
def test_decode_embed(k, H, vocab, D):
    """ns_decode_embed: x is the token's embedding row bit for bit (a zero row for ids outside
    the table) and rot holds cos, sin of fp32(pos) * inv_freq within 2 fp32 ulp of float64
    cos / sin of that same fp32 angle (the oracle's angle), at positions 0 .. 131071."""
    embed = rnd(vocab, H, seed=90)
    freq = R.inv_freq(D, 1000000.0)
    for tok, pos in [(0, 0), (vocab - 1, 1), (vocab // 2, 1023), (vocab // 3, 131071), (-1, 5),
                     (vocab, 7)]:
        print(f"decode_embed H={H} vocab={vocab} D={D} tok={tok} pos={pos}", flush=True)
        t = torch.tensor([tok], dtype=torch.int32, device=DEV)
        p = torch.tensor([pos], dtype=torch.int32, device=DEV)
        x, rot = k.decode_embed(t, p, embed, freq.to(DEV))
        torch.cuda.synchronize()
        want = embed[tok] if 0 <= tok < vocab else torch.zeros_like(embed[0])
        assert torch.equal(x.reshape(-1), want)
        ang = (torch.tensor(float(pos), dtype=torch.float32) * freq.float()).double()
        got = rot.double().cpu()
        ulp = 2.0 ** -23
        assert ((got[0] - torch.cos(ang)).abs() <= 2 * ulp).all()
        assert ((got[1] - torch.sin(ang)).abs() <= 2 * ulp).all()


@pytest.mark.parametrize("Hq,Hk", [(28, 4), (7, 1)])
def test_decode_qkv_attention_rotation_table(k, Hq, Hk):
    """With the step's rotation table from ns_decode_embed, the fused attention gives the same
    output bits and the same appended cache rows as computing the angles itself, at positions
    in the first split, across splits and past the cache."""
    D, max_len = 128, 600
    qn, kn = Hq * D, Hk * D
    freq = R.inv_freq(D, 1000000.0).to(DEV)
    embed = rnd(16, 64, seed=91)
    for i, pos in enumerate([0, 127, 128, 513, 599, 700]):
        print(f"decode_qkv_attention rotation table Hq={Hq} Hk={Hk} pos={pos}", flush=True)
        qkv = rnd(qn + 2 * kn, seed=92 + i, scale=0.5)
        bias = rnd(qn + 2 * kn, seed=99 + i, scale=0.25)
        kc, vc = rnd(Hk, max_len, D, seed=93), rnd(Hk, max_len, D, seed=94)
        kc2, vc2 = kc.clone(), vc.clone()
        p = torch.tensor([pos], dtype=torch.int32, device=DEV)
        t = torch.tensor([3], dtype=torch.int32, device=DEV)
        _, rot = k.decode_embed(t, p, embed, freq)
        wa = k.decode_attention_workspace(Hq, Hk, D, max_len)
        wb = k.decode_attention_workspace(Hq, Hk, D, max_len)
        a = k.decode_qkv_attention(qkv, bias, freq, p, kc, vc, Hq, Hk, D, wa)
        b = k.decode_qkv_attention(qkv, bias, freq, p, kc2, vc2, Hq, Hk, D, wb, rot=rot)
        torch.cuda.synchronize()
        assert torch.equal(a, b)
        assert torch.equal(kc, kc2) and torch.equal(vc, vc2)


def _attn_chunk(k):
    """Cache rows per attention split: the first length at which one more row adds a split
    to the workspace."""
    ws = k.lib.ns_decode_attention_workspace
    return next(n for n in range(1, 4097) if ws(28, 4, 128, n + 1) > ws(28, 4, 128, n))


@pytest.mark.parametrize("max_len", [200, 600, 2000, 4096, 16384])
def test_gemv_decode_attn_merges_splits(k, max_len):
    """The o GEMV fed by unmerged attention splits equals the merged attention output times
    the same weights (one split: the attention's own bf16 output; several: merged in the
    GEMV's activation load); contexts beyond four splits take the GEMV's batch loop."""
    Hq, Hk, D, N = 28, 4, 128, 3584
    qn, kn = Hq * D, Hk * D
    Wq, S = _w4(N, Hq * D, seed=70)
    freq = R.inv_freq(D, 1000000.0).to(DEV)
    work_a = k.decode_attention_workspace(Hq, Hk, D, max_len)
    work_b = k.decode_attention_workspace(Hq, Hk, D, max_len)
    kc, vc = rnd(Hk, max_len, D, seed=71), rnd(Hk, max_len, D, seed=72)
    qkv = rnd(qn + 2 * kn, seed=73, scale=0.5)
    for pos in sorted({0, 100, 127, 128, 255, 256, max_len // 2, max_len - 1}):
        print(f"gemv_decode_attn max_len={max_len} pos={pos}", flush=True)
        p = torch.tensor([pos], dtype=torch.int32, device=DEV)
        merged = k.decode_qkv_attention(qkv, None, freq, p, kc, vc, Hq, Hk, D, work_a)
        ref = k.w4_linear(merged, Wq, S, 128)
        a = torch.empty_like(merged)
        k.decode_qkv_attention(qkv, None, freq, p, kc, vc, Hq, Hk, D, work_b, out=a,
                               merge=False)
        y = k.gemv_decode_attn(a, work_b, p, max_len, Hq, Wq, S)
        torch.cuda.synchronize()
        if pos < _attn_chunk(k):
            assert torch.equal(y, ref)  # one split: the same bf16 activation
        else:  # the two merges round the activation independently: 1 bf16 ulp at most
            close(y, ref.double().cpu(), rtol=2 ** -6, atol=2e-3 * ref.abs().max().item())


@pytest.mark.parametrize("Hq,Hk,N", [(12, 2, 1536), (16, 2, 2048), (32, 8, 4096), (40, 8, 5120),
                                     (64, 8, 8192)])
def test_gemv_decode_attn_model_shapes(k, Hq, Hk, N):
    """The attention-merging o GEMV at the head counts and widths of other model sizes (1.5B,
    3B, Llama-3-8B, 14B/32B, 72B): each takes a layout of the plain GEMV's planner with room
    for the merged activation, and one split gives the plain GEMV's bits."""
    D, max_len, pos = 128, 256, 50
    qn, kn = Hq * D, Hk * D
    Wq, S = _w4(N, qn, seed=Hq + N)
    freq = R.inv_freq(D, 1000000.0).to(DEV)
    work_a = k.decode_attention_workspace(Hq, Hk, D, max_len)
    work_b = k.decode_attention_workspace(Hq, Hk, D, max_len)
    kc, vc = rnd(Hk, max_len, D, seed=Hq + 1), rnd(Hk, max_len, D, seed=Hq + 2)
    qkv = rnd(qn + 2 * kn, seed=Hq + 3, scale=0.5)
    p = torch.tensor([pos], dtype=torch.int32, device=DEV)
    merged = k.decode_qkv_attention(qkv, None, freq, p, kc, vc, Hq, Hk, D, work_a)
    ref = k.w4_linear(merged, Wq, S, 128)
    a = torch.empty_like(merged)
    k.decode_qkv_attention(qkv, None, freq, p, kc, vc, Hq, Hk, D, work_b, out=a, merge=False)
    y = k.gemv_decode_attn(a, work_b, p, max_len, Hq, Wq, S)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)


@pytest.mark.parametrize("Hq,Hk,N", [(56, 8, 7168), (52, 13, 6656), (60, 10, 2048)])
def test_gemv_decode_attn_wide_heads(k, Hq, Hk, N):
    """50 to 63 query heads, where the plain GEMV's layout has fewer threads than the merged
    activation has vectors: the merging GEMV takes sixteen-wave workgroups and agrees with the
    merged attention output times the weights to one bf16 ulp, with one split and with several."""
    D, max_len = 128, 700
    qn, kn = Hq * D, Hk * D
    Wq, S = _w4(N, qn, seed=Hq + 3 * N)
    freq = R.inv_freq(D, 1000000.0).to(DEV)
    work_a = k.decode_attention_workspace(Hq, Hk, D, max_len)
    work_b = k.decode_attention_workspace(Hq, Hk, D, max_len)
    kc, vc = rnd(Hk, max_len, D, seed=Hq + 4), rnd(Hk, max_len, D, seed=Hq + 5)
    qkv = rnd(qn + 2 * kn, seed=Hq + 6, scale=0.5)
    for pos in (50, 600):
        print(f"gemv_decode_attn Hq={Hq} N={N} pos={pos}", flush=True)
        p = torch.tensor([pos], dtype=torch.int32, device=DEV)
        merged = k.decode_qkv_attention(qkv, None, freq, p, kc, vc, Hq, Hk, D, work_a)
        ref = k.w4_linear(merged, Wq, S, 128)
        a = torch.empty_like(merged)
        k.decode_qkv_attention(qkv, None, freq, p, kc, vc, Hq, Hk, D, work_b, out=a,
                               merge=False)
        y = k.gemv_decode_attn(a, work_b, p, max_len, Hq, Wq, S)
        torch.cuda.synchronize()
        close(y, ref.double().cpu(), rtol=2 ** -6, atol=2e-3 * ref.abs().max().item())


# ------------------------------------------------------------------ ns_w4_gemv_decode
def _w4(N, K, seed):
    """Quantized random weights (GPU), as the runner's: N(0, 0.02) bf16 through the quantizer."""
    W = rnd(N, K, seed=seed, scale=0.02)
    return Kernels().w4_quantize(W, 128)


def _ref_linear(x_bf16, Wq, S):
    """float64 x @ deq(Wq, S)^T through the oracle (x: bf16 [K])."""
    xb = x_bf16.reshape(1, -1).cpu().view(torch.int16).numpy().view("uint16")
    return torch.from_numpy(O.linear_f64(xb, Wq.cpu().numpy().view("uint32"),
                                         S.cpu().view(torch.int16).numpy().view("uint16"), 128))


@pytest.mark.parametrize("N,K", [(4608, 3584), (3584, 18944), (100, 256), (64, 128)])
def test_gemv_decode_plain_equals_w4_linear(k, N, K):
    print(f"gemv_decode plain N={N} K={K}", flush=True)
    Wq, S = _w4(N, K, seed=40)
    x = rnd(1, K, seed=41)
    y = k.gemv_decode(Wq, S, 128, x=x)
    torch.cuda.synchronize()
    assert torch.equal(y, k.w4_linear(x, Wq, S, 128))


@pytest.mark.parametrize("N,K", [(4608, 3584), (37888, 3584), (256, 1024), (48, 8192)])
@pytest.mark.parametrize("with_r", [True, False])
def test_gemv_decode_rmsnorm_input(k, N, K, with_r):
    """Activation rmsnorm(res + r) * w fused into the GEMV: the new residual stream bit-exact,
    the output against the oracle's float64 product of the oracle-normalised activation."""
    print(f"gemv_decode rmsnorm N={N} K={K} r={with_r}", flush=True)
    Wq, S = _w4(N, K, seed=42)
    res, r, w = rnd(K, seed=43, scale=3.0), rnd(K, seed=44), rnd(K, seed=45, scale=0.5)
    res_out = torch.full((K,), 7.0, dtype=torch.bfloat16, device=DEV)
    y = k.gemv_decode(Wq, S, 128, res=res, r=r if with_r else None, norm_w=w, eps=1e-6,
                      res_out=res_out)
    torch.cuda.synchronize()
    v_ref, h_ref = R.rmsnorm(res.reshape(1, -1), r.reshape(1, -1) if with_r else None,
                             w, 1e-6)
    if with_r:
        assert torch.equal(res_out.double().cpu(), v_ref.reshape(-1))
    else:
        assert (res_out == 7.0).all()  # nothing added: the residual stream is not rewritten
    ref = _ref_linear(R.bf16_round(h_ref).to(torch.bfloat16), Wq, S)
    # the activation is bf16-rounded from fp32 arithmetic: an element may land one ulp from
    # the oracle's rounding, so the bound is the north-star one
    err = (y.double().cpu() - ref).abs().max().item()
    assert err <= 1e-2 * ref.abs().max().item(), err
    # and against the unfused pair (ns_rmsnorm, then ns_w4_linear)
    res2 = res.clone().reshape(1, -1)
    h = k.rmsnorm(res2, r.reshape(1, -1) if with_r else None, w, 1e-6)
    y2 = k.w4_linear(h, Wq, S, 128)
    torch.cuda.synchronize()
    close(y.reshape(-1), y2.reshape(-1).double().cpu(), rtol=2 ** -7,
          atol=1e-3 * y2.abs().max().item())


@pytest.mark.parametrize("N,K", [(37888, 3584), (2048, 896), (32, 256)])
@pytest.mark.parametrize("norm", [True, False])
def test_gemv_decode_swiglu_output(k, N, K, norm):
    """SwiGLU fused into the output of the interleaved gate/up GEMV equals ns_w4_linear of the
    same weights followed by ns_swiglu of the de-interleaved halves."""
    from nanoserve_amd.qwen import interleave_gate_up

    print(f"gemv_decode swiglu N={N} K={K} norm={norm}", flush=True)
    Wq, S = interleave_gate_up(*_w4(N, K, seed=46))
    x = rnd(1, K, seed=47)
    w = rnd(K, seed=48, scale=0.5)
    if norm:
        act = k.gemv_decode(Wq, S, 128, res=x, norm_w=w, eps=1e-6, swiglu=True)
        xin = k.rmsnorm(x.clone(), None, w, 1e-6)
    else:
        act = k.gemv_decode(Wq, S, 128, x=x, swiglu=True)
        xin = x
    gu = k.gemv_decode(Wq, S, 128, res=x, norm_w=w, eps=1e-6) if norm else k.w4_linear(
        xin, Wq, S, 128)
    I = N // 2
    g4 = gu.view(I // 8, 2, 8)
    ref = k.swiglu(g4[:, 0].reshape(1, I).contiguous(), g4[:, 1].reshape(1, I).contiguous())
    torch.cuda.synchronize()
    assert act.shape == (1, I)
    close(act, ref.double().cpu(), rtol=2 ** -8, atol=1e-6)


@pytest.mark.parametrize("M,N,K,G", [(128, 256, 256, 128), (256, 2048, 1024, 64),
                                     (2048, 37888, 3584, 128), (128, 7168, 18944, 128),
                                     (2048, 3584, 8192, 128), (512, 3584, 8192, 128),
                                     (256, 3584, 3584, 128), (768, 4608, 3584, 128),
                                     (384, 512, 512, 32), (1, 37888, 3584, 128),
                                     (3, 1024, 512, 128), (200, 1024, 512, 128)])
def test_linear_swiglu_equals_linear_then_swiglu(k, M, N, K, G):
    """ns_w4_linear_swiglu (SwiGLU in the GEMM / GEMV epilogue) against ns_w4_linear of the same
    interleaved weights followed by ns_swiglu of the de-interleaved halves: bit for bit (the same
    accumulation, and the products rounded to bf16 before the activation as the unfused pair
    stores them; M = 1 to a bf16 rounding, the decode GEMV may order its fp32 sums differently);
    M = 3 (unfused pair) and M = 200 (zero-row padding) through the wrapper."""
    from nanoserve_amd.qwen import interleave_gate_up

    print(f"linear_swiglu M={M} N={N} K={K} G={G}", flush=True)
    W = rnd(N, K, seed=61, scale=0.02)
    Wq, S = interleave_gate_up(*k.w4_quantize(W, G))
    x = rnd(M, K, seed=62)
    act = k.w4_linear_swiglu(x, Wq, S, G)
    I = N // 2
    g4 = k.w4_linear(x, Wq, S, G).view(M, I // 8, 2, 8)
    ref = k.swiglu(g4[:, :, 0].reshape(M, I).contiguous(), g4[:, :, 1].reshape(M, I).contiguous())
    torch.cuda.synchronize()
    assert act.shape == (M, I)
    if M == 1:  # the fused decode GEMV may split the k-groups differently: fp32 sums reordered
        close(act, ref.double().cpu(), rtol=2 ** -8, atol=1e-6)
    else:
        assert torch.equal(act, ref)
    out = torch.empty(M, I, dtype=torch.bfloat16, device=DEV)
    assert k.w4_linear_swiglu(x, Wq, S, G, out=out) is out
    torch.cuda.synchronize()
    assert torch.equal(out, act)


def test_gemv_decode_rejects(k):
    Wq, S = _w4(64, 256, seed=49)
    x = rnd(1, 256, seed=50)
    with pytest.raises(RuntimeError):  # G != 128
        k.gemv_decode(Wq, S, 64, x=x)
    Wq2, S2 = _w4(40, 256, seed=51)
    with pytest.raises(RuntimeError):  # N % 16 with swiglu
        k.gemv_decode(Wq2, S2, 128, x=x, swiglu=True)
    with pytest.raises(RuntimeError):  # res_out aliasing res
        k.gemv_decode(Wq, S, 128, res=x, r=x, norm_w=x, res_out=x)


# ------------------------------------------------------------------ ns_bf16_gemv (lm_head)
@pytest.mark.parametrize("N,K", [(152064, 3584), (1000, 896), (77, 8), (300, 8192), (64, 4096)])
@pytest.mark.parametrize("norm", [False, True])
def test_bf16_gemv(k, N, K, norm):
    """bf16 one-token product against float64 on the CPU (every row for small N, 256 sampled
    rows of the 1.09 GB lm_head), with and without the fused final add + RMSNorm."""
    print(f"bf16_gemv N={N} K={K} norm={norm}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(80)
    W = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    x, r, w = rnd(K, seed=81, scale=2.0), rnd(K, seed=82), rnd(K, seed=83, scale=0.5)
    if norm:
        y = k.bf16_gemv(W, res=x, r=r, norm_w=w, eps=1e-6)
        _, h = R.rmsnorm(x.reshape(1, -1), r.reshape(1, -1), w, 1e-6)
        a = R.bf16_round(h).reshape(-1)
    else:
        y = k.bf16_gemv(W, x=x)
        a = x.double().cpu()
    torch.cuda.synchronize()
    rows = torch.arange(N) if N <= 4096 else torch.randint(0, N, (256,), generator=torch.Generator().manual_seed(84))
    ref = W[rows.to(DEV)].double().cpu() @ a
    out = y.reshape(-1)[rows.to(DEV)].double().cpu()
    # fp32 accumulation of K products, bf16 output: half a bf16 ulp plus a small floor; with the
    # norm fused the activation may round one ulp away from the oracle's in rare elements
    tol = 2 ** -8 * ref.abs() + (2e-3 if norm else 1e-4) * ref.abs().max()
    assert ((out - ref).abs() <= tol).all(), (out - ref).abs().max().item()


# ------------------------------------------------------------------ packed tile format
@pytest.mark.parametrize("N,K", [(4608, 3584), (40, 384), (3584, 18944), (8960, 1536)])
def test_repack_matches_oracle(k, N, K):
    print(f"repack N={N} K={K}", flush=True)
    Wq, S = _w4(N, K, seed=90)
    Wp, Sp = k.w4_repack(Wq, S)
    torch.cuda.synchronize()
    wp_ref, sp_ref = O.repack_tiles(Wq.cpu().numpy().view("uint32"),
                                    S.cpu().view(torch.int16).numpy().view("uint16"))
    assert (Wp.cpu().numpy().view("uint32").reshape(-1) == wp_ref).all()
    assert (Sp.cpu().view(torch.int16).numpy().view("uint16").reshape(-1) == sp_ref).all()


@pytest.mark.parametrize("N,K", [(4608, 3584), (3584, 3584), (37888, 3584), (8960, 1536),
                                 (40, 384), (3584, 18944), (100, 4096), (1000, 8448),
                                 (264, 20480)])
@pytest.mark.parametrize("M", [2, 5, 8, 16])
def test_w4_linear_packed_equals_w4_linear(k, N, K, M):
    """The packed GEMV computes what ns_w4_linear computes (same exact dequantisation and
    products; ns_w4_linear is checked against the oracle in test_gpu_parity.py); the fp32 sums
    over k-groups run in another order, so outputs agree to one bf16 ulp (most bit for bit).
    K > 4096 takes the long-row kernel, whose activation passes through LDS in chunks of 16
    k-groups (K = 8448: a last chunk of two groups; K = 20480: the largest K it takes)."""
    print(f"w4_linear_packed N={N} K={K} M={M}", flush=True)
    Wq, S = _w4(N, K, seed=91)
    Wp, Sp = k.w4_repack(Wq, S)
    x = rnd(M, K, seed=92)
    y = k.w4_linear_packed(x, Wp, Sp, N)
    ref = k.w4_linear(x, Wq, S, 128) if M <= 8 else torch.cat(
        [k.w4_linear(x[:8], Wq, S, 128), k.w4_linear(x[8:], Wq, S, 128)])
    torch.cuda.synchronize()
    # near-zero outputs (cancelling sums) get an absolute floor from the output scale
    close(y, ref.double().cpu(), rtol=2 ** -7, atol=2e-5 * ref.abs().max().item())
    assert (y == ref).float().mean().item() > 0.9
    # and the packed output against the oracle's float64 product directly
    xb = x.cpu().view(torch.int16).numpy().view("uint16")
    ref64 = torch.from_numpy(O.linear_f64(xb, Wq.cpu().numpy().view("uint32"),
                                          S.cpu().view(torch.int16).numpy().view("uint16"), 128))
    close(y, ref64, rtol=2 ** -8, atol=1e-5 * ref64.abs().max().item())


@pytest.mark.parametrize("M,N,K", [(17, 200, 1024), (129, 1000, 3584), (300, 264, 8448), (64, 40, 384),
                                   (33, 4608, 3584), (256, 3584, 18944), (512, 4608, 3584),
                                   (40, 20000, 384)])
def test_w4_linear_packed_gemm(k, M, N, K):
    """M > 16 on packed weights runs the prefill GEMM on the packed tiles, with the reference
    GEMM's numerics: within half a bf16 ulp (+1e-5 ||ref||) of the oracle's product with every
    weight staged as bf16((q - 8) s) (shapes the float64 oracle finishes in seconds), and within
    one bf16 ulp of ns_w4_linear's GEMM where that takes the shape (N % 128 == 0: the same staged
    weights, fp32 sums in another order). Row tails inside a 256-row tile, column tails inside a
    16-row tile-row and a 128-column tile, and K from 384 to 18944."""
    print(f"w4_linear_packed gemm M={M} N={N} K={K}", flush=True)
    Wq, S = _w4(N, K, seed=93)
    Wp, Sp = k.w4_repack(Wq, S)
    x = rnd(M, K, seed=94)
    y = k.w4_linear_packed(x, Wp, Sp, N)
    torch.cuda.synchronize()
    if N % 128 == 0:
        ref = k.w4_linear(x, Wq, S, 128)
        torch.cuda.synchronize()
        close(y, ref.double().cpu(), rtol=2 ** -7, atol=2e-5 * ref.abs().max().item())
    if M * N * K <= 2 ** 30:
        xb = x.cpu().view(torch.int16).numpy().view("uint16")
        staged = torch.from_numpy(O.linear_f64(xb, Wq.cpu().numpy().view("uint32"),
                                               S.cpu().view(torch.int16).numpy().view("uint16"),
                                               128, bf16_weights=True))
        close(y, staged, rtol=2 ** -8, atol=1e-5 * staged.abs().max().item())


@pytest.mark.parametrize("M,N,K", [(2048, 3584, 8192), (1800, 3560, 8192), (512, 3584, 4096),
                                   (400, 3500, 4096)])
def test_w4_linear_packed_gemm_split_plans(k, M, N, K):
    """The packed GEMM's K-split plans (on MI355X's 256 CUs: 128 x 128 tiles over two wave groups
    for the first two shapes, 128 x 64 tiles over four for the last two), with ragged M and N:
    within one bf16 ulp of ns_w4_linear's GEMM on the first N // 128 * 128 rows, and within half
    an ulp (+1e-5 ||ref||) of the oracle's bf16-staged product on one activation row of every
    128-row band (a different offset per band) over all N columns."""
    print(f"w4_linear_packed gemm split M={M} N={N} K={K}", flush=True)
    Wq, S = _w4(N, K, seed=97)
    Wp, Sp = k.w4_repack(Wq, S)
    x = rnd(M, K, seed=98)
    y = k.w4_linear_packed(x, Wp, Sp, N)
    N1 = N // 128 * 128
    ref = k.w4_linear(x, Wq[:N1], S[:N1], 128)
    torch.cuda.synchronize()
    close(y[:, :N1], ref.double().cpu(), rtol=2 ** -7, atol=2e-5 * ref.abs().max().item())
    rows = [min(M - 1, 128 * b + (37 * b) % 128) for b in range((M + 127) // 128)]
    xb = x[rows].cpu().view(torch.int16).numpy().view("uint16")
    staged = torch.from_numpy(O.linear_f64(xb, Wq.cpu().numpy().view("uint32"),
                                           S.cpu().view(torch.int16).numpy().view("uint16"), 128,
                                           bf16_weights=True))
    close(y[rows], staged, rtol=2 ** -8, atol=1e-5 * staged.abs().max().item())


def test_w4_linear_packed_gemm_graph_and_rows_past_tile(k):
    """The packed GEMM under graph capture repeats the eager call bit for bit (eager calls of
    other shapes between replays), and rows of a partial last tile leave the rows past M alone."""
    N, K = 1000, 3584
    Wq, S = _w4(N, K, seed=95)
    Wp, Sp = k.w4_repack(Wq, S)
    x = rnd(300, K, seed=96)
    big = torch.full((320, N), 7.0, dtype=torch.bfloat16, device=DEV)
    out = big[:300]
    k.w4_linear_packed(x, Wp, Sp, N, out=out)
    eager = out.clone()
    torch.cuda.synchronize()
    assert (big[300:] == 7.0).all()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        yg = k.w4_linear_packed(x, Wp, Sp, N)
    for _ in range(2):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, eager)
        k.w4_linear_packed(x[:20], Wp, Sp, N)
        torch.cuda.synchronize()


# ------------------------------------------------------------------ the runner
@pytest.mark.parametrize("M,N,K", [(2048, 37888, 3584), (1024, 7168, 18944), (512, 3584, 3584),
                                   (200, 1040, 1024), (17, 4096, 512), (300, 37888, 384),
                                   (40, 37888, 384)])
def test_w4_linear_packed_swiglu(k, M, N, K):
    """ns_w4_linear_packed_swiglu (the packed GEMM with the SwiGLU epilogue; on MI355X the first
    shapes take the 128 x 128, two-group K-split and 128 x 64 plans, then ragged M and N) equals
    ns_w4_linear_packed of the same interleaved weights followed by ns_swiglu of the
    de-interleaved halves, bit for bit (the same accumulation; the products rounded to bf16
    before the activation as the unfused pair stores them), and, where ns_w4_linear_swiglu takes
    the shape, the standard format's fused GEMM to one bf16 rounding of its inputs."""
    from nanoserve_amd.qwen import interleave_gate_up

    print(f"w4_linear_packed_swiglu M={M} N={N} K={K}", flush=True)
    Wq, S = interleave_gate_up(*_w4(N, K, seed=101))
    Wp, Sp = k.w4_repack(Wq, S)
    x = rnd(M, K, seed=102)
    act = k.w4_linear_packed_swiglu(x, Wp, Sp, N)
    I = N // 2
    g4 = k.w4_linear_packed(x, Wp, Sp, N).view(M, I // 8, 2, 8)
    ref = k.swiglu(g4[:, :, 0].reshape(M, I).contiguous(), g4[:, :, 1].reshape(M, I).contiguous())
    torch.cuda.synchronize()
    assert act.shape == (M, I)
    assert torch.equal(act, ref)
    if M % 128 == 0 and N % 128 == 0:
        std = k.w4_linear_swiglu(x, Wq, S, 128)
        torch.cuda.synchronize()
        close(act, std.double().cpu(), rtol=2 ** -6, atol=1e-3 * std.abs().max().item())
    out = torch.full((M + 3, I), 5.0, dtype=torch.bfloat16, device=DEV)
    assert k.w4_linear_packed_swiglu(x, Wp, Sp, N, out=out[:M]) is not None
    torch.cuda.synchronize()
    assert torch.equal(out[:M], act) and (out[M:] == 5.0).all()


def _hf_model(H, nh, nkv, I, V, layers, seed):
    pytest.importorskip("transformers")
    return R.tiny_qwen2(H, nh, nkv, I, V, layers, seed)


def _effective_hf(m, runner):
    """A float32 copy of the HF model holding exactly the weights the runner uses: W4 weights
    dequantized by the oracle, everything else rounded to bf16."""
    ref = copy.deepcopy(m)
    s = runner.shape
    D = s.head_dim
    qn, kn, I = s.heads * D, s.kv_heads * D, s.intermediate

    def deq(pair):
        Wq, S = pair
        return torch.from_numpy(O.dequant_f32(Wq.cpu().numpy().view("uint32"),
                                              S.cpu().view(torch.int16).numpy().view("uint16"),
                                              s.group))

    def r16(t):
        return t.detach().to(torch.bfloat16).float()

    with torch.no_grad():
        for layer, L in zip(ref.model.layers, runner.layers):
            at, mlp = layer.self_attn, layer.mlp
            wqkv = deq(L["wqkv"])
            at.q_proj.weight.copy_(wqkv[:qn])
            at.k_proj.weight.copy_(wqkv[qn:qn + kn])
            at.v_proj.weight.copy_(wqkv[qn + kn:])
            for b in (at.q_proj.bias, at.k_proj.bias, at.v_proj.bias):
                b.copy_(r16(b))
            at.o_proj.weight.copy_(deq(L["wo"]))
            wgu = deq(L["wgu"]).view(I // 8, 2, 8, -1)  # gate/up rows interleaved by 8
            mlp.gate_proj.weight.copy_(wgu[:, 0].reshape(I, -1))
            mlp.up_proj.weight.copy_(wgu[:, 1].reshape(I, -1))
            mlp.down_proj.weight.copy_(deq(L["wd"]))
            for ln in (layer.input_layernorm, layer.post_attention_layernorm):
                ln.weight.copy_(r16(ln.weight))
        ref.model.norm.weight.copy_(r16(ref.model.norm.weight))
        ref.model.embed_tokens.weight.copy_(r16(ref.model.embed_tokens.weight))
        ref.lm_head.weight.copy_(r16(ref.lm_head.weight))
    return ref


def _check_logits(out, ref):
    assert R.logits_match(out, ref), R.logits_gap(out, ref)


def test_runner_gptq_calibration(k):
    """from_hf with calibration ids: the runner (GPTQ weights) still matches the HF model holding
    its dequantized weights, and its logits are closer to the unquantized model's than the
    round-to-nearest runner's, on the calibration tokens and on held-out tokens."""
    V = 512
    m = _hf_model(256, 2, 1, 512, V, layers=2, seed=3)
    g = torch.Generator().manual_seed(0)
    calib = torch.randint(0, V, (4, 64), generator=g)
    held = torch.randint(0, V, (1, 48), generator=g)
    rtn = Qwen2Runner.from_hf(m, device=DEV, kernels=k)
    cal = Qwen2Runner.from_hf(m, device=DEV, kernels=k, calib_ids=calib)
    with torch.no_grad():
        dense_c = m(calib[:1]).logits[0]
        dense_h = m(held).logits[0]
        eff_c = _effective_hf(m, cal)(calib[:1]).logits[0]

    def gap(runner, ids, dense):
        out = runner.forward(ids[0].to(DEV), 0).float().cpu()
        return float((out - dense).norm() / dense.norm())

    out = cal.forward(calib[0].to(DEV), 0)
    torch.cuda.synchronize()
    _check_logits(out, eff_c)
    g_c, r_c = gap(cal, calib[:1], dense_c), gap(rtn, calib[:1], dense_c)
    g_h, r_h = gap(cal, held, dense_h), gap(rtn, held, dense_h)
    print(f"logits gap to the dense model: calib gptq {g_c:.4f} rtn {r_c:.4f}; "
          f"held-out gptq {g_h:.4f} rtn {r_h:.4f}", flush=True)
    assert g_c < 0.6 * r_c and g_h < 0.9 * r_h


@pytest.mark.parametrize("H,nh,nkv,I,V,T,cache", [(896, 7, 1, 1024, 1000, 12, 0),
                                                   (256, 2, 1, 512, 512, 5, 0),
                                                   (512, 4, 2, 768, 640, 130, 0),
                                                   (512, 4, 2, 768, 640, 130, 2304)])
def test_runner_matches_hf_qwen2(k, H, nh, nkv, I, V, T, cache):
    """Prompt pass (GEMV for T <= 8, GEMM above) and four decode steps, eager and graph; with a
    cache longer than 16 attention splits the steps merge the splits in the attention's own
    merge kernel and run the plain o GEMV."""
    print(f"runner H={H} heads={nh}/{nkv} I={I} V={V} T={T} cache={cache}", flush=True)
    m = _hf_model(H, nh, nkv, I, V, layers=2, seed=0)
    runner = Qwen2Runner.from_hf(m, device=DEV, kernels=k)
    ref_model = _effective_hf(m, runner)
    n_dec = 4
    ids = torch.randint(0, V, (T + n_dec,), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        ref = ref_model(ids[None]).logits[0]
    runner.alloc_cache(max(T + n_dec, cache))
    assert runner.merge_in_o == (cache == 0)
    prompt = runner.forward(ids[:T].to(DEV), 0, use_cache=True)
    torch.cuda.synchronize()
    _check_logits(prompt, ref[:T])
    # eager decode steps, teacher-forced
    eager = []
    for i in range(n_dec):
        eager.append(runner.forward(ids[T + i:T + i + 1].to(DEV), T + i, use_cache=True))
    torch.cuda.synchronize()
    for i in range(n_dec):
        _check_logits(eager[i], ref[T + i:T + i + 1])
    # the same steps through the captured graph: bit-identical to the eager steps
    runner.capture_decode()
    for i in range(n_dec):
        out = runner.decode(ids[T + i].to(DEV), T + i).clone()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[i]), i


def test_runner_packed_prefill_matches_hf(k):
    """Prompt passes on packed weights (pack_prefill: packed-format GEMMs for more than 16
    tokens, the SwiGLU one for gate/up) match the HF model holding the runner's dequantized
    weights, and the standard-format prompt pass to bf16 roundings; a 40-token prompt continued
    by a 30-token chunk at position 40 (both packed) and decode steps after it read the cache
    the packed passes wrote."""
    V = 640
    m = _hf_model(512, 4, 2, 768, V, layers=2, seed=2)
    runner = Qwen2Runner.from_hf(m, device=DEV, kernels=k)
    ref_model = _effective_hf(m, runner)
    ids = torch.randint(0, V, (74,), generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        ref = ref_model(ids[None]).logits[0]
    std = runner.forward(ids[:40].to(DEV), 0)
    assert runner.pack_prefill() is runner
    runner.alloc_cache(80)
    first = runner.forward(ids[:40].to(DEV), 0, use_cache=True)
    second = runner.forward(ids[40:70].to(DEV), 40, use_cache=True)
    steps = [runner.forward(ids[70 + i:71 + i].to(DEV), 70 + i, use_cache=True) for i in range(4)]
    torch.cuda.synchronize()
    _check_logits(first, ref[:40])
    _check_logits(second, ref[40:70])
    for i in range(4):
        _check_logits(steps[i], ref[70 + i:71 + i])
    _check_logits(first, std.float().cpu())
    # 16 tokens or fewer stay on the standard format
    short = runner.forward(ids[:16].to(DEV), 0)
    runner.packed = None
    short_std = runner.forward(ids[:16].to(DEV), 0)
    torch.cuda.synchronize()
    assert torch.equal(short, short_std)


def test_graph_replays_match_eager_with_work_between(k):
    """Several replays of one captured step at different positions, with eager kernel work and
    synchronisations between them; every replay must equal the eager step."""
    shape = Qwen2Shape(layers=2, hidden=896, heads=7, kv_heads=1, head_dim=128,
                       intermediate=1024, vocab=1000)
    runner = Qwen2Runner.random(shape, device=DEV, seed=3, kernels=k)
    max_len = 200
    runner.alloc_cache(max_len)
    g = torch.Generator(device=DEV).manual_seed(4)
    runner.cache_k.copy_(torch.randn(runner.cache_k.shape, generator=g, device=DEV))
    runner.cache_v.copy_(torch.randn(runner.cache_v.shape, generator=g, device=DEV))
    base_k, base_v = runner.cache_k.clone(), runner.cache_v.clone()
    steps = [(5, 10), (17, 150), (999, 0), (3, 199)]
    eager = []
    for tok, pos in steps:
        eager.append(runner.decode(tok, pos).clone())
    torch.cuda.synchronize()
    runner.cache_k.copy_(base_k)
    runner.cache_v.copy_(base_v)
    runner.capture_decode()
    runner.cache_k.copy_(base_k)  # the capture wrote row max_len - 1
    runner.cache_v.copy_(base_v)
    for i, (tok, pos) in enumerate(steps):
        junk = torch.randn(4096, device=DEV).sum()  # eager work between replays
        out = runner.decode(tok, pos).clone()
        torch.cuda.synchronize()
        assert junk.isfinite()
        assert torch.equal(out, eager[i]), (tok, pos)


def test_generate_graph_equals_eager(k):
    shape = Qwen2Shape(layers=2, hidden=256, heads=2, kv_heads=1, head_dim=128,
                       intermediate=512, vocab=512)
    runner = Qwen2Runner.random(shape, device=DEV, seed=5, kernels=k)
    prompt = torch.randint(0, 512, (9,), generator=torch.Generator().manual_seed(6)).to(DEV)
    a = runner.generate(prompt, 6, use_graph=False)
    b = runner.generate(prompt, 6, use_graph=True)
    assert a == b and len(a) == 6


def _bits16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view("uint16")


def _oracle_layer(L, s, x0, kc, vc, pos, freq):
    """One decoder layer of the fused decode step in float64 (oracle/decode_ref.py operators,
    oracle.w4_oracle.linear_f64 for the W4 projections), with every intermediate rounded to bf16
    where the kernels store it: h = bf16(x1 + d) for the layer's input row x0 [H] (bf16),
    caches [Hk, max_len, D] (bf16, row pos overwritten with the token's k / v)."""
    D, G = s.head_dim, s.group

    def lin(a, pair):  # a: bf16-exact float64 [K] -> float64 [N]
        Wq, S = pair
        return torch.from_numpy(O.linear_f64(_bits16(a.reshape(1, -1).to(torch.bfloat16)),
                                             Wq.cpu().numpy().view("uint32"), _bits16(S), G))[0]

    _, a = R.rmsnorm(x0.reshape(1, -1), None, L["ln_in"], s.eps)
    qkv = R.bf16_round(lin(R.bf16_round(a)[0], L["wqkv"]))
    q, kk, v = R.decode_qkv(qkv.to(torch.bfloat16), L["bqkv"], s.heads, s.kv_heads, D, pos, freq)
    kc, vc = kc.cpu().clone(), vc.cpu().clone()
    kc[:, pos] = kk.reshape(s.kv_heads, D).to(torch.bfloat16)
    vc[:, pos] = v.reshape(s.kv_heads, D).to(torch.bfloat16)
    attn = R.bf16_round(R.decode_attention(q.reshape(-1).to(torch.bfloat16), kc, vc, pos + 1,
                                           s.heads, s.kv_heads))
    o = R.bf16_round(lin(attn, L["wo"]))
    x1 = R.bf16_round(R._f64(x0) + o)
    _, h2 = R.rmsnorm(x1.reshape(1, -1).to(torch.bfloat16), None, L["ln_post"], s.eps)
    gu = R.bf16_round(lin(R.bf16_round(h2)[0], L["wgu"])).view(-1, 2, 8)  # interleaved by 8
    act = R.bf16_round(R.swiglu(gu[:, 0].reshape(-1), gu[:, 1].reshape(-1)))
    d = R.bf16_round(lin(act, L["wd"]))
    return R.bf16_round(x1 + d)


def test_runner_qwen25_7b_shape_context_1024(k):
    """The whole 28-layer Qwen2.5-7B-shaped W4 decode step at context 1024:
    the captured graph replays the eager step bit for bit; and the first and the last layer,
    each run alone as a one-layer step on its own weights and cache, match the float64 oracle
    composition of the decoder layer (residual stream after the layer; bar: the north-star
    1e-2 * max |ref|, with bf16 activations between kernels)."""
    s = Qwen2Shape()
    ctx, tok, pos = 1024, 1234, 1023
    print("runner 7B shape: building 28 layers", flush=True)
    runner = Qwen2Runner.random(s, device=DEV, seed=7, kernels=k)
    runner.alloc_cache(ctx)
    g = torch.Generator(device=DEV).manual_seed(8)
    runner.cache_k.copy_(torch.randn(runner.cache_k.shape, generator=g, device=DEV))
    runner.cache_v.copy_(torch.randn(runner.cache_v.shape, generator=g, device=DEV))
    eager = runner.decode(tok, pos).clone()
    torch.cuda.synchronize()
    assert torch.isfinite(eager.float()).all()
    runner.capture_decode()
    for _ in range(2):
        replay = runner.decode(tok, pos).clone()
        torch.cuda.synchronize()
        assert torch.equal(replay, eager)
    freq = R.inv_freq(s.head_dim, s.rope_theta)
    x0 = runner.embed[tok]
    for li in (0, s.layers - 1):
        print(f"runner 7B shape: layer {li} alone against the oracle", flush=True)
        one = Qwen2Runner(dataclasses.replace(s, layers=1), runner.embed, runner.final_norm,
                          runner.lm_head, [runner.layers[li]], k)
        one.alloc_cache(ctx)
        one.cache_k[0].copy_(runner.cache_k[li])
        one.cache_v[0].copy_(runner.cache_v[li])
        kc, vc = one.cache_k[0].clone(), one.cache_v[0].clone()
        one.decode(tok, pos)
        torch.cuda.synchronize()
        # one layer: the residual stream after it is bf16(x2 + d) (x2 holds the stream after the
        # attention block, d the down projection not yet added)
        h = R.bf16_round(R._f64(one.x2[0]) + R._f64(one.d[0]))
        ref = _oracle_layer(runner.layers[li], s, x0, kc, vc, pos, freq)
        err = float((h - ref).abs().max() / ref.abs().max())
        print(f"runner 7B shape: layer {li} max rel err {err:.2e}", flush=True)
        assert err <= 1e-2, (li, err)
        del one
    del runner
    torch.cuda.empty_cache()
