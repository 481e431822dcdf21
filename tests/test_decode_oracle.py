"""CPU checks that pin oracle/decode_ref.py (the checker of the decoder-step kernels) against
independent implementations: Hugging Face transformers' Qwen2 modules (Qwen2RMSNorm,
Qwen2RotaryEmbedding + apply_rotary_pos_emb, the MLP activation), PyTorch's
scaled_dot_product_attention in float64, and closed forms. A wrong sign, index or term in the
oracle fails one of these."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import decode_ref as R

transformers = pytest.importorskip("transformers")
from transformers import Qwen2Config  # noqa: E402
from transformers.models.qwen2 import modeling_qwen2 as hfq  # noqa: E402


def _bf16(*shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("H", [8, 896, 3584])
@pytest.mark.parametrize("with_r", [False, True])
def test_rmsnorm_matches_hf_qwen2rmsnorm(H, with_r):
    x, r, w = _bf16(5, H, seed=1), _bf16(5, H, seed=2), _bf16(H, seed=3, scale=0.3)
    v, y = R.rmsnorm(x, r if with_r else None, w, 1e-6)
    m = hfq.Qwen2RMSNorm(H, eps=1e-6).double()
    with torch.no_grad():
        m.weight.copy_(w.double())
    # the HF module on the same residual stream: same formula, independent code; it computes
    # in float32 internally whatever the input type, hence the float32-level tolerance
    ref = m(v)
    torch.testing.assert_close(y, ref, rtol=1e-6, atol=1e-7)
    if with_r:
        # residual stream: bf16(x + r); the sum of two bf16 values is exact in float32
        torch.testing.assert_close(v, (x.float() + r.float()).to(torch.bfloat16).double(),
                                   rtol=0, atol=0)
    else:
        assert torch.equal(v, x.double())


def test_rmsnorm_closed_form():
    # a constant row c normalises to sign(c) * w (up to eps)
    x = torch.full((1, 64), -3.0).to(torch.bfloat16)
    w = _bf16(64, seed=4)
    _, y = R.rmsnorm(x, None, w, 0.0)
    torch.testing.assert_close(y[0], -w.double(), rtol=1e-12, atol=0)


@pytest.mark.parametrize("theta", [10000.0, 1000000.0])
def test_inv_freq_matches_hf(theta):
    cfg = Qwen2Config(hidden_size=896, num_attention_heads=7, num_key_value_heads=1,
                      rope_theta=theta)
    hf = hfq.Qwen2RotaryEmbedding(cfg)
    torch.testing.assert_close(R.inv_freq(128, theta), hf.inv_freq.float(), rtol=0, atol=0)


@pytest.mark.parametrize("pos0", [0, 7, 1023, 32000])
def test_rope_matches_hf_apply_rotary_pos_emb(pos0):
    Hq, Hk, D, T = 7, 1, 128, 3
    cfg = Qwen2Config(hidden_size=Hq * D, num_attention_heads=Hq, num_key_value_heads=Hk,
                      rope_theta=1000000.0)
    emb = hfq.Qwen2RotaryEmbedding(cfg)
    q, k = _bf16(T, Hq * D, seed=5), _bf16(T, Hk * D, seed=6)
    pos = torch.arange(pos0, pos0 + T)
    freq = R.inv_freq(D, 1000000.0)
    qo, ko = R.rope(q, Hq, D, pos, freq), R.rope(k, Hk, D, pos, freq)
    # HF: float32 cos / sin of the float32 angle, applied in float64 here
    cos, sin = emb(q.float(), pos[None])
    qh = q.double().reshape(1, T, Hq, D).transpose(1, 2)
    kh = k.double().reshape(1, T, Hk, D).transpose(1, 2)
    qr, kr = hfq.apply_rotary_pos_emb(qh, kh, cos.double(), sin.double())
    qr = qr.transpose(1, 2).reshape(T, Hq * D)
    kr = kr.transpose(1, 2).reshape(T, Hk * D)
    # the only difference is float32 vs float64 cos / sin of the same float32 angle
    torch.testing.assert_close(qo, qr, rtol=0, atol=1e-5)
    torch.testing.assert_close(ko, kr, rtol=0, atol=1e-5)


def test_rope_closed_forms():
    D = 128
    x = _bf16(1, 2 * D, seed=7)
    freq = R.inv_freq(D, 10000.0)
    # position 0 is the identity
    torch.testing.assert_close(R.rope(x, 2, D, torch.tensor([0]), freq), x.double(), rtol=0,
                               atol=0)
    # a rotation keeps each (i, i + D/2) pair's norm
    y = R.rope(x, 2, D, torch.tensor([12345]), freq).reshape(2, D)
    xv = x.double().reshape(2, D)
    n_in = xv[:, : D // 2] ** 2 + xv[:, D // 2:] ** 2
    n_out = y[:, : D // 2] ** 2 + y[:, D // 2:] ** 2
    torch.testing.assert_close(n_out, n_in, rtol=1e-12, atol=1e-12)
    # pair 0 (inv_freq 1) at position p: (x cos p - y sin p, y cos p + x sin p)
    p = 3
    y3 = R.rope(x, 2, D, torch.tensor([p]), freq).reshape(2, D)
    a, b = xv[0, 0], xv[0, D // 2]
    ang = float(torch.tensor(float(p), dtype=torch.float32) * freq[0])
    assert abs(float(y3[0, 0]) - (a * math.cos(ang) - b * math.sin(ang))) < 1e-12
    assert abs(float(y3[0, D // 2]) - (b * math.cos(ang) + a * math.sin(ang))) < 1e-12


def test_swiglu_matches_silu():
    g, u = _bf16(4, 256, seed=8, scale=4.0), _bf16(4, 256, seed=9)
    ref = F.silu(g.double()) * u.double()
    torch.testing.assert_close(R.swiglu(g, u), ref, rtol=1e-14, atol=1e-14)


@pytest.mark.parametrize("n", [1, 5, 64, 300])
@pytest.mark.parametrize("Hq,Hk", [(28, 4), (7, 1), (4, 4)])
def test_decode_attention_matches_sdpa(n, Hq, Hk):
    D, max_len = 128, 320
    q = _bf16(Hq * D, seed=10)
    kc, vc = _bf16(Hk, max_len, D, seed=11), _bf16(Hk, max_len, D, seed=12)
    out = R.decode_attention(q, kc, vc, n, Hq, Hk)
    qh = q.double().reshape(1, Hq, 1, D)
    kh = kc[:, :n].double()[None].repeat_interleave(Hq // Hk, dim=1)
    vh = vc[:, :n].double()[None].repeat_interleave(Hq // Hk, dim=1)
    ref = F.scaled_dot_product_attention(qh, kh, vh).reshape(-1)
    torch.testing.assert_close(out, ref, rtol=1e-12, atol=1e-12)
    if n == 1:  # one row: the output is that row's value, for every head of the group
        rep = Hq // Hk
        for h in range(Hq):
            torch.testing.assert_close(out.reshape(Hq, D)[h], vc[h // rep, 0].double(), rtol=0,
                                       atol=1e-15)


def test_decode_qkv_matches_hf_rope_of_biased_projection():
    Hq, Hk, D, pos = 7, 1, 128, 77
    qkv = _bf16((Hq + 2 * Hk) * D, seed=13)
    bias = _bf16((Hq + 2 * Hk) * D, seed=14, scale=0.5)
    freq = R.inv_freq(D, 1000000.0)
    q, k, v = R.decode_qkv(qkv, bias, Hq, Hk, D, pos, freq)
    biased = (qkv.float() + bias.float()).to(torch.bfloat16)  # the reference's bf16 `q += bq`
    cfg = Qwen2Config(hidden_size=Hq * D, num_attention_heads=Hq, num_key_value_heads=Hk,
                      rope_theta=1000000.0)
    cos, sin = hfq.Qwen2RotaryEmbedding(cfg)(biased.float(), torch.tensor([[pos]]))
    qh = biased[: Hq * D].double().reshape(1, Hq, 1, D)
    kh = biased[Hq * D:(Hq + Hk) * D].double().reshape(1, Hk, 1, D)
    qr, kr = hfq.apply_rotary_pos_emb(qh, kh, cos.double(), sin.double())
    # q and k are bf16-rounded by decode_qkv: within half a bf16 ulp of HF's unrounded values
    torch.testing.assert_close(q.reshape(-1), qr.reshape(-1), rtol=2 ** -8, atol=1e-5)
    torch.testing.assert_close(k.reshape(-1), kr.reshape(-1), rtol=2 ** -8, atol=1e-5)
    assert torch.equal(v.reshape(-1), biased[(Hq + Hk) * D:].double())


def _logits(m, ids):
    with torch.no_grad():
        return m(ids[None]).logits[0]


@pytest.mark.parametrize("H,nh,nkv,I,V", [(896, 7, 1, 1024, 1000), (512, 4, 2, 768, 640)])
def test_logits_bar_accepts_bf16_and_rejects_mistakes(H, nh, nkv, I, V):
    """The runner's acceptance bar (R.logits_match) against float32 Hugging Face logits: the
    same model run in bf16 passes it; the same model with one plausible mistake fails it."""
    import copy

    m = R.tiny_qwen2(H, nh, nkv, I, V, layers=2, seed=0)
    ids = torch.randint(0, V, (16,), generator=torch.Generator().manual_seed(1))
    ref = _logits(m, ids)
    assert R.logits_match(_logits(copy.deepcopy(m).to(torch.bfloat16), ids).float(), ref)

    def mutated(fn):
        mm = copy.deepcopy(m)
        with torch.no_grad():
            fn(mm)
        return _logits(mm, ids)

    def no_bias(mm):
        for layer in mm.model.layers:
            layer.self_attn.q_proj.bias.zero_()
            layer.self_attn.k_proj.bias.zero_()

    def wrong_theta(mm):
        emb = mm.model.rotary_emb
        emb.inv_freq.copy_(R.inv_freq(H // nh, 10000.0))
        emb.original_inv_freq = emb.inv_freq

    def unit_norm_weights(mm):
        for layer in mm.model.layers:
            layer.post_attention_layernorm.weight.fill_(1.0)

    def gate_up_swapped(mm):
        for layer in mm.model.layers:
            g = layer.mlp.gate_proj.weight.clone()
            layer.mlp.gate_proj.weight.copy_(layer.mlp.up_proj.weight)
            layer.mlp.up_proj.weight.copy_(g)

    def v_bias_dropped(mm):
        for layer in mm.model.layers:
            layer.self_attn.v_proj.bias.zero_()

    for fn in (no_bias, wrong_theta, unit_norm_weights, gate_up_swapped, v_bias_dropped):
        out = mutated(fn)
        assert not R.logits_match(out, ref), (fn.__name__, R.logits_gap(out, ref))
