"""CPU references for the decoder-step operators -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and ``__graft_entry__.smoke()`` may import this module, as the checker of the
HIP kernels in ``nanoserve_amd/csrc/decode_ops.hip``; the product package never imports it.

Float64 PyTorch restatements of what the reference's kernels compute (fp32 there; float64
here so the reference itself adds no rounding beyond the bf16 stores the kernels make).
Inputs are bf16 tensors (any device; computed on the CPU); outputs are float64 unless noted.
Each function cites the reference lines it follows. They are pinned, in
tests/test_decode_oracle.py, against independent implementations: Hugging Face transformers'
Qwen2RMSNorm, Qwen2RotaryEmbedding + apply_rotary_pos_emb and the MLP activation, and
PyTorch's scaled_dot_product_attention, plus closed forms (a rotation preserves norms,
attention over one row returns that row's value).
"""
from __future__ import annotations

import math

import torch


def _f64(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to("cpu", torch.float64)


def bf16_round(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (RNE) and return as float64."""
    return t.to(torch.float32).to(torch.bfloat16).to(torch.float64)


def add_residual(x: torch.Tensor, r: torch.Tensor) -> torch.Tensor:
    """x + r rounded to bf16: the residual stream the fused kernel stores
    (kernels/fused/rmsnorm.cuh:27-32). Exact: the sum of two bf16 values is exact in float64,
    so one rounding of it equals the kernel's fp32 add + round."""
    return bf16_round(_f64(x) + _f64(r))


def rmsnorm(x: torch.Tensor, r: torch.Tensor | None, w: torch.Tensor, eps: float):
    """(new residual stream, normalised output before the bf16 store) of ns_rmsnorm
    (kernels/fused/rmsnorm.cuh:10-45): v = bf16(x + r) (or x), y = v * rsqrt(mean(v^2) + eps) * w,
    one rounding at the store."""
    v = add_residual(x, r) if r is not None else _f64(x)
    inv = 1.0 / torch.sqrt((v * v).mean(-1, keepdim=True) + eps)
    return v, v * inv * _f64(w)


def inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """theta^(-2i/D) in fp32, as the reference computes it (python/nanoserve/qwen.py:64-65)."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))


def rope(x: torch.Tensor, n_heads: int, head_dim: int, pos: torch.Tensor,
         freq: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of x [T, n_heads*head_dim] at positions pos [T]
    (kernels/fused/rope.cuh:1-9, 27-34): the angle is the fp32 product fp32(pos) * inv_freq[i]
    (as the kernel forms it), then cos / sin and the rotation in float64."""
    T = x.shape[0]
    ang = (pos.to(torch.float32)[:, None] * freq.to(torch.float32)[None, :]).to(torch.float64)
    c, s = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    v = _f64(x).reshape(T, n_heads, head_dim)
    x1, x2 = v[..., : head_dim // 2], v[..., head_dim // 2:]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1).reshape(T, n_heads * head_dim)


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up (kernels/fused/swiglu.cuh:8, 56-66)."""
    g = _f64(gate)
    return g / (1.0 + torch.exp(-g)) * _f64(up)


def decode_qkv(qkv: torch.Tensor, bias: torch.Tensor | None, n_heads: int, n_kv: int,
               head_dim: int, pos: int, freq: torch.Tensor):
    """One decode token's q, k, v (bf16-exact float64 values) after the bias add and RoPE, as
    python/nanoserve/qwen.py:147-151 computes them with the fused rope kernel: every element
    is bf16(qkv + bias), then q and k are rotated and stored as bf16."""
    qn, kn = n_heads * head_dim, n_kv * head_dim
    v = _f64(qkv).reshape(1, -1)
    if bias is not None:
        v = bf16_round(v + _f64(bias).reshape(1, -1))
    p = torch.tensor([pos])
    q = bf16_round(rope(v[:, :qn], n_heads, head_dim, p, freq))
    k = bf16_round(rope(v[:, qn:qn + kn], n_kv, head_dim, p, freq))
    return q, k, v[:, qn + kn:]


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, n: int,
                     n_heads: int, n_kv: int) -> torch.Tensor:
    """Attention of one query token over cache rows 0..n-1 (python/nanoserve/qwen.py:124-133:
    SDPA with the kv heads repeated Hq/Hk times, scale 1/sqrt(D)). q [Hq*D]; caches
    [Hk, max_len, D]; returns [Hq*D] float64."""
    D = k_cache.shape[-1]
    qh = _f64(q).reshape(n_heads, D)
    rep = n_heads // n_kv
    out = torch.empty(n_heads, D, dtype=torch.float64)
    for h in range(n_heads):
        K = _f64(k_cache[h // rep, :n])
        V = _f64(v_cache[h // rep, :n])
        s = (K @ qh[h]) / math.sqrt(D)
        p = torch.softmax(s, dim=0)
        out[h] = p @ V
    return out.reshape(-1)


# Acceptance bar for a whole decoder's logits against a float32 reference with the same
# weights: bf16 activations between kernels (as the reference's runner has) put the measured
# gap of the test models at about 1e-2 * max|ref|; the plausible mistakes checked in
# tests/test_decode_oracle.py land far outside it.
LOGITS_REL_TOL = 3e-2
LOGITS_MIN_COS = 0.999


def logits_gap(out: torch.Tensor, ref: torch.Tensor):
    """(max |out - ref| / max |ref|, cosine similarity) of two logits tensors."""
    out, ref = out.detach().double().cpu(), ref.detach().double().cpu()
    rel = ((out - ref).abs().max() / ref.abs().max()).item()
    cos = torch.nn.functional.cosine_similarity(out.flatten(), ref.flatten(), dim=0).item()
    return rel, cos


def logits_match(out: torch.Tensor, ref: torch.Tensor) -> bool:
    rel, cos = logits_gap(out, ref)
    return rel <= LOGITS_REL_TOL and cos >= LOGITS_MIN_COS


def tiny_qwen2(H: int, n_heads: int, n_kv: int, I: int, V: int, layers: int, seed: int):
    """A small random Hugging Face Qwen2ForCausalLM in float32 (eager attention, rope theta
    1e6, untied lm_head) with non-zero q/k/v biases and non-unit norm weights, so every term
    of the decoder is exercised."""
    import transformers

    torch.manual_seed(seed)
    cfg = transformers.Qwen2Config(vocab_size=V, hidden_size=H, intermediate_size=I,
                                   num_hidden_layers=layers, num_attention_heads=n_heads,
                                   num_key_value_heads=n_kv, max_position_embeddings=4096,
                                   rope_theta=1000000.0, rms_norm_eps=1e-6,
                                   tie_word_embeddings=False)
    cfg._attn_implementation = "eager"
    m = transformers.Qwen2ForCausalLM(cfg).float().eval()
    with torch.no_grad():
        for layer in m.model.layers:
            at = layer.self_attn
            for b in (at.q_proj.bias, at.k_proj.bias, at.v_proj.bias):
                b.normal_(0, 0.1)
            for ln in (layer.input_layernorm, layer.post_attention_layernorm):
                ln.weight.copy_(1 + 0.05 * torch.randn(H))
        m.model.norm.weight.copy_(1 + 0.05 * torch.randn(H))
    return m
