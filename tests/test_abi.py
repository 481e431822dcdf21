"""CPU-only checks of the C-ABI boundary (no GPU): the library loads without a GPU, exports
exactly what include/*.h declare, and rejects every invalid argument with the reference's
return codes (csrc/nanoserve_ops.cu:20-90) before touching HIP."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

from nanoserve_amd import LIB_PATH, Kernels
from nanoserve_amd.ops import SIGNATURES

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h)
           for h in ("nanoserve_w4.h", "nanoserve_decode.h", "nanoserve_probe.h")]


def declared_symbols():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(?:int|size_t)\s+(ns_\w+)\s*\(", text))
    return sorted(names)


def test_headers_are_all_listed():
    assert sorted(os.listdir(os.path.join(ROOT, "include"))) == sorted(
        os.path.basename(h) for h in HEADERS)


def test_header_declares_the_reference_entry_points():
    # the reference's W4 and fused-op entry points (csrc/nanoserve_ops.cu:20-90), plus the
    # decode-step attention operators the reference does with PyTorch ops
    assert declared_symbols() == sorted([
        "ns_w4_linear", "ns_w4_quantize", "ns_w4_repack", "ns_w4_linear_packed",
        "ns_w4_linear_packed_swiglu",
        "ns_rmsnorm", "ns_rope", "ns_swiglu",
        "ns_decode_qkv", "ns_decode_attention_workspace", "ns_decode_attention",
        "ns_decode_qkv_attention", "ns_w4_gemv_decode", "ns_w4_gemv_decode_attn", "ns_decode_embed",
        "ns_bf16_gemv", "ns_w4_gptq_workspace", "ns_w4_gptq", "ns_w4_linear_swiglu",
        "ns_probe_read", "ns_probe_empty", "ns_probe_linear_loop", "ns_decode_attention_noalloc",
        "ns_w4_linear_workspace", "ns_w4_linear_ws"])


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


# ------------------------------------------------------------------ decoder-step operators
def test_rmsnorm_rejects_bad_arguments(k):
    assert k.lib.ns_rmsnorm(P, None, P, P, 1, 12, 1e-6, None) == -1        # H % 8
    assert k.lib.ns_rmsnorm(P, None, P, P, 1, 8200, 1e-6, None) == -1      # H > 8192
    assert k.lib.ns_rmsnorm(P, None, P, P, -1, 64, 1e-6, None) == -1
    assert k.lib.ns_rmsnorm(None, None, P, P, 1, 64, 1e-6, None) == -1
    assert k.lib.ns_rmsnorm(P + 2, None, P, P, 1, 64, 1e-6, None) == -1
    assert k.lib.ns_rmsnorm(P, P + 8, P, P, 1, 64, 1e-6, None) == -1
    assert k.lib.ns_rmsnorm(P, None, P, P, 0, 64, 1e-6, None) == 0


def test_rope_rejects_bad_arguments(k):
    assert k.lib.ns_rope(P, P, P, 1, 2, 1, 72, 0, -1, -1, None) == -1       # D % 16
    assert k.lib.ns_rope(P, P, P, 1, 2, 1, 128, 0, 260, -1, None) == -1     # stride % 8
    assert k.lib.ns_rope(P, P, P, -1, 2, 1, 128, 0, -1, -1, None) == -1
    assert k.lib.ns_rope(None, P, P, 1, 2, 1, 128, 0, -1, -1, None) == -1
    assert k.lib.ns_rope(P, P + 8, P, 1, 2, 1, 128, 0, -1, -1, None) == -1
    assert k.lib.ns_rope(P, P, P, 0, 2, 1, 128, 0, -1, -1, None) == 0


def test_swiglu_rejects_bad_arguments(k):
    assert k.lib.ns_swiglu(P, P, P, 1, 12, None) == -1                      # T*I % 8
    assert k.lib.ns_swiglu(P, P, P, -1, 8, None) == -1
    assert k.lib.ns_swiglu(P, P + 4, P, 1, 8, None) == -1
    assert k.lib.ns_swiglu(None, None, None, 0, 8, None) == 0


def test_decode_qkv_rejects_bad_arguments(k):
    assert k.lib.ns_decode_qkv(P, None, P, P, P, P, 28, 4, 72, 64, None) == -2
    assert k.lib.ns_decode_qkv(P, None, P, P, P, P, 0, 4, 128, 64, None) == -2
    assert k.lib.ns_decode_qkv(P, None, P, P, P, P, 28, 4, 128, 0, None) == -2
    assert k.lib.ns_decode_qkv(P, None, P, None, P, P, 28, 4, 128, 64, None) == -2
    assert k.lib.ns_decode_qkv(P, P + 2, P, P, P, P, 28, 4, 128, 64, None) == -2


def test_linear_workspace_sizes_and_rejects(k):
    """The K-split workspace is needed only by the M = 2..8 GEMV past 32 pairs (K > 8192) and is
    ks * M * N fp32 partials, ks = ceil(K / 8192); ns_w4_linear_ws rejects a missing, short or
    misaligned workspace before any HIP call."""
    ws = k.lib.ns_w4_linear_workspace
    assert ws(8, 3584, 18944, 128) == 3 * 8 * 3584 * 4
    assert ws(2, 1536, 8960, 128) == 2 * 2 * 1536 * 4
    assert ws(4, 4104, 16384, 128) == 2 * 4 * 4104 * 4
    assert ws(8, 3584, 8192, 128) == 0      # 32 pairs: one pass
    assert ws(1, 3584, 18944, 128) == 0     # M = 1 kernel
    assert ws(9, 3584, 18944, 128) == 0     # not a GEMV shape
    assert ws(128, 3584, 18944, 128) == 0   # GEMM
    assert ws(8, 3584, 18944, 64) == 0      # generic GEMV (G % 128 != 0)
    assert ws(8, 3584, 18944, 100) == 0     # invalid format
    assert ws(0, 3584, 18944, 128) == 0
    P = 1 << 20
    need = ws(8, 64, 18944, 128)
    call = k.lib.ns_w4_linear_ws
    assert call(P, P, P, P, 8, 64, 18944, 128, None, need, None) == -2
    assert call(P, P, P, P, 8, 64, 18944, 128, P, need - 4, None) == -2
    assert call(P, P, P, P, 8, 64, 18944, 128, P + 8, need, None) == -2
    # shapes ns_w4_linear rejects are rejected the same way, workspace or not
    assert call(P, P, P, P, 9, 64, 18944, 128, P, need, None) == -2
    assert call(P, P, P, P, 8, 64, 18944, 100, P, need, None) == -2


def test_decode_attention_workspace_and_rejects(k):
    ws = k.lib.ns_decode_attention_workspace(28, 4, 128, 1024)
    assert ws == 8 * 28 * 130 * 4  # 128-row splits x heads x (D + max + sum) floats
    assert k.lib.ns_decode_attention_workspace(28, 4, 64, 1024) == 0
    assert k.lib.ns_decode_attention_workspace(28, 4, 128, 0) == 0
    assert k.lib.ns_decode_attention_workspace(28, 0, 128, 64) == 0

    def call(work_bytes=ws, Hq=28, Hk=4, D=128, L=1024, q=P, work=P):
        return k.lib.ns_decode_attention(q, P, P, P, P, work, work_bytes, Hq, Hk, D, L, None)

    assert call(work_bytes=ws - 1) == -2
    assert call(D=64) == -2
    assert call(Hq=27) == -2                   # Hq % Hk
    assert call(Hq=36, Hk=4) == -2             # more than 8 query heads per kv head
    assert call(L=0) == -2
    assert call(q=None) == -2
    assert call(work=P + 4) == -2

    def fused(work_bytes=ws, Hq=28, Hk=4, D=128, L=1024, qkv=P, work=P, rot=None):
        return k.lib.ns_decode_qkv_attention(qkv, None, P, P, P, P, P, work, work_bytes, Hq, Hk,
                                             D, L, 1, rot, None)

    assert fused(work_bytes=ws - 1) == -2
    assert fused(D=64) == -2
    assert fused(Hq=36) == -2
    assert fused(qkv=None) == -2
    assert fused(qkv=P + 8) == -2
    assert fused(work=None) == -2
    assert fused(rot=P + 4) == -2               # the rotation table is read 16 bytes at a time


def test_runner_split_rows_match_library(k):
    """The runner's rows per attention split (it picks where the o GEMV stops merging the
    splits by it) are the library's: the workspace grows by one split every that many rows."""
    from nanoserve_amd.qwen import ATTN_SPLIT_ROWS

    ws = k.lib.ns_decode_attention_workspace
    assert ws(28, 4, 128, 1) == ws(28, 4, 128, ATTN_SPLIT_ROWS)
    assert ws(28, 4, 128, ATTN_SPLIT_ROWS + 1) == 2 * ws(28, 4, 128, ATTN_SPLIT_ROWS)


def test_decode_embed_rejects(k):
    """ns_decode_embed checks its sizes and pointers before any HIP call."""
    def call(vocab=1000, H=3584, D=128, tok=P, pos=P, embed=P, x=P, rot=P):
        return k.lib.ns_decode_embed(tok, pos, embed, vocab, H, P, D, x, rot, None)

    assert call(vocab=0) == -2
    assert call(H=0) == -2
    assert call(H=3583) == -2
    assert call(D=120) == -2
    assert call(D=1024) == -2
    for name in ("tok", "pos", "embed", "x", "rot"):
        assert call(**{name: None}) == -2, name
    assert call(embed=P + 8) == -2
    assert call(x=P + 8) == -2
    assert call(rot=P + 4) == -2
    assert call(tok=P + 2) == -2


def test_decode_attention_noalloc_rejects(k):
    """The allocation-free attention takes the workspace's checks from its sizes: beyond its
    4 MiB scratch (at Hq = 28: max_len > 36864) it returns -2, as for any other rejected shape
    or pointer, without touching HIP."""
    def call(Hq=28, Hk=4, D=128, L=1024, q=P, out=P):
        return k.lib.ns_decode_attention_noalloc(q, P, P, P, out, Hq, Hk, D, L, None)

    assert k.lib.ns_decode_attention_workspace(28, 4, 128, 36864) <= 4 << 20
    assert k.lib.ns_decode_attention_workspace(28, 4, 128, 36865) > 4 << 20
    assert call(L=36865) == -2
    assert call(Hq=64, Hk=8, L=16129) == -2     # 127 splits x 64 heads x 130 floats > 4 MiB
    assert call(D=64) == -2
    assert call(Hq=27) == -2
    assert call(Hq=36, Hk=4) == -2
    assert call(L=0) == -2
    assert call(q=None) == -2
    assert call(q=P + 8) == -2
    assert call(out=None) == -2


def test_gemv_decode_rejects_bad_arguments(k):
    def call(X=P, res=None, r=None, nw=None, res_out=None, N=64, K=256, G=128, swiglu=0):
        return k.lib.ns_w4_gemv_decode(X, res, r, nw, 1e-6, res_out, P, P, P, N, K, G, swiglu,
                                       None)

    assert call(G=64) == -2
    assert call(K=192) == -2                       # K % 128
    assert call(N=0) == -2
    assert call(X=None) == -2                      # no activation
    assert call(res=P) == -2                       # norm without weight
    assert call(res=P, nw=P, K=16512) == -2        # norm row longer than 16384
    assert call(N=40, swiglu=1) == -2              # SwiGLU pairs need N % 16 == 0
    assert call(X=P + 8) == -2
    assert call(res=P, nw=P, r=P + 0x1000, res_out=P) == -2  # res_out aliases res


def test_gemv_decode_attn_rejects_bad_arguments(k):
    def call(a=P, work=P, pos=P, L=1024, Hq=28, N=64, K=3584, G=128):
        return k.lib.ns_w4_gemv_decode_attn(a, work, pos, L, Hq, P, P, P, N, K, G, None)

    assert call(K=3456) == -2          # K != Hq * 128
    assert call(G=64) == -2
    assert call(L=0) == -2
    assert call(work=None) == -2
    assert call(pos=None) == -2
    assert call(a=P + 8) == -2


def test_bf16_gemv_rejects_bad_arguments(k):
    def call(X=P, res=None, nw=None, N=64, K=256, W=P):
        return k.lib.ns_bf16_gemv(X, res, None, nw, 1e-6, W, P, N, K, None)

    assert call(K=100) == -2          # K % 8
    assert call(K=8200) == -2         # K > 8192
    assert call(N=0) == -2
    assert call(X=None) == -2
    assert call(res=P) == -2          # norm without weight
    assert call(W=P + 8) == -2


def test_packed_entry_points_reject_bad_arguments(k):
    assert k.lib.ns_w4_repack(P, P, P, P, 64, 256, 64, None) == -2      # G != 128
    assert k.lib.ns_w4_repack(P, P, P, P, 64, 200, 128, None) == -2     # K % 128
    assert k.lib.ns_w4_repack(P, P, P + 8, P, 64, 256, 128, None) == -2
    # M > 16 (the packed GEMM) past 31-bit activation offsets: (M + 256) K * 2 >= 2^31
    assert k.lib.ns_w4_linear_packed(P, P, P, P, 17, 64, 3933184, 128, None) == -2
    assert k.lib.ns_w4_linear_packed(P, P, P, P, 0, 64, 256, 128, None) == -2
    assert k.lib.ns_w4_linear_packed(P, P, P, P, 2, 64, 20608, 128, None) == -2  # K > 20480
    assert k.lib.ns_w4_linear_packed(P, P, P, P, 1, 64, 256, 128, None) == -2    # M = 1: ns_w4_linear
    assert k.lib.ns_w4_linear_packed(P + 8, P, P, P, 2, 64, 256, 128, None) == -2
    # the SwiGLU GEMM: prefill only, gate/up rows in blocks of 8
    assert k.lib.ns_w4_linear_packed_swiglu(P, P, P, P, 16, 64, 256, 128, None) == -2  # M <= 16
    assert k.lib.ns_w4_linear_packed_swiglu(P, P, P, P, 32, 72, 256, 128, None) == -2  # N % 16
    assert k.lib.ns_w4_linear_packed_swiglu(P, P, P, P, 32, 64, 200, 128, None) == -2  # K % 128
    assert k.lib.ns_w4_linear_packed_swiglu(P, P, P, P, 32, 64, 256, 64, None) == -2   # G != 128
    assert k.lib.ns_w4_linear_packed_swiglu(P, P, P, P, 17, 64, 3933184, 128, None) == -2
    assert k.lib.ns_w4_linear_packed_swiglu(P, P + 8, P, P, 32, 64, 256, 128, None) == -2


def test_gptq_workspace_and_rejects(k):
    assert k.lib.ns_w4_gptq_workspace(0) == 0
    assert k.lib.ns_w4_gptq_workspace(-3) == 0
    assert k.lib.ns_w4_gptq_workspace(37888) == 128 * 37888 * 4
    ws = 128 * 64 * 4
    assert k.lib.ns_w4_gptq(P, P, P, P, P, ws, 64, 256, 64, None) == -2      # G != 128
    assert k.lib.ns_w4_gptq(P, P, P, P, P, ws, 64, 200, 128, None) == -2     # K % 128
    assert k.lib.ns_w4_gptq(P, P, P, P, P, ws, 0, 256, 128, None) == -2      # N <= 0
    assert k.lib.ns_w4_gptq(P, P, P, P, P, ws - 4, 64, 256, 128, None) == -2  # small workspace
    assert k.lib.ns_w4_gptq(P + 8, P, P, P, P, ws, 64, 256, 128, None) == -2  # W misaligned
    assert k.lib.ns_w4_gptq(P, P + 4, P, P, P, ws, 64, 256, 128, None) == -2  # U misaligned
    assert k.lib.ns_w4_gptq(P, P, P, P, None, ws, 64, 256, 128, None) == -2


def test_linear_swiglu_rejects(k):
    f = k.lib.ns_w4_linear_swiglu
    assert f(P, P, P, P, 128, 264, 256, 128, None) == -2     # N % 16
    assert f(P, P, P, P, 4, 256, 256, 128, None) == -2       # M not 1 or a multiple of 128
    assert f(P, P, P, P, 128, 272, 256, 128, None) == -2     # GEMM needs N % 128
    assert f(P, P, P, P, 128, 256, 288, 32, None) == -2      # GEMM needs K % 64
    assert f(P, P, P, P, 128, 256, 384, 96, None) == -2      # G not a power of two
    assert f(P, P, P, P, 1, 256, 256, 64, None) == -2        # GEMV needs G == 128
    assert f(P + 8, P, P, P, 128, 256, 256, 128, None) == -2
    assert f(P, P, P, None, 128, 256, 256, 128, None) == -2
