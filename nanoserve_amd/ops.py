"""ctypes bindings to libnanoserve_amd.so: the W4A16 part of the reference's ``Kernels`` class
(Uttaprexa/nanoserve python/nanoserve/ops.py:15-39, 76-97), same method names, argument
meaning, return values and exceptions.

The library is loaded with ctypes exactly as the reference loads build/libnanoserve.so; loading
needs no GPU. There is no CPU fallback: a missing library raises at construction, and tensors
that are not on the GPU raise before any native call.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnanoserve_amd.so")

# Exported symbols and their ctypes signatures (include/nanoserve_w4.h,
# include/nanoserve_decode.h, include/nanoserve_probe.h); every function returns int except
# where RESTYPES says otherwise.
_VP, _I32, _I64, _F32, _SZ = (ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float,
                              ctypes.c_size_t)
SIGNATURES = {
    "ns_w4_quantize": [_VP, _VP, _VP, _I32, _I32, _I32, _VP],
    "ns_w4_linear": [_VP, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP],
    "ns_rmsnorm": [_VP, _VP, _VP, _VP, _I32, _I32, _F32, _VP],
    "ns_rope": [_VP, _VP, _VP, _I32, _I32, _I32, _I32, _I32, _I64, _I64, _VP],
    "ns_swiglu": [_VP, _VP, _VP, _I32, _I32, _VP],
    "ns_decode_qkv": [_VP, _VP, _VP, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP],
    "ns_decode_attention_workspace": [_I32, _I32, _I32, _I32],
    "ns_decode_attention": [_VP, _VP, _VP, _VP, _VP, _VP, _SZ, _I32, _I32, _I32, _I32, _VP],
    "ns_decode_qkv_attention": [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _SZ, _I32, _I32, _I32,
                                _I32, _I32, _VP, _VP],
    "ns_decode_embed": [_VP, _VP, _VP, _I32, _I32, _VP, _I32, _VP, _VP, _VP],
    "ns_w4_gemv_decode_attn": [_VP, _VP, _VP, _I32, _I32, _VP, _VP, _VP, _I32, _I32, _I32, _VP],
}
SIGNATURES["ns_w4_gemv_decode"] = [_VP, _VP, _VP, _VP, _F32, _VP, _VP, _VP, _VP, _I32, _I32, _I32,
                                   _I32, _VP]
SIGNATURES["ns_bf16_gemv"] = [_VP, _VP, _VP, _VP, _F32, _VP, _VP, _I32, _I32, _VP]
SIGNATURES["ns_w4_repack"] = [_VP, _VP, _VP, _VP, _I32, _I32, _I32, _VP]
SIGNATURES["ns_w4_linear_packed"] = [_VP, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP]
SIGNATURES["ns_w4_linear_packed_swiglu"] = [_VP, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP]
SIGNATURES["ns_w4_linear_swiglu"] = [_VP, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP]
SIGNATURES["ns_w4_linear_workspace"] = [_I32, _I32, _I32, _I32]
SIGNATURES["ns_w4_linear_ws"] = [_VP, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP, _SZ, _VP]
SIGNATURES["ns_w4_gptq_workspace"] = [_I32]
SIGNATURES["ns_w4_gptq"] = [_VP, _VP, _VP, _VP, _VP, _SZ, _I32, _I32, _I32, _VP]
SIGNATURES["ns_decode_attention_noalloc"] = [_VP, _VP, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _VP]
SIGNATURES["ns_probe_read"] = [_VP, _SZ, _VP, _I32, _I32, _I32, _VP]
SIGNATURES["ns_probe_empty"] = [_I32, _I32, _VP]
SIGNATURES["ns_probe_linear_loop"] = [_VP] * 7 + [_I32, _I32, _VP]
RESTYPES = {"ns_decode_attention_workspace": _SZ, "ns_w4_gptq_workspace": _SZ,
            "ns_w4_linear_workspace": _SZ}


if hasattr(torch._C, "_cuda_getCurrentRawStream"):
    _raw_stream = torch._C._cuda_getCurrentRawStream
else:  # pragma: no cover - older torch builds
    def _raw_stream(device):
        return torch.cuda.current_stream(device).cuda_stream


def _require_gpu_tensor(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got device {t.device})")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")


def _rot_ptr(rot, head_dim):
    _require_gpu_tensor(rot, "rot", torch.float32)
    if not rot.is_contiguous() or rot.numel() != head_dim:
        raise ValueError("rot must be a contiguous [2, head_dim / 2] float32 tensor")
    return rot.data_ptr()


def _check_out(out: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    _require_gpu_tensor(out, "out", like.dtype)
    if out.shape != like.shape or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous tensor of shape {tuple(like.shape)}")
    return out


class Kernels:
    """W4A16 kernels through the C ABI. ``path`` defaults to the in-tree library."""

    def __init__(self, path: str = LIB_PATH):
        path = os.path.abspath(path)
        if not os.path.exists(path):
            raise OSError(f"{path} not found: build it with `python -m nanoserve_amd.build` "
                          "(there is no CPU fallback)")
        self.lib = ctypes.CDLL(path)
        for name, args in SIGNATURES.items():
            fn = getattr(self.lib, name)
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, ctypes.c_int)

    # reference ops.py:32-34: the current torch stream (a hipStream_t on ROCm), read as a raw
    # handle (no Stream object per call: the eager launch path runs this for every operator)
    @staticmethod
    def _stream():
        return ctypes.c_void_p(_raw_stream(torch.cuda.current_device()))

    # reference ops.py:36-39
    @staticmethod
    def _check(rc: int, name: str):
        if rc != 0:
            raise RuntimeError(f"{name} failed with code {rc}")

    def w4_quantize(self, W, group=128):
        """W [N, K] bf16 -> (Wq int32 [N, K // 8], S bf16 [N, K // group]). Reference
        ops.py:76-83 (kernel: kernels/quant/w4a16.cuh:272-301)."""
        _require_gpu_tensor(W, "W", torch.bfloat16)
        N, K = W.shape
        Wq = torch.empty((N, K // 8), dtype=torch.int32, device=W.device)
        S = torch.empty((N, K // group), dtype=torch.bfloat16, device=W.device)
        W = W.contiguous()
        rc = self.lib.ns_w4_quantize(W.data_ptr(), Wq.data_ptr(), S.data_ptr(), N, K, group,
                                     self._stream())
        self._check(rc, "ns_w4_quantize")
        return Wq, S

    def w4_linear_swiglu(self, x, Wq, S, group=128, out=None):
        """x [M, K] bf16 -> [M, N // 2] bf16 = swiglu of x @ deq(Wq, S)^T whose rows are gate and
        up rows interleaved in blocks of 8 (``qwen.interleave_gate_up``): one launch for M = 1
        and M % 128 == 0 (ns_w4_linear_swiglu). Other M pad with zero rows to a multiple of 128
        above 8, and run as ``w4_linear`` + ``swiglu`` for M = 2..8 (not in the reference,
        whose MLP is swiglu(linear(h, "g"), linear(h, "u")), qwen.py:159)."""
        _require_gpu_tensor(x, "x", torch.bfloat16)
        _require_gpu_tensor(Wq, "Wq", torch.int32)
        _require_gpu_tensor(S, "S", torch.bfloat16)
        M, K = x.shape
        N = Wq.shape[0]
        if N % 16:
            raise ValueError("the interleaved gate/up matrix needs N % 16 == 0")
        I = N // 2
        if out is not None:
            _require_gpu_tensor(out, "out", torch.bfloat16)
            if tuple(out.shape) != (M, I) or not out.is_contiguous():
                raise ValueError(f"out must be a contiguous tensor of shape {(M, I)}")
        if M == 0:
            return out if out is not None else x.new_empty((0, I))
        if 2 <= M <= 8:
            gu = self.w4_linear(x, Wq, S, group).view(M, I // 8, 2, 8)
            return self.swiglu(gu[:, :, 0].reshape(M, I), gu[:, :, 1].reshape(M, I), out=out)
        Mp = M if M == 1 else ((M + 127) // 128) * 128
        if Mp != M:
            x = torch.cat([x, x.new_zeros(Mp - M, K)])
        x = x.contiguous()
        y = out if out is not None and Mp == M else torch.empty((Mp, I), dtype=torch.bfloat16,
                                                                 device=x.device)
        rc = self.lib.ns_w4_linear_swiglu(x.data_ptr(), Wq.contiguous().data_ptr(),
                                          S.contiguous().data_ptr(), y.data_ptr(), Mp, N, K,
                                          group, self._stream())
        self._check(rc, "ns_w4_linear_swiglu")
        if Mp != M:
            y = y[:M]
            if out is not None:
                out.copy_(y)
                return out
        return y

    def w4_gptq(self, W, U, group=128):
        """Calibrated quantization (not in the reference, whose README.md:233-235 names it as
        the next step): W [N, K] (any float dtype) and U [K, K] fp32, the upper Cholesky factor
        of the layer's damped inverse Hessian (``nanoserve_amd.gptq.hessian_factor``) ->
        (Wq int32 [N, K // 8], S bf16 [N, K // group]) in w4_quantize's format. W is not
        modified (the kernels work on an fp32 copy)."""
        if not isinstance(W, torch.Tensor) or not W.is_cuda:
            raise ValueError("W must be a CUDA (HIP) tensor")
        _require_gpu_tensor(U, "U", torch.float32)
        N, K = W.shape
        if tuple(U.shape) != (K, K):
            raise ValueError(f"U must be [{K}, {K}], got {tuple(U.shape)}")
        Wf = W.to(torch.float32).contiguous().clone()
        U = U.contiguous()
        Wq = torch.empty((N, K // 8), dtype=torch.int32, device=W.device)
        S = torch.empty((N, K // group), dtype=torch.bfloat16, device=W.device)
        nbytes = self.lib.ns_w4_gptq_workspace(N)
        work = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=W.device)
        rc = self.lib.ns_w4_gptq(Wf.data_ptr(), U.data_ptr(), Wq.data_ptr(), S.data_ptr(),
                                 work.data_ptr(), work.numel(), N, K, group, self._stream())
        self._check(rc, "ns_w4_gptq")
        return Wq, S

    def w4_linear_workspace(self, M, N, K, group=128, device=None):
        """A uint8 device tensor of the workspace ``w4_linear(..., work=)`` uses for this shape
        (the K split of the M = 2..8 GEMV for K > 8192), or None when the shape needs none."""
        n = int(self.lib.ns_w4_linear_workspace(M, N, K, group))
        return torch.empty(n, dtype=torch.uint8, device=device or "cuda") if n else None

    def w4_linear(self, x, Wq, S, group=128, out=None, work=None):
        """x [M, K] bf16 -> y [M, N] bf16 = x @ deq(Wq, S)^T. Reference ops.py:85-97.

        M <= 8 runs natively (the reference pads 3 -> 4 and 5..7 -> 8 with zero rows, which
        does not change any output row); larger M is padded with zero rows up to a multiple
        of 128, as the reference does. ``out`` (not in the reference): a contiguous [M, N]
        bf16 tensor to write instead of a new one, for M that needs no padding. ``work`` (not in
        the reference): a workspace from ``w4_linear_workspace``; with it the M = 2..8 GEMV
        may split long rows over K (ns_w4_linear_ws), without it no shape is split
        (ns_w4_linear)."""
        _require_gpu_tensor(x, "x", torch.bfloat16)
        _require_gpu_tensor(Wq, "Wq", torch.int32)
        _require_gpu_tensor(S, "S", torch.bfloat16)
        M, K = x.shape
        N = Wq.shape[0]
        Mp = M if M <= 8 else ((M + 127) // 128) * 128
        if M == 0:
            Mp = 1
        if Mp != M:
            x = torch.cat([x, x.new_zeros(Mp - M, K)])
        x = x.contiguous()
        Wq = Wq.contiguous()
        S = S.contiguous()
        if out is not None:
            _require_gpu_tensor(out, "out", torch.bfloat16)
            if Mp != M or tuple(out.shape) != (M, N) or not out.is_contiguous():
                raise ValueError(f"out must be a contiguous [{M}, {N}] tensor and M must need "
                                 "no padding")
            y = out
        else:
            y = torch.empty((Mp, N), dtype=torch.bfloat16, device=x.device)
        if work is None:
            rc = self.lib.ns_w4_linear(x.data_ptr(), Wq.data_ptr(), S.data_ptr(), y.data_ptr(), Mp,
                                       N, K, group, self._stream())
            self._check(rc, "ns_w4_linear")
        else:
            _require_gpu_tensor(work, "work", torch.uint8)
            rc = self.lib.ns_w4_linear_ws(x.data_ptr(), Wq.data_ptr(), S.data_ptr(), y.data_ptr(),
                                          Mp, N, K, group, work.data_ptr(), work.numel(),
                                          self._stream())
            self._check(rc, "ns_w4_linear_ws")
        return y if Mp == M else y[:M]

    # ------------------------------------------------------------------ decoder-step operators
    def rmsnorm(self, x, r, w, eps, out=None):
        """x [T, H] residual stream, updated in place to x + r when r is given; returns
        rmsnorm(x) * w. Reference ops.py:41-48 (kernel: kernels/fused/rmsnorm.cuh:10-52).
        ``out`` (not in the reference): a contiguous tensor like x to write the result to."""
        _require_gpu_tensor(x, "x", torch.bfloat16)
        _require_gpu_tensor(w, "w", torch.bfloat16)
        if not x.is_contiguous():
            raise ValueError("x must be contiguous (it is updated in place)")
        if r is not None:
            _require_gpu_tensor(r, "r", torch.bfloat16)
            r = r.contiguous()
        y = torch.empty_like(x) if out is None else _check_out(out, x)
        rc = self.lib.ns_rmsnorm(x.data_ptr(), None if r is None else r.data_ptr(),
                                 w.contiguous().data_ptr(), y.data_ptr(), x.shape[0], x.shape[1],
                                 eps, self._stream())
        self._check(rc, "ns_rmsnorm")
        return y

    def rope(self, q, k, inv_freq, n_heads, n_kv_heads, head_dim, pos0):
        """In place on q [T, Hq*D] and k [T, Hk*D] (row stride may exceed Hq*D / Hk*D).
        Reference ops.py:50-54 (kernel: kernels/fused/rope.cuh:14-46)."""
        _require_gpu_tensor(q, "q", torch.bfloat16)
        _require_gpu_tensor(k, "k", torch.bfloat16)
        _require_gpu_tensor(inv_freq, "inv_freq", torch.float32)
        for t, n in ((q, "q"), (k, "k")):
            if t.stride(-1) != 1:
                raise ValueError(f"{n} rows must be contiguous")
        rc = self.lib.ns_rope(q.data_ptr(), k.data_ptr(), inv_freq.contiguous().data_ptr(),
                              q.shape[0], n_heads, n_kv_heads, head_dim, pos0, q.stride(0),
                              k.stride(0), self._stream())
        self._check(rc, "ns_rope")

    def swiglu(self, gate, up, out=None):
        """silu(gate) * up, gate and up contiguous [T, I]. Reference ops.py:56-62 (kernel:
        kernels/fused/swiglu.cuh:35-52). ``out`` (not in the reference): a contiguous tensor
        like gate to write the result to."""
        _require_gpu_tensor(gate, "gate", torch.bfloat16)
        _require_gpu_tensor(up, "up", torch.bfloat16)
        if not (gate.is_contiguous() and up.is_contiguous()):
            raise ValueError("gate and up must be contiguous")
        out = torch.empty_like(gate) if out is None else _check_out(out, gate)
        rc = self.lib.ns_swiglu(gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.shape[0],
                                gate.shape[1], self._stream())
        self._check(rc, "ns_swiglu")
        return out

    def decode_qkv(self, qkv, bias, inv_freq, pos, k_cache, v_cache, n_heads, n_kv_heads,
                   head_dim):
        """One decode token: bias add + RoPE at position pos[0] (device int32) in place on the
        fused projection output qkv [(Hq + 2Hk) * D], and the k / v heads appended to one
        layer's cache slices k_cache / v_cache [Hk, max_len, D]. The reference does these
        steps with PyTorch ops (qwen.py:119-122, 147-151)."""
        _require_gpu_tensor(qkv, "qkv", torch.bfloat16)
        _require_gpu_tensor(inv_freq, "inv_freq", torch.float32)
        _require_gpu_tensor(pos, "pos", torch.int32)
        for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
            _require_gpu_tensor(t, n, torch.bfloat16)
            if not t.is_contiguous():
                raise ValueError(f"{n} must be contiguous")
        if bias is not None:
            _require_gpu_tensor(bias, "bias", torch.bfloat16)
        if not qkv.is_contiguous():
            raise ValueError("qkv must be contiguous")
        rc = self.lib.ns_decode_qkv(qkv.data_ptr(), None if bias is None else bias.data_ptr(),
                                    inv_freq.data_ptr(), pos.data_ptr(), k_cache.data_ptr(),
                                    v_cache.data_ptr(), n_heads, n_kv_heads, head_dim,
                                    k_cache.shape[-2], self._stream())
        self._check(rc, "ns_decode_qkv")

    def decode_attention_workspace(self, n_heads, n_kv_heads, head_dim, max_len, device=None):
        """A uint8 device tensor of the workspace decode_attention and decode_qkv_attention
        need (per-split partial results). Launches that may overlap in time need workspaces of
        their own."""
        n = int(self.lib.ns_decode_attention_workspace(n_heads, n_kv_heads, head_dim, max_len))
        if n == 0:
            raise ValueError("unsupported attention sizes (head_dim must be 128)")
        return torch.zeros(n, dtype=torch.uint8, device=device or "cuda")

    def decode_attention(self, q, k_cache, v_cache, pos, n_heads, n_kv_heads, head_dim,
                         work, out=None):
        """Attention of one query token q [Hq * D] over cache rows 0 .. pos[0] of one layer's
        k_cache / v_cache [Hk, max_len, D]; returns out [1, Hq * D] bf16. The reference uses
        PyTorch SDPA for this (qwen.py:124-133). work: from decode_attention_workspace."""
        _require_gpu_tensor(q, "q", torch.bfloat16)
        _require_gpu_tensor(pos, "pos", torch.int32)
        _require_gpu_tensor(work, "work", torch.uint8)
        if out is None:
            out = torch.empty((1, n_heads * head_dim), dtype=torch.bfloat16, device=q.device)
        rc = self.lib.ns_decode_attention(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                          pos.data_ptr(), out.data_ptr(), work.data_ptr(),
                                          work.numel(), n_heads, n_kv_heads, head_dim,
                                          k_cache.shape[-2], self._stream())
        self._check(rc, "ns_decode_attention")
        return out

    def decode_attention_noalloc(self, q, k_cache, v_cache, pos, n_heads, n_kv_heads, head_dim,
                                 out):
        """decode_attention without a workspace, for callers that cannot allocate: the partials
        go to the library's per-GPU scratch (include/nanoserve_decode.h), so calls that overlap
        on one GPU race. ``out`` [1, Hq * D] bf16 is required (nothing is allocated here)."""
        _require_gpu_tensor(q, "q", torch.bfloat16)
        _require_gpu_tensor(pos, "pos", torch.int32)
        _require_gpu_tensor(out, "out", torch.bfloat16)
        rc = self.lib.ns_decode_attention_noalloc(q.data_ptr(), k_cache.data_ptr(),
                                                  v_cache.data_ptr(), pos.data_ptr(),
                                                  out.data_ptr(), n_heads, n_kv_heads, head_dim,
                                                  k_cache.shape[-2], self._stream())
        self._check(rc, "ns_decode_attention_noalloc")
        return out

    def decode_qkv_attention(self, qkv, bias, inv_freq, pos, k_cache, v_cache, n_heads,
                             n_kv_heads, head_dim, work, out=None, merge=True, rot=None):
        """decode_qkv followed by decode_attention in one launch, qkv left unchanged: bias +
        RoPE of the q heads, the token's k / v row appended to the cache at pos[0], attention
        over rows 0 .. pos[0]. Returns out [1, Hq * D] bf16. With ``merge=False`` the split
        partials stay in ``work`` for gemv_decode_attn (out is written only for one split).
        ``rot``: the step's rotation table from ``decode_embed`` (same outputs, fewer
        instructions per workgroup)."""
        _require_gpu_tensor(qkv, "qkv", torch.bfloat16)
        _require_gpu_tensor(inv_freq, "inv_freq", torch.float32)
        _require_gpu_tensor(pos, "pos", torch.int32)
        _require_gpu_tensor(work, "work", torch.uint8)
        for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
            _require_gpu_tensor(t, n, torch.bfloat16)
            if not t.is_contiguous():
                raise ValueError(f"{n} must be contiguous")
        if bias is not None:
            _require_gpu_tensor(bias, "bias", torch.bfloat16)
        if not qkv.is_contiguous():
            raise ValueError("qkv must be contiguous")
        if out is None:
            out = torch.empty((1, n_heads * head_dim), dtype=torch.bfloat16, device=qkv.device)
        rc = self.lib.ns_decode_qkv_attention(
            qkv.data_ptr(), None if bias is None else bias.data_ptr(), inv_freq.data_ptr(),
            pos.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(),
            work.data_ptr(), work.numel(), n_heads, n_kv_heads, head_dim, k_cache.shape[-2],
            1 if merge else 0, None if rot is None else _rot_ptr(rot, head_dim), self._stream())
        self._check(rc, "ns_decode_qkv_attention")
        return out

    def decode_embed(self, tok, pos, embed, inv_freq, x=None, rot=None):
        """Start of a decode step (no counterpart in the reference, whose runner gathers the
        row with F.embedding, qwen.py:141): x [1, H] = embed[tok[0]] (zeros for an id outside
        the table) and rot [2, D/2] fp32 = cos, sin of pos[0] * inv_freq, the table
        decode_qkv_attention takes. Returns (x, rot)."""
        _require_gpu_tensor(tok, "tok", torch.int32)
        _require_gpu_tensor(pos, "pos", torch.int32)
        _require_gpu_tensor(embed, "embed", torch.bfloat16)
        _require_gpu_tensor(inv_freq, "inv_freq", torch.float32)
        if not embed.is_contiguous() or embed.dim() != 2:
            raise ValueError("embed must be a contiguous [vocab, H] tensor")
        vocab, H = embed.shape
        D = 2 * inv_freq.numel()
        if x is None:
            x = torch.empty((1, H), dtype=torch.bfloat16, device=embed.device)
        if rot is None:
            rot = torch.empty((2, D // 2), dtype=torch.float32, device=embed.device)
        rc = self.lib.ns_decode_embed(tok.data_ptr(), pos.data_ptr(), embed.data_ptr(), vocab, H,
                                      inv_freq.data_ptr(), D, x.data_ptr(), _rot_ptr(rot, D),
                                      self._stream())
        self._check(rc, "ns_decode_embed")
        return x, rot

    def gemv_decode_attn(self, attn_out, work, pos, max_len, n_heads, Wq, S, group=128,
                         out=None):
        """y [1, N] = a . deq(Wq, S)^T where a is the output of a preceding
        decode_qkv_attention(..., merge=False) with the same work, pos, max_len and heads: its
        split partials are merged while the activation is loaded."""
        _require_gpu_tensor(attn_out, "attn_out", torch.bfloat16)
        _require_gpu_tensor(work, "work", torch.uint8)
        _require_gpu_tensor(pos, "pos", torch.int32)
        _require_gpu_tensor(Wq, "Wq", torch.int32)
        _require_gpu_tensor(S, "S", torch.bfloat16)
        N, K = Wq.shape[0], Wq.shape[1] * 8
        if out is None:
            out = torch.empty((1, N), dtype=torch.bfloat16, device=Wq.device)
        rc = self.lib.ns_w4_gemv_decode_attn(attn_out.data_ptr(), work.data_ptr(),
                                             pos.data_ptr(), max_len, n_heads, Wq.data_ptr(),
                                             S.data_ptr(), out.data_ptr(), N, K, group,
                                             self._stream())
        self._check(rc, "ns_w4_gemv_decode_attn")
        return out

    def gemv_decode(self, Wq, S, group=128, x=None, res=None, r=None, norm_w=None, eps=1e-6,
                    res_out=None, swiglu=False, out=None):
        """One-token W4 GEMV with its neighbours fused (no reference counterpart; its runner
        launches them separately, qwen.py:145-162). Activation: x [K] / [1, K], or, with res,
        rmsnorm(res + r) * norm_w (res_out receives bf16(res + r)). Output: y [1, N], or with
        ``swiglu`` (gate/up rows interleaved in blocks of 8) silu(gate) * up [1, N/2]."""
        for t, n in ((Wq, "Wq"), (S, "S")):
            _require_gpu_tensor(t, n, torch.int32 if n == "Wq" else torch.bfloat16)
            if not t.is_contiguous():
                raise ValueError(f"{n} must be contiguous")
        N, K = Wq.shape[0], Wq.shape[1] * 8
        vecs = {"x": x, "res": res, "r": r, "norm_w": norm_w, "res_out": res_out}
        for n, t in vecs.items():
            if t is not None:
                _require_gpu_tensor(t, n, torch.bfloat16)
                if t.numel() != K or not t.is_contiguous():
                    raise ValueError(f"{n} must be a contiguous tensor of {K} elements")
        n_out = N // 2 if swiglu else N
        if out is None:
            out = torch.empty((1, n_out), dtype=torch.bfloat16, device=Wq.device)
        elif out.numel() != n_out or not out.is_contiguous() or out.dtype != torch.bfloat16:
            raise ValueError(f"out must be a contiguous bf16 tensor of {n_out} elements")

        def ptr(t):
            return None if t is None else t.data_ptr()

        rc = self.lib.ns_w4_gemv_decode(ptr(x), ptr(res), ptr(r), ptr(norm_w), eps, ptr(res_out),
                                        Wq.data_ptr(), S.data_ptr(), out.data_ptr(), N, K, group,
                                        1 if swiglu else 0, self._stream())
        self._check(rc, "ns_w4_gemv_decode")
        return out

    def bf16_gemv(self, W, x=None, res=None, r=None, norm_w=None, eps=1e-6, out=None):
        """One-token bf16 product y [1, N] = a . W^T (W [N, K] bf16), the reference's lm_head
        F.linear (qwen.py:164); a is x, or with res the fused rmsnorm(res + r) * norm_w."""
        _require_gpu_tensor(W, "W", torch.bfloat16)
        if not W.is_contiguous():
            raise ValueError("W must be contiguous")
        N, K = W.shape
        for n, t in (("x", x), ("res", res), ("r", r), ("norm_w", norm_w)):
            if t is not None:
                _require_gpu_tensor(t, n, torch.bfloat16)
                if t.numel() != K or not t.is_contiguous():
                    raise ValueError(f"{n} must be a contiguous tensor of {K} elements")
        if out is None:
            out = torch.empty((1, N), dtype=torch.bfloat16, device=W.device)

        def ptr(t):
            return None if t is None else t.data_ptr()

        rc = self.lib.ns_bf16_gemv(ptr(x), ptr(res), ptr(r), ptr(norm_w), eps, W.data_ptr(),
                                   out.data_ptr(), N, K, self._stream())
        self._check(rc, "ns_bf16_gemv")
        return out

    # ------------------------------------------------------------------ packed tile format
    def w4_repack(self, Wq, S, group=128):
        """(Wq [N, K/8] int32, S [N, K/128] bf16) -> packed tiles (Wp int32 [ceil(N/16), K/128,
        256], Sp bf16 [ceil(N/16), K/128, 16]) for w4_linear_packed (include/nanoserve_w4.h)."""
        _require_gpu_tensor(Wq, "Wq", torch.int32)
        _require_gpu_tensor(S, "S", torch.bfloat16)
        N, K = Wq.shape[0], Wq.shape[1] * 8
        NT, C = (N + 15) // 16, K // 128
        Wp = torch.empty((NT, C, 256), dtype=torch.int32, device=Wq.device)
        Sp = torch.empty((NT, C, 16), dtype=torch.bfloat16, device=Wq.device)
        rc = self.lib.ns_w4_repack(Wq.contiguous().data_ptr(), S.contiguous().data_ptr(),
                                   Wp.data_ptr(), Sp.data_ptr(), N, K, group, self._stream())
        self._check(rc, "ns_w4_repack")
        return Wp, Sp

    def w4_linear_packed(self, x, Wp, Sp, N, group=128, out=None):
        """x [M, K] bf16 (M >= 2: batched decode up to 16 rows, prefill beyond) -> y [M, N]
        bf16, as w4_linear on the packed weights of w4_repack (agreeing with it to one bf16
        ulp; M > 16 with the GEMM's bf16-staged weights, as w4_linear's GEMM). M = 1 is
        rejected: the standard format (w4_linear) is the faster one there."""
        _require_gpu_tensor(x, "x", torch.bfloat16)
        _require_gpu_tensor(Wp, "Wp", torch.int32)
        _require_gpu_tensor(Sp, "Sp", torch.bfloat16)
        M, K = x.shape
        if Wp.shape[0] * 16 < N or Wp.shape[1] * 128 != K:
            raise ValueError("packed weights do not match N and x's K")
        if out is None:
            out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
        rc = self.lib.ns_w4_linear_packed(x.contiguous().data_ptr(), Wp.data_ptr(), Sp.data_ptr(),
                                          out.data_ptr(), M, N, K, group, self._stream())
        self._check(rc, "ns_w4_linear_packed")
        return out

    def w4_linear_packed_swiglu(self, x, Wp, Sp, N, group=128, out=None):
        """x [M, K] bf16 (M > 16) -> bf16(silu(g) * u) [M, N/2] on packed weights of gate/up
        rows interleaved in blocks of 8 (qwen.interleave_gate_up, then w4_repack): the packed
        GEMM with the SwiGLU epilogue (include/nanoserve_w4.h)."""
        _require_gpu_tensor(x, "x", torch.bfloat16)
        _require_gpu_tensor(Wp, "Wp", torch.int32)
        _require_gpu_tensor(Sp, "Sp", torch.bfloat16)
        M, K = x.shape
        if Wp.shape[0] * 16 < N or Wp.shape[1] * 128 != K:
            raise ValueError("packed weights do not match N and x's K")
        if out is None:
            out = torch.empty((M, N // 2), dtype=torch.bfloat16, device=x.device)
        rc = self.lib.ns_w4_linear_packed_swiglu(x.contiguous().data_ptr(), Wp.data_ptr(),
                                                 Sp.data_ptr(), out.data_ptr(), M, N, K, group,
                                                 self._stream())
        self._check(rc, "ns_w4_linear_packed_swiglu")
        return out

    # ------------------------------------------------------------------ measurement kernels
    def probe_read(self, buf, grid, waves, depth, sink):
        """Read-only stream over the bytes of ``buf`` (a 16-byte aligned GPU tensor) with the W4
        GEMV's access pattern (include/nanoserve_probe.h); ``sink`` a GPU int32 tensor."""
        rc = self.lib.ns_probe_read(buf.data_ptr(), buf.numel() * buf.element_size(),
                                    sink.data_ptr(), grid, waves, depth, self._stream())
        self._check(rc, "ns_probe_read")

    def probe_empty(self, grid=1, threads=64):
        """Launch an empty kernel (the per-launch floor of a graph of kernels)."""
        self._check(self.lib.ns_probe_empty(grid, threads, self._stream()), "ns_probe_empty")

    def linear_loop(self, calls, group=128):
        """Issue ns_w4_linear for each (x, Wq, S, y) of ``calls`` back to back from the C++ host
        loop of ns_probe_linear_loop (no Python between the launches), on the current stream.
        Every tensor must satisfy ns_w4_linear's own contract without padding (M <= 8 or a
        multiple of 128, contiguous, y [M, N])."""
        n = len(calls)
        ptrs, ints = ctypes.c_void_p * n, ctypes.c_int * n
        rc = self.lib.ns_probe_linear_loop(
            ptrs(*[c[0].data_ptr() for c in calls]), ptrs(*[c[1].data_ptr() for c in calls]),
            ptrs(*[c[2].data_ptr() for c in calls]), ptrs(*[c[3].data_ptr() for c in calls]),
            ints(*[c[0].shape[0] for c in calls]), ints(*[c[1].shape[0] for c in calls]),
            ints(*[c[0].shape[1] for c in calls]), group, n, self._stream())
        self._check(rc, "ns_probe_linear_loop")
