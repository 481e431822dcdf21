#!/usr/bin/env python3
"""Benchmark of the W4A16 linear-layer hot path on one MI355X.

Headline (value): BASELINE config 2 -- the Qwen2.5-7B-shaped decode linear set at M=1 (fused
QKV 4608x3584, O 3584x3584, fused gate+up 37888x3584, down 3584x18944; int4 group 128). One
"step" is one pass of the four ns_w4_linear launches over one batch. value = algorithmic bytes
of the step / step time, in GB/s. Inputs are resident in HBM; weight copies rotate over
>= 1.1 GiB so each step reads HBM, not the 256 MB Infinity Cache.

Timing: warmup steps, then exactly --steps steps, each group captured in a HIP graph (no host
launch gaps inside the timed region), bracketed by synchronize() and HIP events recorded on
the stream the kernels run on. Also reported under "extra": per-layer launch durations,
the M=8 set (config 3), the 1.5B gate (config 1), the prefill GEMMs (config 4), the same
M=1 step launched eagerly from Python, and a whole 28-layer W4 Qwen2.5-7B decode step at
context 1024 (config 5, tokens/s against its 4.513 GB/token HBM floor).

roofline: the dominant kernel (gate+up GEMV, M=1): algorithmic bytes per launch / its average
launch duration (HIP events around a graph of back-to-back launches on rotating copies),
against 8 TB/s. cpu_baseline: the PyTorch-CPU dequant+matmul restatement of the reference's
CPU loop (oracle/w4_oracle.py), timed on this host's cores on the full M=1 set.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2516.6      # MI355X dense bf16 MFMA (256 CU x 4096 flop/clk x 2.4 GHz)
G = 128
ROTATE_BYTES = int(1.1 * (1 << 30))
# HBM bytes per launch of the dominant kernel, from FETCH_SIZE / WRITE_SIZE counter passes scaled
# by a 1 GiB copy's readings (the summary holds the commands and the arithmetic).
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "w4_gemv_m1_kernel.gate_up_m1.md")


def profiled_traffic(path):
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-extra", action="store_true", help="headline only")
    p.add_argument("--cpu-seconds", type=float, default=20.0, help="CPU baseline time budget")
    p.add_argument("--dominant-only", action="store_true",
                   help="only the dominant-kernel launches (gate_up, M=1), e.g. under a profiler")
    p.add_argument("--gemm-only", action="store_true",
                   help="only the prefill GEMM launches (config 4), e.g. under a profiler")
    p.add_argument("--m1-only", action="store_true",
                   help="only the config-2 set (the four layers at M=1), e.g. under a profiler")
    p.add_argument("--m8-only", action="store_true",
                   help="only the config-3 set (the four layers at M=8), e.g. under a profiler")
    p.add_argument("--packed-only", action="store_true",
                   help="only the packed-format launches (config-3 set and config-4 GEMMs), e.g. "
                        "under a profiler")
    p.add_argument("--decode-only", action="store_true",
                   help="only the config-5 decode step (28-layer W4 Qwen2.5-7B, context 1024)")
    p.add_argument("--prefill-only", action="store_true",
                   help="only the Qwen2.5-7B-shaped prompt pass on the standard and packed formats")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only 1 GiB device-to-device copies: the known-size reference for HBM "
                        "byte counters read under a profiler")
    return p.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: this build measures one GPU only (each GPU box has "
              "one MI355X); multi-GPU sharding is design-only.", file=sys.stderr)
        sys.exit(2)

    import torch

    from nanoserve_amd import Kernels, synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel(), "copy_bytes_written": dst.numel(),
                          "launches": 8}), flush=True)
        return
    kern = Kernels()
    dev = torch.device("cuda", 0)

    def dev_bits(a, dtype):
        view = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32}[a.dtype]
        return torch.from_numpy(np.ascontiguousarray(a).view(view)).view(dtype).to(dev)

    layers = synth.QWEN7B_LAYERS
    set_bytes = sum(N * K // 2 + N * (K // G) * 2 for _, N, K in layers)
    copies = max(2, -(-ROTATE_BYTES // set_bytes))

    # Host inputs (one seeded draw per layer), device copies rotated for timing.
    host_w = {name: synth.weights(N, K, G, seed=10 + i) for i, (name, N, K) in enumerate(layers)}
    dev_w = {name: [] for name, _, _ in layers}
    for name, N, K in layers:
        Wq, S = host_w[name]
        wq0, s0 = dev_bits(Wq, torch.int32), dev_bits(S, torch.bfloat16)
        dev_w[name].append((wq0, s0))
        for _ in range(copies - 1):
            dev_w[name].append((wq0.clone(), s0.clone()))
    x1 = {name: dev_bits(synth.activations(1, K, seed=100 + i), torch.bfloat16)
          for i, (name, N, K) in enumerate(layers)}
    x8 = {name: dev_bits(synth.activations(8, K, seed=200 + 8 * i, per_row_seed=True),
                         torch.bfloat16) for i, (name, N, K) in enumerate(layers)}
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    # K-split workspaces of the M = 8 layers (ns_w4_linear_ws: only the down projection, K =
    # 18944, asks for one; on MI355X it runs the one-pass chunked kernel and leaves it unused)
    ws8 = {name: kern.w4_linear_workspace(8, N, K, G, device=dev) for name, N, K in layers}

    def step(xs, i, which=None):
        for name, N, K in layers:
            if which is not None and name != which:
                continue
            wq, s = dev_w[name][i % copies]
            kern.w4_linear(xs[name], wq, s, G, work=ws8[name] if xs is x8 else None)

    def graph_of(fn, n):
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn(0)  # allocator and launch-cache warm-up outside capture
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):  # the stream that ran the warm-up
            for i in range(n):
                fn(i)
        torch.cuda.synchronize()
        return g

    def time_graph(g, reps=1):
        st = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(st)
        for _ in range(reps):
            g.replay()
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)  # ms

    def steady_ms(g, n, warm_ms=20.0, rounds=7):
        """Per-launch ms of a graph of n launches: replays until warm_ms of GPU time have passed
        (the core clock settles under sustained load: right after an idle gap the same graph
        ran 3-25 % slower on MI355X), then the median of `rounds` single replays."""
        spent = 0.0
        for _ in range(200):
            spent += time_graph(g)
            if spent >= warm_ms:
                break
        return statistics.median(time_graph(g) for _ in range(rounds)) / n

    def deq_f32(wq, s):
        """Plain-torch fp32 dequantization on the GPU (the reference's CPU loop restated,
        bench/bench_w4a16.cu:156-173): nibble i of word j is k = 8j + i, w = (q - 8) * s."""
        N, KW = wq.shape
        shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=wq.device)
        q = (wq.unsqueeze(-1) >> shifts) & 0xF
        w = q.reshape(N, KW * 8).to(torch.float32) - 8.0
        return (w.view(N, s.shape[1], -1) * s.float().unsqueeze(-1)).view(N, KW * 8)

    def max_rel(y, ref):
        return float((y.float() - ref).abs().max() / ref.abs().max())

    def correctness_gate():
        """Before any timing, as the reference's bench does (bench_w4a16.cu:138-204): every
        config-2 layer at M = 1 and M = 8 and the config-4 GEMMs at M = 512 against a plain
        torch fp32 dequant + fp32 matmul on the GPU; max |y - ref| / max |ref| <= 1e-2."""
        errs = {}
        for name, N, K in layers:
            wq, s = dev_w[name][0]
            w = deq_f32(wq, s)
            cases = [(1, x1[name]), (8, x8[name])]
            if name in ("gate_up", "down"):
                cases.append((512, dev_bits(synth.activations(512, K, seed=512), torch.bfloat16)))
            for M, x in cases:
                y = kern.w4_linear(x, wq, s, G)
                ref = x.float() @ w.t()
                errs[f"{name}_m{M}"] = max_rel(y, ref)
                if M == 8 and ws8[name] is not None:  # the K-split form the M = 8 set times
                    errs[f"{name}_m8_ksplit"] = max_rel(kern.w4_linear(x, wq, s, G, work=ws8[name]), ref)
            del w
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        q = quantization_case()
        ok = (all(v <= 1e-2 for v in errs.values()) and q["codes_bit_exact"] and
              abs(q["quant_error_pct"] - q["oracle_pct"]) <= 0.05)
        return {"max_rel_err": {k: float(f"{v:.3e}") for k, v in errs.items()},
                "tolerance": 1e-2, "pass": ok,
                "reference": "torch fp32 dequant + fp32 matmul on the GPU", "quantization": q}

    def quantization_case():
        """The reference's correctness case (bench_w4a16.cu:143-196: N = 256, K = 512, G = 128,
        128 hash-filled activation rows, its inputs frozen in tests/golden/quant_case.npz): the
        GPU quantizer's codes and scales against the fixture's, and the 4-bit quantization error
        ||Y_w4 - Y_bf16|| / ||Y_bf16|| of the GPU GEMM's output against the bf16 weights' fp32
        product -- the figure the reference prints per run (7.05 %)."""
        z = np.load(os.path.join(ROOT, "tests", "golden", "quant_case.npz"))
        W = dev_bits(z["W"], torch.bfloat16)
        X = dev_bits(z["X"], torch.bfloat16)
        wq, s = kern.w4_quantize(W, int(z["G"]))
        torch.cuda.synchronize()
        same = (np.array_equal(wq.cpu().view(torch.int32).numpy().view(np.uint32), z["Wq"]) and
                np.array_equal(s.cpu().view(torch.int16).numpy().view(np.uint16), z["S"]))
        y_w4 = kern.w4_linear(X, wq, s, int(z["G"])).float()
        y_bf16 = X.float() @ W.float().t()
        err = float(((y_w4 - y_bf16).norm() / y_bf16.norm()).item()) * 100
        return {"codes_bit_exact": bool(same), "quant_error_pct": round(err, 2),
                "oracle_pct": round(float(z["quant_error_pct"]), 2), "reference_pct": 7.05}

    def ceiling():
        """The launch floor (an empty kernel in a graph, per launch) and the read-only stream
        ceiling at each config-2 layer's byte count (ns_probe_read: the GEMV's 1 KiB-per-wave
        access pattern and cache policy, rotating buffers past the MALL, best of a few grid
        shapes). The reference reports its GEMVs against a measured copy ceiling
        (bench_w4a16.cu:122-136); a GEMV only reads, so its ceiling is a read stream."""
        sink = torch.zeros(4, dtype=torch.int32, device=dev)
        ge = graph_of(lambda i: kern.probe_empty(1, 64), 64)
        time_graph(ge)
        floor_us = statistics.median(time_graph(ge) for _ in range(5)) / 64 * 1e3
        out = {"launch_floor_us": round(floor_us, 3), "read": {}}
        shapes = ((1024, 8, 1), (2048, 4, 1), (512, 16, 1), (768, 8, 1))
        for name, N, K in layers:
            nb = synth.gemv_bytes(1, N, K, G) // 1024 * 1024
            nbuf = max(4, -(-ROTATE_BYTES // nb))
            bufs = [torch.ones(nb // 4, dtype=torch.int32, device=dev) for _ in range(nbuf)]
            best = None
            for grid, waves, depth in shapes:
                g = graph_of(lambda i: kern.probe_read(bufs[i % nbuf], grid, waves, depth, sink),
                             2 * nbuf)
                us = steady_ms(g, 2 * nbuf, warm_ms=10.0, rounds=3) * 1e3
                if best is None or us < best[0]:
                    best = (us, grid, waves, depth)
                del g
            us, grid, waves, depth = best
            out["read"][name] = {"bytes": nb, "us": round(us, 3), "gbs": round(nb / us / 1e3, 1),
                                 "frac_hbm": round(nb / us / 1e3 / HBM_PEAK_GBS, 4),
                                 "grid": grid, "waves": waves, "depth": depth}
            del bufs
        torch.cuda.empty_cache()
        return out

    def gemm_set():
        """config 4: prefill GEMMs, gate_up and down at M = 512 and 2048"""
        gemm = {}
        for name, N, K in layers:
            if name not in ("gate_up", "down"):
                continue
            for M in (512, 2048):
                xa = dev_bits(synth.activations(M, K, seed=M), torch.bfloat16)
                ws = dev_w[name]
                reps = 6
                g = graph_of(lambda i: kern.w4_linear(xa, *ws[i % copies], G), reps)
                ms = steady_ms(g, reps)
                tf = synth.gemm_flops(M, N, K) / (ms * 1e-3) / 1e12
                gemm[f"{name}_m{M}"] = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1),
                                        "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4)}
                del xa
        return gemm

    def decode_step(reps=40, ctx=1024, decode=True, prefill=True):
        """config 5: one decode step of a random-init W4A16 Qwen2.5-7B (28 layers, fused QKV and
        gate+up, bf16 lm_head) at context 1024 with a bf16 KV cache filled with N(0,1); the step
        is one HIP graph replay: ns_decode_embed (embedding row + the position's rotation
        table), then per layer ns_w4_gemv_decode (q/k/v, add + RMSNorm in),
        ns_decode_qkv_attention, ns_w4_gemv_decode_attn (o), ns_w4_gemv_decode (gate/up, add +
        RMSNorm in, SwiGLU out), ns_w4_gemv_decode (down); then ns_bf16_gemv (final add + RMSNorm
        + lm_head)."""
        from nanoserve_amd.qwen import Qwen2Runner, Qwen2Shape

        shape = Qwen2Shape()
        runner = Qwen2Runner.random(shape, device=dev, seed=7, kernels=kern)
        if not decode:
            pre = prefill_pass(runner, shape)
            del runner
            torch.cuda.empty_cache()
            return None, pre
        runner.alloc_cache(ctx)
        gen = torch.Generator(device=dev).manual_seed(8)
        runner.cache_k.copy_(torch.randn(runner.cache_k.shape, generator=gen, device=dev))
        runner.cache_v.copy_(torch.randn(runner.cache_v.shape, generator=gen, device=dev))
        runner.capture_decode()
        runner.decode(1234, ctx - 1)
        torch.cuda.synchronize()
        st = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        times = []
        for _ in range(5):
            e0.record(st)
            for _ in range(reps):
                runner.graph.replay()
            e1.record(st)
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) / reps)
        ms = statistics.median(times)
        runner.graph = None
        for _ in range(3):
            runner.decode(1234, ctx - 1)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(10):
            runner.decode(1234, ctx - 1)
        torch.cuda.synchronize()
        ms_eager = (time.perf_counter() - t0) * 1e3 / 10
        finite = bool(torch.isfinite(runner.logits).all())
        nbytes = shape.decode_bytes(ctx)
        runner.graph = None
        runner.cache_k = runner.cache_v = None
        pre = prefill_pass(runner, shape) if prefill else None
        del runner
        torch.cuda.empty_cache()
        gbs = nbytes / (ms * 1e-3) / 1e9
        return {"ms_per_token": round(ms, 4), "tokens_per_s": round(1e3 / ms, 1),
                "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                "bytes_per_token": nbytes, "hbm_floor_ms": round(nbytes / HBM_PEAK_GBS / 1e6, 4),
                "eager_ms_per_token": round(ms_eager, 3), "context": ctx, "logits_finite": finite,
                "timing": f"median of 5 x {reps} graph replays, hip events"}, pre

    def prefill_pass(runner, shape, tokens=(512, 2048), reps=3):
        """The same model's prompt pass (Qwen2Runner.forward over T new tokens, last-token
        logits): W4 GEMMs on the standard format (ns_w4_linear, ns_w4_linear_swiglu), then on the
        packed tile format after pack_prefill (ns_w4_linear_packed, ns_w4_linear_packed_swiglu);
        norms, rope and the causal attention as the runner runs them (attention in fp32
        PyTorch). Median of reps passes after one warm pass, hip events."""
        st = torch.cuda.current_stream()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)

        def timed(ids):
            runner.forward(ids, 0, last_only=True)
            torch.cuda.synchronize()
            ts = []
            for _ in range(reps):
                e0.record(st)
                runner.forward(ids, 0, last_only=True)
                e1.record(st)
                torch.cuda.synchronize()
                ts.append(e0.elapsed_time(e1))
            return statistics.median(ts)

        res = {}
        for T in tokens:
            ids = torch.randint(0, shape.vocab, (T,), generator=torch.Generator().manual_seed(9)).to(dev)
            runner.packed = None
            ms_std = timed(ids)
            ref = runner.forward(ids, 0, last_only=True).float()
            if runner.packed is None:
                runner.pack_prefill()
            ms_pk = timed(ids)
            out = runner.forward(ids, 0, last_only=True).float()
            gap = ((out - ref).abs().max() / ref.abs().max()).item()
            cos = torch.nn.functional.cosine_similarity(out.flatten(), ref.flatten(), dim=0).item()
            w4_flops = 2 * T * sum(n * kk for n, kk in (
                (shape.qkv_rows, shape.hidden), (shape.hidden, shape.heads * shape.head_dim),
                (2 * shape.intermediate, shape.hidden), (shape.hidden, shape.intermediate))) * shape.layers
            res[f"t{T}"] = {"ms_standard": round(ms_std, 3), "ms_packed": round(ms_pk, 3),
                            "tokens_per_s_standard": round(T / ms_std * 1e3, 1),
                            "tokens_per_s_packed": round(T / ms_pk * 1e3, 1),
                            "w4_tflops_packed": round(w4_flops / (ms_pk * 1e-3) / 1e12, 1),
                            "logits_gap_packed_vs_standard": round(gap, 5),
                            "logits_cos_packed_vs_standard": round(cos, 6)}
        runner.packed = None
        res["timing"] = (f"Qwen2.5-7B-shaped random-init runner, one prompt pass of T tokens from "
                         f"position 0, median of {reps} after a warm pass, hip events; "
                         "w4_tflops counts the W4 GEMM flops only (the pass also runs attention, "
                         "norms, rope and the lm_head); the logits gap is max |packed - standard| / "
                         "max |standard| of the last token: both formats stage the same bf16 weights "
                         "and differ in fp32 summation order, which 28 random-init layers amplify")
        return res

    def gptq_set():
        """The calibrated quantizer (ns_w4_gptq) on the gate_up and down layers: one call after a
        warm-up call, hip events; the float64 factor U separately (host clock, synchronised);
        quality as the layer's output error on calibration rows through ns_w4_linear relative to
        round to nearest's. Calibration activations: a rank-32 component plus noise."""
        from nanoserve_amd import gptq as gq

        res = {}
        gen = torch.Generator(device=dev).manual_seed(5)
        for name, N, K in layers:
            if name not in ("gate_up", "down"):
                continue
            W = (torch.randn(N, K, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
            X = (torch.randn(512, 32, device=dev, generator=gen)
                 @ torch.randn(32, K, device=dev, generator=gen) / 32 ** 0.5
                 + 0.3 * torch.randn(512, K, device=dev, generator=gen))
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            U, _ = gq.hessian_factor(gq.hessian(X))
            torch.cuda.synchronize()
            t_factor = time.perf_counter() - t0
            kern.w4_gptq(W, U, G)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            Wq, S = kern.w4_gptq(W, U, G)
            e1.record()
            torch.cuda.synchronize()
            Wr, Sr = kern.w4_quantize(W, G)
            xb = X[:128].to(torch.bfloat16)
            ref = xb.float() @ W.float().t()
            err_g = float((kern.w4_linear(xb, Wq, S, G).float() - ref).norm())
            err_r = float((kern.w4_linear(xb, Wr, Sr, G).float() - ref).norm())
            res[name] = {"shape": [N, K], "ms": round(e0.elapsed_time(e1), 2),
                         "factor_s": round(t_factor, 3), "err_vs_rtn": round(err_g / err_r, 4)}
            del W, X, U, Wq, S, Wr, Sr
        torch.cuda.empty_cache()
        return res

    def library_reference():
        """What vendor library kernels reach on the same box and shapes, for context: the bf16
        GEMM (torch.matmul -> hipBLASLt; unquantized bf16 weights, so twice the weight bytes of
        the W4 GEMM but no dequantization) at the config-4 shapes, and torch's device copy of the
        dominant layer's byte count (rotating buffers past the MALL) as a library stream rate."""
        ref = {}
        for name, N, K in layers:
            if name not in ("gate_up", "down"):
                continue
            wb = torch.randn(N, K, device=dev).to(torch.bfloat16)
            for M in (512, 2048):
                xa = torch.randn(M, K, device=dev).to(torch.bfloat16)
                torch.matmul(xa, wb.t())
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                runs = []
                for _ in range(3):
                    e0.record()
                    for _ in range(6):
                        torch.matmul(xa, wb.t())
                    e1.record()
                    torch.cuda.synchronize()
                    runs.append(e0.elapsed_time(e1) / 6)
                ms = statistics.median(runs)
                tf = synth.gemm_flops(M, N, K) / (ms * 1e-3) / 1e12
                ref[f"hipblaslt_bf16_{name}_m{M}"] = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1),
                                                      "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4)}
                del xa
            del wb
        nb = synth.gemv_bytes(1, 37888, 3584, G)
        nbuf = max(2, -(-ROTATE_BYTES // (2 * nb)))
        srcs = [torch.ones(nb // 4, dtype=torch.int32, device=dev) for _ in range(nbuf)]
        dsts = [torch.empty_like(t) for t in srcs]
        for a, b in zip(dsts, srcs):
            a.copy_(b)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        runs = []
        for _ in range(3):
            e0.record()
            for a, b in zip(dsts, srcs):
                a.copy_(b)
            e1.record()
            torch.cuda.synchronize()
            runs.append(e0.elapsed_time(e1) / nbuf)
        ms = statistics.median(runs)
        ref["torch_copy_gate_up_bytes"] = {"bytes_read": nb, "bytes_written": nb,
                                           "us": round(ms * 1e3, 2),
                                           "gbs_read_plus_write": round(2 * nb / (ms * 1e-3) / 1e9, 1)}
        del srcs, dsts
        torch.cuda.empty_cache()
        return ref

    def packed_sets():
        """The config-3 set (M = 8) and the config-4 GEMMs on the packed tile format:
        ns_w4_repack once, then ns_w4_linear_packed for every layer (K <= 4096: activation in
        registers; the down projection, K = 18944, through the long-row kernel's LDS chunks),
        per layer and as a set, beside the standard format's config-3 set, and the prefill
        GEMMs (M > 16) beside config4_gemm. The packed format serves batched decode (M = 2..16)
        and prefill; at M = 1 ns_w4_linear_packed is not offered (the standard kernel is faster
        there)."""
        pk = {name: [kern.w4_repack(wq, s, G) for wq, s in dev_w[name]] for name, _, _ in layers}
        torch.cuda.synchronize()
        res = {}
        M, xs = 8, x8

        def run(i, which=None):
            for name, N, K in layers:
                if which is None or name == which:
                    kern.w4_linear_packed(xs[name], *pk[name][i % copies], N, G)

        nl = 4 * copies  # launches per timed graph, as the per-layer legs
        for name, N, K in layers:
            g = graph_of(lambda i, name=name: run(i, which=name), nl)
            ms = steady_ms(g, nl)
            b = synth.gemv_bytes(M, N, K, G)
            res[f"{name}_m{M}"] = {"us": round(ms * 1e3, 3), "gbs": round(b / (ms * 1e-3) / 1e9, 1)}
        g = graph_of(lambda i: run(i), 4 * copies)
        ms = steady_ms(g, 4 * copies)
        b = sum(synth.gemv_bytes(M, N, K, G) for _, N, K in layers)
        res[f"set_m{M}"] = {"us": round(ms * 1e3, 3), "gbs": round(b / (ms * 1e-3) / 1e9, 1),
                            "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        # the config-4 prefill GEMMs on the packed tiles (ns_w4_linear_packed at M > 16)
        for name, N, K in layers:
            if name not in ("gate_up", "down"):
                continue
            for Mg in (512, 2048):
                xa = dev_bits(synth.activations(Mg, K, seed=Mg), torch.bfloat16)
                reps = 6
                g = graph_of(lambda i, name=name, xa=xa, N=N: kern.w4_linear_packed(
                    xa, *pk[name][i % copies], N, G), reps)
                ms = steady_ms(g, reps)
                tf = synth.gemm_flops(Mg, N, K) / (ms * 1e-3) / 1e12
                res[f"gemm_{name}_m{Mg}"] = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1),
                                             "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4)}
                del xa
        del pk
        torch.cuda.empty_cache()
        return res

    if args.gemm_only:
        print(json.dumps({"config4_gemm": gemm_set()}), flush=True)
        return
    if args.packed_only:
        print(json.dumps({"packed_format": packed_sets()}), flush=True)
        return
    if args.decode_only:
        dec, _ = decode_step(prefill=False)
        print(json.dumps({"config5_decode": dec}), flush=True)
        return
    if args.prefill_only:
        _, pre = decode_step(decode=False)
        print(json.dumps({"config5_prefill": pre}), flush=True)
        return

    def m8_set():
        g8 = graph_of(lambda i: step(x8, i), 4 * copies)
        ms8 = steady_ms(g8, 4 * copies)
        bytes_m8 = sum(synth.gemv_bytes(8, N, K, G) for _, N, K in layers)
        return {"gbs": round(bytes_m8 / (ms8 * 1e-3) / 1e9, 1), "us_per_step": round(ms8 * 1e3, 3),
                "frac_hbm": round(bytes_m8 / (ms8 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}

    if args.m8_only:
        print(json.dumps({"config3_m8_set": m8_set(), "launches": 4 * (4 * copies) * 4 + 4}), flush=True)
        return

    if args.m1_only:
        g1 = graph_of(lambda i: step(x1, i), 4 * copies)
        ms1 = steady_ms(g1, 4 * copies)
        bytes_set = sum(synth.gemv_bytes(1, N, K, G) for _, N, K in layers)
        print(json.dumps({"config2_m1_set": {
            "gbs": round(bytes_set / (ms1 * 1e-3) / 1e9, 1), "us_per_step": round(ms1 * 1e3, 3)},
            "launches": 4 * (4 * copies) * 4 + 4}), flush=True)
        return

    bytes_m1 = sum(synth.gemv_bytes(1, N, K, G) for _, N, K in layers)
    gate = None if args.dominant_only else correctness_gate()
    if gate is not None and not gate["pass"]:
        print(json.dumps({"metric": "W4A16 GEMV HBM GB/s (% of peak) at M=1/8; prefill GEMM "
                          "TFLOP/s (% MFMA)", "value": None, "error": "correctness gate failed",
                          "correctness": gate}), flush=True)
        sys.exit(1)
    value = ms_step = None
    if not args.dominant_only:
        # ---------------- headline: M=1 set, exactly args.steps steps
        g_warm = graph_of(lambda i: step(x1, i), max(args.warmup, 1))
        g_main = graph_of(lambda i: step(x1, i), args.steps)
        if args.warmup > 0:
            time_graph(g_warm)
        ms_total = time_graph(g_main)
        ms_step = ms_total / args.steps
        value = bytes_m1 / (ms_step * 1e-3) / 1e9

    # ---------------- dominant kernel: gate+up GEMV, M=1, back-to-back launches, timed warm
    # (steady_ms)
    n_launch = 4 * copies
    g_gu = graph_of(lambda i: step(x1, i, which="gate_up"), n_launch)
    ms_gu = steady_ms(g_gu, n_launch)
    N_gu, K_gu = [(N, K) for n, N, K in layers if n == "gate_up"][0]
    bytes_gu = synth.gemv_bytes(1, N_gu, K_gu, G)
    achieved = bytes_gu / (ms_gu * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": profiled_traffic(TRAFFIC_PROFILE),
                "kernel": "w4_gemv_m1_kernel<7, 2, 16, 0, 0, 4, true, false> (gate_up 37888x3584, M=1)",
                "bytes_per_launch": bytes_gu, "avg_launch_us": round(ms_gu * 1e3, 3),
                "timing": "hip events on the launch stream around graph replays of "
                          f"{n_launch} launches on rotating weight copies, after >= 20 ms of "
                          "warm replays; median of 7 (the same measurement is "
                          "extra.per_layer.gate_up_m1)"}

    if args.dominant_only:
        print(json.dumps({"roofline": roofline, "launches": 6 * n_launch}), flush=True)
        return

    extra = {}
    ceil = None
    if not args.no_extra:
        ceil = ceiling()
        extra["ceiling"] = ceil
        roofline["ceiling_gbs"] = ceil["read"]["gate_up"]["gbs"]
        roofline["frac_of_ceiling"] = round(achieved / ceil["read"]["gate_up"]["gbs"], 4)
        per_layer = {}
        for name, N, K in layers:
            for M, xs in ((1, x1), (8, x8)):
                if name == "gate_up" and M == 1:
                    ms = ms_gu  # one measurement of the dominant kernel feeds both figures
                else:
                    g = graph_of(lambda i, name=name, xs=xs: step(xs, i, which=name), n_launch)
                    ms = steady_ms(g, n_launch)
                b = synth.gemv_bytes(M, N, K, G)
                per_layer[f"{name}_m{M}"] = {"us": round(ms * 1e3, 3),
                                             "gbs": round(b / (ms * 1e-3) / 1e9, 1),
                                             "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                             "frac_ceiling": round(ceil["read"][name]["us"] / (ms * 1e3), 4)}
                if M == 8 and ws8[name] is not None:
                    per_layer[f"{name}_m{M}"]["entry"] = "ns_w4_linear_ws"
        extra["per_layer"] = per_layer

        extra["config3_m8_set"] = m8_set()

        # eager launches (Python + ctypes per call), for reference only
        for i in range(10):
            step(x1, i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            step(x1, i)
        torch.cuda.synchronize()
        ms_eager = (time.perf_counter() - t0) * 1e3 / args.steps
        extra["config2_m1_eager_gbs"] = round(bytes_m1 / (ms_eager * 1e-3) / 1e9, 1)

        # the same steps as back-to-back launches from a C++ host loop (the reference's own
        # benchmark method, bench/bench_w4a16.cu:42-78): no graph, no Python between launches
        def loop_calls(xs, n):
            out = []
            for i in range(n):
                for name, N, K in layers:
                    wq, s = dev_w[name][i % copies]
                    out.append((xs[name], wq, s, ys1[name]))
            return out
        ys1 = {name: torch.empty(1, N, dtype=torch.bfloat16, device=dev) for name, N, K in layers}
        warm_calls, main_calls = loop_calls(x1, max(args.warmup, 1)), loop_calls(x1, args.steps)
        loop_ms = []
        for _ in range(3):
            kern.linear_loop(warm_calls, G)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            kern.linear_loop(main_calls, G)
            e1.record()
            torch.cuda.synchronize()
            loop_ms.append(e0.elapsed_time(e1) / args.steps)
        ms_loop = statistics.median(loop_ms)
        extra["config2_m1_stream_launch"] = {"us_per_step": round(ms_loop * 1e3, 3),
                                             "gbs": round(bytes_m1 / (ms_loop * 1e-3) / 1e9, 1)}

        # config 1: Qwen2.5-1.5B gate, M=1
        name, N, K = synth.QWEN15B_GATE
        Wq, S = synth.weights(N, K, G, seed=1)
        c1b = N * K // 2 + N * (K // G) * 2
        c1n = max(2, -(-ROTATE_BYTES // c1b))
        wq0, s0 = dev_bits(Wq, torch.int32), dev_bits(S, torch.bfloat16)
        c1w = [(wq0, s0)] + [(wq0.clone(), s0.clone()) for _ in range(c1n - 1)]
        xc1 = dev_bits(synth.activations(1, K, seed=3), torch.bfloat16)
        g1 = graph_of(lambda i: kern.w4_linear(xc1, *c1w[i % c1n], G), 2 * c1n)
        ms1 = steady_ms(g1, 2 * c1n)
        b1 = synth.gemv_bytes(1, N, K, G)
        extra["config1_gate_m1"] = {"us": round(ms1 * 1e3, 3), "gbs": round(b1 / (ms1 * 1e-3) / 1e9, 1)}
        del c1w, wq0, s0

        extra["packed_format"] = packed_sets()
        extra["config4_gemm"] = gemm_set()
        extra["config5_decode"], extra["config5_prefill"] = decode_step()
        extra["gptq"] = gptq_set()
        extra["library_reference"] = library_reference()


    # ---------------- CPU baseline (PyTorch CPU dequant + fp32 matmul), full M=1 set
    cpu = None
    if not args.no_cpu:
        from oracle.w4_oracle import torch_cpu_linear

        cpu_in = []
        for i, (name, N, K) in enumerate(layers):
            Wq, S = host_w[name]
            cpu_in.append((torch.from_numpy(synth.activations(1, K, seed=100 + i).view(np.int16).copy()).view(torch.bfloat16),
                           torch.from_numpy(Wq.view(np.int32).copy()),
                           torch.from_numpy(S.view(np.int16).copy()).view(torch.bfloat16)))
        for (name, N, K), (x, _, _) in zip(layers, cpu_in):  # the same bytes as the GPU's inputs
            assert torch.equal(x, x1[name].cpu()), name

        def cpu_step():
            return [torch_cpu_linear(x, wq, s, G) for x, wq, s in cpu_in]

        cpu_out = cpu_step()  # warmup; its outputs check the GPU's on the same inputs
        gpu_err = {}
        for (name, N, K), ref in zip(layers, cpu_out):
            y = kern.w4_linear(x1[name], *dev_w[name][0], G).float().cpu()
            gpu_err[name] = float(f"{float((y - ref).abs().max() / ref.abs().max()):.3e}")
        times = []
        t_start = time.perf_counter()
        while len(times) < 5 or (time.perf_counter() - t_start < args.cpu_seconds and len(times) < 50):
            t0 = time.perf_counter()
            cpu_step()
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - t_start > 3 * args.cpu_seconds:
                break
        med = statistics.median(times)
        model = platform.processor() or ""
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
        cpu = {"value": round(bytes_m1 / med / 1e9, 2), "unit": "GB/s", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"full config-2 M=1 set (4 layers), median of {len(times)} runs, "
                         f"{med * 1e3:.1f} ms/step; PyTorch CPU unpack + (q-8)*s fp32 + fp32 matmul",
               "os_cpu_count": os.cpu_count(), "cpu_model": model,
               "max_rel_err": gpu_err, "pass": all(v <= 1e-2 for v in gpu_err.values())}

    line = {
        "metric": "W4A16 GEMV HBM GB/s (% of peak) at M=1/8; prefill GEMM TFLOP/s (% MFMA)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded int4 nibbles, |N(0,1)|*0.02 bf16 scales, N(0,1) bf16 activations)",
        "config": {"workload": "config2: Qwen2.5-7B-shaped decode linear set, M=1, W4 group 128 "
                               "(qkv 4608x3584, o 3584x3584, gate_up 37888x3584, down 3584x18944)",
                   "frac_hbm": round(value / HBM_PEAK_GBS, 4), "bytes_per_step": bytes_m1,
                   "weight_copies": copies, "timing": "hip graph replay, hip events"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "correctness": gate,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    if cpu is not None and not cpu["pass"]:
        print("bench.py: GPU outputs differ from the CPU baseline's beyond 1e-2", file=sys.stderr)
        sys.exit(1)


if __name__ == "__main__":
    main()
