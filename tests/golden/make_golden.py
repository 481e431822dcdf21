"""Writes the golden fixtures under tests/golden/ from the CPU oracle (oracle/w4_oracle.c).

The oracle is pinned against the reference's own recorded results for its correctness case
(bench/bench_w4a16.cu:143-173: N=256, K=512, G=128, hash-filled inputs, seeds 11 and 12;
recorded figures in results/ncu/w4_gemv_m8.txt:7-11), so these files freeze that pinned state:
a later change to the oracle or to the kernels is checked against them.

    python tests/golden/make_golden.py        # rewrites the .npz files beside this script

Files:
  ref_case.npz  the reference correctness case: quantizer outputs Wq/S of the hash-filled W,
                activations X (rows 0..7), y_exact = fp32-dequant double-accumulated outputs,
                y_staged = the same with bf16-staged weights (the reference GEMM's semantics)
  edge_case.npz a small non-default format: G=32, K=96, N=48, M=3 (bf16 bits throughout)
  quant_case.npz the same correctness case's bf16 inputs, W [256, 512] and all 128 rows of X,
                with its 4-bit quantization error ||Y_w4 - Y_bf16|| / ||Y_bf16|| in percent
                (the reference prints it per run, bench/bench_w4a16.cu:192-196: 7.05 %); read by
                bench.py, which measures the same figure with the GPU quantizer and GEMM
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import w4_oracle as orc  # noqa: E402


def ref_case():
    N, K, G, M = 256, 512, 128, 8
    W = orc.hash_fill(N * K, 11, 0.05).reshape(N, K)
    X = orc.hash_fill(128 * K, 12, 1.0).reshape(128, K)[:M]
    Wq, S = orc.quantize(W, G)
    return dict(N=N, K=K, G=G, Wq=Wq, S=S, X=X,
                y_exact=orc.linear_f64(X, Wq, S, G).astype(np.float32),
                y_staged=orc.linear_f64(X, Wq, S, G, bf16_weights=True).astype(np.float32))


def edge_case():
    N, K, G, M = 48, 96, 32, 3
    W = orc.hash_fill(N * K, 21, 0.2).reshape(N, K)
    W[0, :G] = 0                                        # an all-zero group: scale 0
    X = orc.hash_fill(M * K, 22, 1.0).reshape(M, K)
    Wq, S = orc.quantize(W, G)
    return dict(N=N, K=K, G=G, W=W, Wq=Wq, S=S, X=X,
                y_exact=orc.linear_f64(X, Wq, S, G).astype(np.float32))


def quant_case():
    N, K, G, Mmax = 256, 512, 128, 128
    W = orc.hash_fill(N * K, 11, 0.05).reshape(N, K)
    X = orc.hash_fill(Mmax * K, 12, 1.0).reshape(Mmax, K)
    Wq, S = orc.quantize(W, G)
    y_w4 = orc.linear_f64(X, Wq, S, G).astype(np.float32)
    y_bf16 = orc.linear_dense_f64(X, orc.bf16_to_f32(W))
    return dict(N=N, K=K, G=G, W=W, X=X, Wq=Wq, S=S,
                quant_error_pct=np.float64(100 * orc.rel_fro(y_w4, y_bf16)))


CASES = {"ref_case": ref_case, "edge_case": edge_case, "quant_case": quant_case}


def main():
    for name, fn in CASES.items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **fn())
        print("wrote", name + ".npz")


if __name__ == "__main__":
    main()
