"""Seeded synthetic inputs for the W4A16 benchmark configurations (host-side, numpy).

Distributions follow the benchmark configurations: packed nibbles q uniform in [0, 15] (4
random bits each), 8 per uint32 low nibble first along K; per-(row, group) bf16 scales
bf16_rne(|N(0,1)| * 0.02); activations bf16_rne(N(0,1)). The same bytes feed the GPU, the CPU
baseline and the checker. All arrays are raw bit patterns: uint32 words, uint16 bf16 bits.
"""
from __future__ import annotations

import numpy as np

# Qwen2.5-7B-shaped decode linear set (fused QKV, O, fused gate+up, down) and the 1.5B gate.
QWEN7B_LAYERS = (
    ("qkv", 4608, 3584),
    ("o", 3584, 3584),
    ("gate_up", 37888, 3584),
    ("down", 3584, 18944),
)
QWEN15B_GATE = ("gate", 8960, 1536)


def bf16_rne_bits(f: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def weights(N: int, K: int, G: int = 128, seed: int = 0):
    """(Wq uint32 [N, K/8], S uint16 [N, K/G]): random nibbles and |N(0,1)| * 0.02 scales."""
    rng = np.random.Generator(np.random.PCG64(seed))
    Wq = rng.integers(0, 1 << 32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    S = bf16_rne_bits((np.abs(rng.standard_normal((N, K // G))) * 0.02).astype(np.float32))
    return Wq, S


def activations(M: int, K: int, seed: int = 1, per_row_seed: bool = False) -> np.ndarray:
    """X uint16 [M, K] = bf16(N(0,1)). With per_row_seed, row m uses seed + m."""
    if per_row_seed:
        rows = [np.random.Generator(np.random.PCG64(seed + m)).standard_normal(K) for m in range(M)]
        x = np.stack(rows) if rows else np.zeros((0, K))
    else:
        x = np.random.Generator(np.random.PCG64(seed)).standard_normal((M, K))
    return bf16_rne_bits(x.astype(np.float32))


def gemv_bytes(M: int, N: int, K: int, G: int = 128) -> int:
    """Algorithmic HBM bytes of one W4A16 GEMV/GEMM launch: packed W, scales, X and bf16 Y."""
    return N * K // 2 + N * (K // G) * 2 + M * K * 2 + M * N * 2


def gemm_flops(M: int, N: int, K: int) -> float:
    return 2.0 * M * N * K
