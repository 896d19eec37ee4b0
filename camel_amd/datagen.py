"""Seeded synthetic inputs shared by the tests and bench.py.

Counter-based SplitMix64 (S. Vigna, public domain): value i of stream `seed` is
mix(seed + (i+1) * 0x9E3779B97F4A7C15).  Uniforms take the top 24 bits,
u = (x >> 40) * 2^-24, exact in fp32, and U(lo, hi) = lo + (hi-lo)*u in fp32
(exact for U(0,1) and U(-1,1)).  Normals use Box-Muller in fp64 on the host
and are rounded to fp32 once.  The same host buffers feed the CPU oracle and
(after H2D) the GPU, so both sides see bit-identical inputs.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

# Seeds of the benchmark configurations (one stream per tensor).
SEED_MATMUL_A, SEED_MATMUL_B = 0x5EED0001, 0x5EED0002
SEED_MLP = 0x5EED0010
SEED_GEMM = 0x5EED0020
SEED_CONV_X, SEED_CONV_W = 0x5EED0040, 0x5EED0041
SEED_CNN = 0x5EED0050
SEED_ELT = 0x5EED0060


def splitmix64(seed: int, start: int, count: int) -> np.ndarray:
    idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + idx * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


def uniform(seed: int, shape, lo: float = 0.0, hi: float = 1.0, chunk: int = 1 << 24) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    span = np.float32(hi) - np.float32(lo)
    for s in range(0, n, chunk):
        c = min(chunk, n - s)
        u = (splitmix64(seed, s, c) >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
        out[s:s + c] = np.float32(lo) + span * u
    return out.reshape(shape)


def normal(seed: int, shape, std: float = 1.0, chunk: int = 1 << 23) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, chunk):
        c = min(chunk, n - s)
        x = splitmix64(seed, 2 * s, 2 * c)
        u1 = 1.0 - (x[0::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53  # (0, 1]
        u2 = (x[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        out[s:s + c] = (z * std).astype(np.float32)
    return out.reshape(shape)
