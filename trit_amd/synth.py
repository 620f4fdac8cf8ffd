"""Seeded synthetic inputs in the shapes of Trit's benchmark workloads.

The generator is xorshift64* (the one Trit's kernel bench uses,
src/cpu/v2/bench.rs:13-26), run as many independent streams side by side
so numpy can vectorise it: stream ``s`` of a tensor is seeded with
splitmix64(seed + s). Uniforms take the top 24 bits; normals are Box-Muller
in float64, rounded to float32. The same seed gives the same bytes on every
machine, so the CPU oracle and the GPU library are fed identical inputs.
"""

from __future__ import annotations

import numpy as np

BASE_SEED = 0x9E3779B97F4A7C15
_MUL = np.uint64(0x2545F4914F6CDD1D)
_M64 = (1 << 64) - 1


def _splitmix64(x: np.ndarray) -> np.ndarray:
    x = (x + np.uint64(0x9E3779B97F4A7C15)).astype(np.uint64)
    z = x.copy()
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    z = z ^ (z >> np.uint64(31))
    z[z == 0] = np.uint64(1)
    return z


class Streams:
    """`count` xorshift64* streams stepped together."""

    def __init__(self, seed: int, count: int):
        with np.errstate(over="ignore"):
            base = np.uint64(seed & _M64) + np.arange(count, dtype=np.uint64)
            self.state = _splitmix64(base)

    def next(self) -> np.ndarray:
        s = self.state
        with np.errstate(over="ignore"):
            s ^= s >> np.uint64(12)
            s ^= s << np.uint64(25)
            s ^= s >> np.uint64(27)
            return s * _MUL

    def uniform(self, cols: int) -> np.ndarray:
        """[count, cols] float64 in [0, 1) with 24-bit resolution."""
        out = np.empty((self.state.shape[0], cols), dtype=np.float64)
        for j in range(cols):
            out[:, j] = (self.next() >> np.uint64(40)).astype(np.float64) / float(1 << 24)
        return out

    def ints(self, cols: int, lo: int, hi: int) -> np.ndarray:
        """[count, cols] int64 uniform in [lo, hi]."""
        span = np.uint64(hi - lo + 1)
        out = np.empty((self.state.shape[0], cols), dtype=np.int64)
        for j in range(cols):
            top = self.next() >> np.uint64(32)
            with np.errstate(over="ignore"):
                out[:, j] = ((top * span) >> np.uint64(32)).astype(np.int64) + lo
        return out

    def normal(self, cols: int) -> np.ndarray:
        """[count, cols] float64 standard normals (Box-Muller)."""
        u1 = self.uniform(cols)
        u2 = self.uniform(cols)
        u1 = np.maximum(u1, 1.0 / (1 << 25))
        return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def seed_for(config: int, tensor: int) -> int:
    """Seed of tensor number `tensor` of workload `config`."""
    return (BASE_SEED + (config << 32) + (tensor << 48)) & _M64


def f16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> IEEE binary16 bits, round to nearest even."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def q8_0_blocks(codes: np.ndarray, scale_bits: np.ndarray) -> np.ndarray:
    """GGUF Q8_0 bytes: per block of 32 codes, the f16 scale (LE) then the codes.

    codes: int8 [n, k]; scale_bits: uint16 [n, k/32]. Returns uint8 [n*k/32*34].
    """
    n, k = codes.shape
    nb = k // 32
    out = np.empty((n, nb, 34), dtype=np.uint8)
    out[:, :, 0:2] = scale_bits.astype("<u2").reshape(n, nb, 1).view(np.uint8)
    out[:, :, 2:] = codes.reshape(n, nb, 32).view(np.uint8)
    return out.reshape(-1)


def q8_0_matrix(seed: int, n: int, k: int, scale: str = "uniform", lo: float = 0.002, hi: float = 0.02,
                sigma: float = 0.02):
    """Random Q8_0 weights: codes uniform in [-127, 127] and one f16 scale per block.

    scale "uniform": U[lo, hi]; "normal": N(0, sigma)/127 (sign kept).
    Returns (codes int8 [n,k], scale bits uint16 [n,k/32]).
    """
    codes = Streams(seed, n).ints(k, -127, 127).astype(np.int8)
    s = Streams(seed ^ 0x5555, n)
    if scale == "uniform":
        d = lo + (hi - lo) * s.uniform(k // 32)
    else:
        d = s.normal(k // 32) * sigma / 127.0
    return codes, f16_bits(d.astype(np.float32))


def activations(seed: int, m: int, k: int) -> np.ndarray:
    """float32 [m, k] standard normals."""
    return Streams(seed, m).normal(k).astype(np.float32)
