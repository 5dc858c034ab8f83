"""Seeded synthetic inputs for the five workloads (host side, numpy).

The reference has no random number generator, so the inputs are defined
here once and shared by the GPU path, the CPU oracle, the tests and the
benchmark:

* SplitMix64(seed): state += 0x9E3779B97F4A7C15, then the two xor-shift /
  multiply rounds of Steele, Lea and Flood (2014); draw i uses state
  seed + (i+1)*gamma, so a stream is generated vectorised.
* uniform u = (r >> 40) * 2**-24 in [0, 1); U(a, b) = a + (b - a) * u.
* normal: Box-Muller in float64 on consecutive pairs, u1 = 1 - u (never 0),
  z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = sqrt(-2 ln u1) sin(2 pi u2), rounded
  to float32.
* masks: per row, a partial Fisher-Yates shuffle picks exactly k positions.
* seeds: 0xC0FFEE + workload index (1-based, C1..C5).
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
SEED_BASE = 0xC0FFEE


def seed_for(config_index: int) -> int:
    return SEED_BASE + int(config_index)


class SplitMix64:
    """Counter-based view of one SplitMix64 stream."""

    def __init__(self, seed: int):
        self.state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
        self.count = 0

    def next_u64(self, n: int) -> np.ndarray:
        idx = np.arange(self.count + 1, self.count + 1 + n, dtype=np.uint64)
        self.count += n
        with np.errstate(over="ignore"):
            z = self.state + idx * _GAMMA
            z = (z ^ (z >> np.uint64(30))) * _M1
            z = (z ^ (z >> np.uint64(27))) * _M2
            z = z ^ (z >> np.uint64(31))
        return z

    def uniform01(self, n: int) -> np.ndarray:
        """float64 values k * 2**-24, k in [0, 2**24)."""
        r = self.next_u64(n)
        return (r >> np.uint64(40)).astype(np.float64) * (2.0 ** -24)

    def uniform(self, shape, lo: float, hi: float) -> np.ndarray:
        n = int(np.prod(shape))
        u = self.uniform01(n)
        return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)

    def normal(self, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        n = int(np.prod(shape))
        m = (n + 1) // 2
        u = self.uniform01(2 * m)
        u1 = 1.0 - u[0::2]
        u2 = u[1::2]
        rad = np.sqrt(-2.0 * np.log(u1))
        z = np.empty(2 * m, np.float64)
        z[0::2] = rad * np.cos(2.0 * np.pi * u2)
        z[1::2] = rad * np.sin(2.0 * np.pi * u2)
        return (mean + std * z[:n]).astype(np.float32).reshape(shape)

    def randint(self, n: int, high: int) -> np.ndarray:
        return (self.next_u64(n) % np.uint64(high)).astype(np.int32)

    def mask_rows(self, rows: int, cols: int, k: int) -> np.ndarray:
        """Boolean [rows, cols] with exactly k True per row (partial Fisher-Yates)."""
        out = np.zeros((rows, cols), dtype=bool)
        for r in range(rows):
            draws = self.next_u64(k)
            perm = np.arange(cols, dtype=np.int64)
            spans = np.arange(cols, cols - k, -1, dtype=np.uint64)
            picks = (draws % spans).astype(np.int64) + np.arange(k, dtype=np.int64)
            for t in range(k):
                j = picks[t]
                perm[t], perm[j] = perm[j], perm[t]
            out[r, perm[:k]] = True
        return out


# ------------------------------------------------------------ workloads

def c1_softmax(rows: int = 512, cols: int = 1024) -> np.ndarray:
    """C1: fp32 [512, 1024], N(0,1)*4."""
    return SplitMix64(seed_for(1)).normal((rows, cols), 0.0, 4.0)


def c2_reduce(rows: int = 4096, cols: int = 4096) -> np.ndarray:
    """C2: fp32 [4096, 4096] ~ U(-1, 1)."""
    return SplitMix64(seed_for(2)).uniform((rows, cols), -1.0, 1.0)


def c3_affine(rows: int = 8192, cols: int = 8192):
    """C3: X ~ N(0,1) [rows, cols], bias ~ N(0, 0.1) [cols], scale ~ U(0.5, 1.5)
    [cols], upstream dY ~ N(0, 1) [rows, cols]."""
    g = SplitMix64(seed_for(3))
    x = g.normal((rows, cols))
    bias = g.normal((cols,), 0.0, 0.1)
    scale = g.uniform((cols,), 0.5, 1.5)
    dy = g.normal((rows, cols))
    return x, scale, bias, dy


def c4_long_softmax(rows: int = 64, cols: int = 131072, masked_frac: float = 0.1):
    """C4: fp32 [64, 131072] ~ N(0,1)*8 with floor(0.1*cols) entries per row
    set to -inf; upstream gradient ~ N(0,1)."""
    g = SplitMix64(seed_for(4))
    x = g.normal((rows, cols), 0.0, 8.0)
    k = int(masked_frac * cols)
    mask = g.mask_rows(rows, cols, k)
    x[mask] = -np.inf
    dy = g.normal((rows, cols))
    return x, dy


def c5_mlp(batch: int = 4096, dims=(784, 1024, 1024, 10)):
    """C5: input U(0,1) [batch, 784], labels U{0..9}, He-normal weights
    (sigma = sqrt(2/fan_in)), zero biases."""
    g = SplitMix64(seed_for(5))
    x = g.uniform((batch, dims[0]), 0.0, 1.0)
    labels = g.randint(batch, dims[-1])
    params = {}
    for li in range(3):
        fan_in, fan_out = dims[li], dims[li + 1]
        params[f"w{li + 1}"] = g.normal((fan_in, fan_out), 0.0, float(np.sqrt(2.0 / fan_in)))
        params[f"b{li + 1}"] = np.zeros(fan_out, np.float32)
    return x, labels, params
