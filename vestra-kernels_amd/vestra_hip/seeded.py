"""Seeded synthetic inputs shared by the parity tests and the benchmark.

The reference publishes no N(0, sigma^2) generator (its tests use xorshift32,
an LCG and sin/cos ramps), so inputs for the DA3 configurations come from this
one: splitmix64 -> 53-bit uniform -> Box-Muller in float64 -> float32.  The
same host arrays feed the CPU oracle and the HIP backend.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int) -> np.ndarray:
    """`count` consecutive splitmix64 outputs starting from state `seed`."""
    with np.errstate(over="ignore"):
        state = np.uint64(seed) + _GOLDEN * np.arange(1, count + 1, dtype=np.uint64)
        z = state
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform01(seed: int, count: int) -> np.ndarray:
    """float64 uniforms in [0, 1) with 53 random bits."""
    return (splitmix64(seed, count) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))


def normal(seed: int, count: int, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """float32 N(mean, std^2) samples (Box-Muller on pairs of uniforms)."""
    pairs = (count + 1) // 2
    u = uniform01(seed, 2 * pairs)
    u1 = 1.0 - u[0::2]  # (0, 1]: log is finite
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * pairs, np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (z[:count] * std + mean).astype(np.float32)


def tensor_seed(base: int, layer: int, tensor_id: int) -> int:
    """Fixed seed per (base, layer, tensor id) so every tensor is independent."""
    return (base * 1_000_003 + layer * 1009 + tensor_id * 7919) & 0xFFFFFFFFFFFFFFFF


def xorshift32_values(length: int, seed: int) -> np.ndarray:
    """The reference tests' xorshift32 stream mapped to [-1, 1)
    (tests/attention_matches_naive.rs:5-16, src/attention.rs:239-249)."""
    out = np.empty(length, np.float32)
    s = seed & 0xFFFFFFFF
    umax = np.float32(4294967295.0)
    for i in range(length):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = (np.float32(s) / umax) * np.float32(2.0) - np.float32(1.0)
    return out
