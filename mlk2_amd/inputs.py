"""Seeded synthetic inputs shared by the HIP backend's tests and bench.

Counter-mode SplitMix64: ``u_i = (mix(seed + i*0x9E3779B97F4A7C15) >> 40) * 2^-24``
gives u in [0, 1) with 24 significant bits, exact in f32. ``mix`` is the
SplitMix64 output function (Steele, Lea, Flood, "Fast splittable
pseudorandom number generators", OOPSLA 2014). Uniform draws are computed in
f64 and rounded once to the buffer dtype (RNE); normal draws use Box-Muller on
consecutive pairs with u1 <- 1 - u. Both sides of every comparison receive the
same dtype-rounded values, widened exactly to f64 for the CPU oracle.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)

# Seeds per config (one per tensor).
SEEDS = {
    "c1_x": 0x5EED0001, "c2_x": 0x5EED0002, "c3_x": 0x5EED0003, "c3_b": 0x5EED0004,
    "c4a_A": 0x5EED0005, "c4a_B": 0x5EED0006, "c4b_A": 0x5EED0007, "c4b_B": 0x5EED0008,
    "c5_Q": 0x5EED0009, "c5_K": 0x5EED000A, "c5_bias": 0x5EED000B,
}

NP_DTYPE = {"f16": np.float16, "f32": np.float32, "f64": np.float64}


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    with np.errstate(over="ignore"):
        i = np.arange(start, start + n, dtype=np.uint64)
        z = np.uint64(seed) + i * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        z = z ^ (z >> np.uint64(31))
    return z


def unit(seed: int, n: int) -> np.ndarray:
    """u in [0,1), 24-bit resolution, as f64."""
    return (splitmix64(seed, n) >> np.uint64(40)).astype(np.float64) * (2.0 ** -24)


def uniform(seed: int, n: int, lo: float, hi: float, dtype: str = "f32") -> np.ndarray:
    u = unit(seed, n)
    return (lo + (hi - lo) * u).astype(NP_DTYPE[dtype])


def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0, dtype: str = "f32") -> np.ndarray:
    m = n + (n & 1)
    u = unit(seed, m)
    u1 = 1.0 - u[0::2]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (mean + std * z[:n]).astype(NP_DTYPE[dtype])


def config_inputs(config: str, scale: dict | None = None) -> dict:
    """Seeded inputs for a config at its benchmark shape, or at the reduced
    shape given by ``scale`` (same generators, fewer elements)."""
    s = scale or {}
    if config == "c1":
        n = s.get("n", 1 << 24)
        return {"x": uniform(SEEDS["c1_x"], n, -4.0, 4.0)}
    if config == "c2":
        m, k = s.get("m", 8192), s.get("k", 4096)
        return {"x": normal(SEEDS["c2_x"], m * k, 0.0, 2.0).reshape(m, k)}
    if config == "c3":
        r, c = s.get("rows", 4096), s.get("cols", 4096)
        return {"x": uniform(SEEDS["c3_x"], r * c, -2.0, 2.0).reshape(r, c),
                "b": uniform(SEEDS["c3_b"], c, -1.0, 1.0)}
    if config == "c4a":
        m, k, n = s.get("m", 1024), s.get("k", 1024), s.get("n", 1024)
        return {"A": uniform(SEEDS["c4a_A"], m * k, -1.0, 1.0).reshape(m, k),
                "B": uniform(SEEDS["c4a_B"], k * n, -1.0, 1.0).reshape(k, n)}
    if config == "c4b":
        m, k, n = s.get("m", 4096), s.get("k", 4096), s.get("n", 4096)
        return {"A": uniform(SEEDS["c4b_A"], m * k, -1.0, 1.0, "f16").reshape(m, k),
                "B": uniform(SEEDS["c4b_B"], k * n, -1.0, 1.0, "f16").reshape(k, n)}
    if config == "c5":
        b, sq, d = s.get("batch", 16), s.get("seq", 2048), s.get("dim", 128)
        return {"Q": normal(SEEDS["c5_Q"], b * sq * d, 0.0, 1.0, "f16").reshape(b, sq, d),
                "K": normal(SEEDS["c5_K"], b * sq * d, 0.0, 1.0, "f16").reshape(b, sq, d),
                "bias": normal(SEEDS["c5_bias"], sq, 0.0, 0.1, "f32")}
    raise KeyError(config)
