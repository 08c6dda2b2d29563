"""Seeded synthetic inputs (counter-based splitmix64), identical on every host.

Element i of a stream with seed s is splitmix64(s + (i + 1) * 0x9E3779B97F4A7C15),
so any slice of a tensor can be regenerated independently.  Uniform floats use
the top 24 bits (exact in float32); normals use Box-Muller in float64 on two
independent streams; every result is rounded once to float32.
"""
from __future__ import annotations

import zlib

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def bits(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        idx = np.arange(1, n + 1, dtype=np.uint64)
        return _mix(np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN)


def uniform(seed: int, shape, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    u = (bits(seed, n) >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    u1 = ((bits(seed, n) >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / (1 << 53))
    u2 = (bits(seed ^ 0x5DEECE66D, n) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + std * z).astype(np.float32).reshape(shape)


def randint(seed: int, shape, lo: int, hi: int, dtype=np.int32) -> np.ndarray:
    """Uniform integers in [lo, hi] inclusive."""
    n = int(np.prod(shape))
    span = np.uint64(hi - lo + 1)
    r = ((bits(seed, n) >> np.uint64(32)) * span) >> np.uint64(32)
    return (r.astype(np.int64) + lo).astype(dtype).reshape(shape)


def layer_seed(model_seed: int, name: str, part: int) -> int:
    """Seed of tensor `part` (0: weights, 1: bias) of the layer called `name`
    (its ONNX node name) in a model generated from `model_seed`: a layer's
    random weights depend on its name only, not on where a builder creates it."""
    return (int(model_seed) << 40) + (zlib.crc32(name.encode()) << 2) + int(part)
