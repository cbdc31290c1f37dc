"""Seeded synthetic inputs for the benchmark configurations.

The reference has no normal generator of its own (its tools draw xorshift
uniforms), so the harness owns generation: numpy's PCG64 stream with a fixed
seed per tensor name, N(0, sigma) in float32.  The same image on every box
gives the same bytes, which is what lets the GPU backend and the reference
CPU build see identical inputs.
"""
from __future__ import annotations

import zlib

import numpy as np

BASE_SEED = 20261201


def seed_for(name: str) -> int:
    return BASE_SEED ^ zlib.crc32(name.encode())


def normal(name: str, shape, sigma: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed_for(name))
    out = rng.standard_normal(size=shape, dtype=np.float32)
    if sigma != 1.0:
        out *= np.float32(sigma)
    return out


def bernoulli_mask(name: str, shape, p_keep: float = 0.5) -> np.ndarray:
    rng = np.random.default_rng(seed_for(name))
    return (rng.random(size=shape) < p_keep).astype(np.uint8)
