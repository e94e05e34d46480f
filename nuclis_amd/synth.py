"""Seeded synthetic inputs shared by the tests, smoke() and bench.py.

Generator: numpy PCG64 (`np.random.default_rng(seed)`), standard normal
draws in float32, scaled by the stated deviation. Weights are N(0, 0.02),
activations N(0, 1), as the benchmark configurations specify."""
import numpy as np


def gaussian(seed: int, shape, std: float = 1.0) -> np.ndarray:
    out = np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)
    if std != 1.0:
        out *= np.float32(std)
    return out
