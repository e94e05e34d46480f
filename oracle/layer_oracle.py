"""CPU composition of the configuration-3 decode step (one 27B-shaped layer
plus the Q6_K lm_head at M=1) from the oracle's matvec. TEST
INFRASTRUCTURE ONLY: tests/ and bench.py's checks use it to confirm the GPU
step's greedy token; the product path never imports it.

The operations follow the reference's CPU path: matvecs with F64
accumulation (backends/cpu/root.zig:112-165) and silu(x) = f32(x *
logistic(x)) in F64 (cpu/vector.zig:178-181). The step's shape is the one
nuclis_amd/layer.py runs (models/qwen35_metal.zig:1593-1616, :637-639).
"""
from __future__ import annotations

import numpy as np

from . import oracle as orc

HIDDEN, Q_ROWS, HEAD_DIM, GQA = 5120, 6144, 128, 6


def cpu_step(shapes: dict, weights: dict, x: np.ndarray) -> np.ndarray:
    """shapes: name -> (encoding, rows, columns, seed); weights: name -> raw
    GGUF bytes [rows][stride]. Returns the F32 logits."""
    def mv(name, v):
        enc, _, cols, _ = shapes[name]
        w = weights[name]
        return orc.matvec(enc, w.shape[0], cols, w, v)
    v = mv("v", x)
    idx = (np.arange(Q_ROWS) // (HEAD_DIM * GQA)) * HEAD_DIM + np.arange(Q_ROWS) % HEAD_DIM
    h1 = (x + mv("o", v[idx])).astype(np.float32)
    g = mv("gate", h1).astype(np.float64)
    u = mv("up", h1)
    silu = (g / (1.0 + np.exp(-g))).astype(np.float32)
    act = (silu * u).astype(np.float32)
    h2 = (h1 + mv("down", act)).astype(np.float32)
    return mv("lm_head", h2)
