"""CPU composition of the configuration-3 decode step (one 27B-shaped layer
plus the Q6_K lm_head at M=1) from the oracle's matvec. TEST
INFRASTRUCTURE ONLY: tests/ and bench.py's checks use it to confirm the GPU
step's greedy token; the product path never imports it.

The operations follow the reference's CPU path: matvecs with F64
accumulation (backends/cpu/root.zig:112-165) and silu(x) = f32(x *
logistic(x)) with logistic in F64 in its two-branch form
(backends/cpu/vector.zig:177-196). At the first position single-token
attention has softmax = 1, so query head h outputs the values of KV head
h // (query_heads / kv_heads) (backends/metal/kernels/attention.metal:40).
The step's shape is the one nuclis_amd/layer.py runs
(models/qwen35_metal.zig:1593-1616, :637-639).

Pinned by tests/test_layer_oracle.py against an independent numpy
construction (decoded matrices, np.repeat for the head broadcast,
scipy's expit for the logistic).
"""
from __future__ import annotations

import numpy as np

from . import oracle as orc

HEAD_DIM = 128


def logistic(g: np.ndarray) -> np.ndarray:
    """vector.zig:191-196, F64: 1/(1+e^-x) for x >= 0, e^x/(1+e^x) below."""
    g = np.asarray(g, np.float64)
    out = np.empty_like(g)
    pos = g >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-g[pos]))
    e = np.exp(g[~pos])
    out[~pos] = e / (1.0 + e)
    return out


def silu(g: np.ndarray) -> np.ndarray:
    """vector.zig:177-181: f32(f64(x) * logistic(x)); -Inf -> -0."""
    g = np.asarray(g, np.float32)
    with np.errstate(invalid="ignore"):  # -Inf * 0, replaced below
        out = (g.astype(np.float64) * logistic(g)).astype(np.float32)
    return np.where(np.isneginf(g), np.float32(-0.0), out)


def cpu_step(shapes: dict, weights: dict, x: np.ndarray) -> np.ndarray:
    """shapes: name -> (encoding, rows, columns, seed); weights: name -> raw
    GGUF bytes [rows][stride]. The query width is o's column count and the
    KV width v's row count, both whole 128-value heads. Returns the F32
    logits."""
    def mv(name, v):
        enc, _, cols, _ = shapes[name]
        w = weights[name]
        return orc.matvec(enc, w.shape[0], cols, w, v)
    q_rows, kv_rows = shapes["o"][2], shapes["v"][1]
    group = (q_rows // HEAD_DIM) // (kv_rows // HEAD_DIM)  # query heads per KV head
    v = mv("v", x)
    r = np.arange(q_rows)
    idx = (r // HEAD_DIM) // group * HEAD_DIM + r % HEAD_DIM  # kv head of query head r // 128
    h1 = (x + mv("o", v[idx])).astype(np.float32)
    g = mv("gate", h1)
    u = mv("up", h1)
    act = (silu(g) * u).astype(np.float32)
    h2 = (h1 + mv("down", act)).astype(np.float32)
    return mv("lm_head", h2)
