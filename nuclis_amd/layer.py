"""One decode step of a 27B-shaped dense layer plus lm_head (M = 1), composed
from the backend's entry points, and its greedy argmax.

The shape and order follow nuclis's Metal plan for a full-attention layer at
the first position (models/qwen35_metal.zig:1593-1616, :637-639, :664-670):
single-token attention at visible=1 has softmax = 1, so the attention output
is V repeated across each KV head's query-head group (GQA 6x here); then
  h1 = x + W_o * repeat6(W_v * x)        (q and k are computed as the merged
                                          q/k/v projection does, but do not
                                          contribute at position 0)
  h2 = h1 + W_down * (silu(W_gate * h1) * (W_up * h1))
  logits = W_lm_head * h2,  token = argmax(logits)
Norms are omitted (the configuration is the projections and lm_head).
All projections run in libnuq.so; torch only moves data (residual adds and
the GQA gather are torch element-wise ops on device tensors).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import backend as nb
from .synth import gaussian

HIDDEN = 5120
Q_ROWS, KV_ROWS, FFN, VOCAB = 6144, 1024, 17408, 151936
HEAD_DIM, GQA = 128, 6

# name -> (encoding, rows, columns, seed)
SHAPES = {
    "q": (nb.Q4_K, Q_ROWS, HIDDEN, 10),
    "k": (nb.Q4_K, KV_ROWS, HIDDEN, 11),
    "v": (nb.Q4_K, KV_ROWS, HIDDEN, 12),
    "o": (nb.Q4_K, HIDDEN, Q_ROWS, 13),
    "gate": (nb.Q4_K, FFN, HIDDEN, 14),
    "up": (nb.Q4_K, FFN, HIDDEN, 15),
    "down": (nb.Q4_K, HIDDEN, FFN, 16),
    "lm_head": (nb.Q6_K, VOCAB, HIDDEN, 17),
}


def quantized_weights(scale_rows: float = 1.0) -> dict[str, np.ndarray]:
    """Seeded N(0, 0.02) weights quantized to their GGUF encodings (host).
    `scale_rows` < 1 keeps only the first rows of lm_head (for quick tests)."""
    out = {}
    for name, (enc, rows, cols, seed) in SHAPES.items():
        if name == "lm_head" and scale_rows < 1.0:
            rows = max(256, int(rows * scale_rows) // 256 * 256)
        out[name] = nb.quantize(enc, gaussian(seed, (rows, cols), 0.02))
    return out


def weight_bytes(weights: dict[str, np.ndarray]) -> int:
    return int(sum(w.nbytes for w in weights.values()))


@dataclass
class DeviceLayer:
    mats: dict
    buffers: dict


def upload(weights: dict[str, np.ndarray]) -> DeviceLayer:
    import torch
    mats = {}
    for name, w in weights.items():
        enc, _, cols, _ = SHAPES[name]
        mats[name] = nb.Matrix(enc, w.shape[0], cols, torch.from_numpy(w).cuda())
    dev = "cuda"
    bufs = {
        "qkv": torch.empty(Q_ROWS + 2 * KV_ROWS, device=dev),
        "h1": torch.empty(HIDDEN, device=dev),
        "attn_o": torch.empty(HIDDEN, device=dev),
        "act": torch.empty(FFN, device=dev),
        "h2": torch.empty(HIDDEN, device=dev),
        "down": torch.empty(HIDDEN, device=dev),
        "logits": torch.empty(mats["lm_head"].rows, device=dev),
        "attn": torch.empty(Q_ROWS, device=dev),
        "gqa_index": (torch.arange(Q_ROWS, device=dev) // (HEAD_DIM * GQA)) * HEAD_DIM
                     + torch.arange(Q_ROWS, device=dev) % HEAD_DIM,
    }
    return DeviceLayer(mats, bufs)


def step(backend: nb.Backend, layer: DeviceLayer, x) -> None:
    """Enqueues one decode step for device vector x (F32, HIDDEN); logits end
    in layer.buffers['logits']."""
    m, b = layer.mats, layer.buffers
    qkv = b["qkv"]
    q, k, v = qkv[:Q_ROWS], qkv[Q_ROWS:Q_ROWS + KV_ROWS], qkv[Q_ROWS + KV_ROWS:]
    backend.matvec_segments([(m["q"], q), (m["k"], k), (m["v"], v)], x, nb.SEGMENT_PLAIN)
    torch_gather(v, b["gqa_index"], b["attn"])  # GQA: query head j reads KV head j // 6
    backend.matvec(m["o"], b["attn"], b["attn_o"])
    h1 = b["h1"]
    torch_add(x, b["attn_o"], h1)
    backend.matvec_segments([(m["gate"], b["act"]), (m["up"], b["act"])], h1, nb.SEGMENT_SILU_MUL_PAIR)
    backend.matvec(m["down"], b["act"], b["down"])
    torch_add(h1, b["down"], b["h2"])
    backend.matvec(m["lm_head"], b["h2"], b["logits"])


def torch_gather(src, index, out) -> None:
    import torch
    torch.index_select(src, 0, index, out=out)


def torch_add(a, c, out) -> None:
    import torch
    torch.add(a, c, out=out)


def run(backend: nb.Backend, layer: DeviceLayer, x) -> int:
    step(backend, layer, x)
    return backend.argmax(layer.buffers["logits"])
