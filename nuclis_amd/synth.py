"""Seeded synthetic inputs shared by the tests, smoke() and bench.py, and a
GGUF v3 writer for synthetic model files.

Generator: numpy PCG64 (`np.random.default_rng(seed)`), standard normal
draws in float32, scaled by the stated deviation. Weights are N(0, 0.02),
activations N(0, 1), as the benchmark configurations specify."""
import struct

import numpy as np


def gaussian(seed: int, shape, std: float = 1.0) -> np.ndarray:
    out = np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)
    if std != 1.0:
        out *= np.float32(std)
    return out


def _gstr(text) -> bytes:
    b = text.encode() if isinstance(text, str) else text
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, tensors, metadata=None, alignment=32) -> None:
    """GGUF v3 file: tensors = [(name, dims (GGUF order: columns first),
    encoding, raw bytes)]; metadata = [(key, tag, packed value bytes)].
    Tensor data is laid out in order, each at a multiple of `alignment`."""
    meta = [(b"general.architecture", 8, _gstr("nuq-test")), (b"general.alignment", 4, struct.pack("<I", alignment))]
    meta += [(k.encode() if isinstance(k, str) else k, t, v) for k, t, v in (metadata or [])]
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta)))
    for k, t, v in meta:
        out += _gstr(k) + struct.pack("<I", t) + v
    offsets, at = [], 0
    for _, _, _, raw in tensors:
        offsets.append(at)
        at += len(raw)
        at += (alignment - at % alignment) % alignment
    for (name, dims, enc, _), off in zip(tensors, offsets):
        out += _gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", enc, off)
    out += bytes((alignment - len(out) % alignment) % alignment)
    data = bytearray(at)
    for (_, _, _, raw), off in zip(tensors, offsets):
        data[off:off + len(raw)] = np.asarray(raw, dtype=np.uint8).tobytes()
    with open(path, "wb") as f:
        f.write(out)
        f.write(data)


# Seeds of the benchmark configurations (BASELINE.json `configs`), shared by
# the config tests and bench.py: name -> (encoding, rows N, columns K, weight
# seed). Activations: x seed 1 for the GEMVs, seed 4 for the M=8 verify
# activations, seed 5 for the prefill activations (N(0,1), f16 for the
# tiles).
CONFIGS = {
    "c1_q8_0": (8, 4096, 4096, 0),       # configs[0]: W from seed 0
    "c2_gate": (12, 17408, 5120, 2),     # configs[1] gate/up 5120 -> 17408
    "c2_down": (12, 5120, 17408, 3),     # configs[1] down 17408 -> 5120
    "c5_gate": (12, 17408, 5120, 2),     # configs[4] Q4_K gate
    "c5_down": (14, 5120, 17408, 3),     # configs[4] Q6_K down
}
X_SEED_GEMV, X_SEED_VERIFY, X_SEED_PREFILL = 1, 4, 5
