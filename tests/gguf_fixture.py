"""GGUF wire-format builders for the tests.

`fixture(**options)` writes the same bytes as the reference's test fixture
(inference/src/formats/gguf.zig:424-471, FixtureOptions and fixture()): the
header, three metadata entries (architecture, alignment, a two-string token
array), two rank-1 tensors and 64 bytes of zero data. `write_model` (in
nuclis_amd.synth) writes real GGUF v3 files for the device-upload tests.
"""
from __future__ import annotations

import struct

from nuclis_amd.synth import write_gguf as write_model  # noqa: F401


def gstr(text) -> bytes:
    b = text.encode() if isinstance(text, str) else text
    return struct.pack("<Q", len(b)) + b


def fixture(version=3, alignment=32, duplicate_metadata=False, duplicate_tensor=False, second_offset=32,
            encoding_id=0, dimension=4) -> bytes:
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, 2, 3)
    out += gstr("general.architecture") + struct.pack("<I", 8) + gstr("fixture")
    out += gstr("general.architecture" if duplicate_metadata else "general.alignment")
    out += struct.pack("<II", 4, alignment)
    out += gstr("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 2) + gstr("a") + gstr("unicode: λ")
    for i in range(2):
        out += gstr("first" if i == 0 or duplicate_tensor else "second")
        out += struct.pack("<IQIQ", 1, dimension, encoding_id, 0 if i == 0 else second_offset)
    out += bytes((32 - len(out) % 32) % 32)
    out += bytes(64)
    return bytes(out)


# Byte offset of the first metadata entry's type tag: the 24-byte fixed
# header, the key's length, then the key (gguf.zig:666).
FIRST_TAG = 24 + 8 + len("general.architecture")


def header(tensors: int, metadata: int) -> bytes:
    return b"GGUF" + struct.pack("<IQQ", 3, tensors, metadata)


def array_i32(key: str, values) -> bytes:
    return gstr(key) + struct.pack("<IIQ", 9, 5, len(values)) + b"".join(struct.pack("<i", v) for v in values)


def array_str(key: str, values) -> bytes:
    return gstr(key) + struct.pack("<IIQ", 9, 8, len(values)) + b"".join(gstr(v) for v in values)


def pad32(b: bytes) -> bytes:
    return b + bytes((32 - len(b) % 32) % 32)
