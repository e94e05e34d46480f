"""Pure-Python GGUF v3 directory reader. TEST INFRASTRUCTURE ONLY.

A second, independent restatement of gguf.parseDiagnosed
(inference/src/formats/gguf.zig:311-410) and gguf.ArrayReader
(gguf.zig:63-104), used only by tests/ as the checker of libnuq's C++ reader.
The product never imports it.

`parse(data, file_bytes, limits)` returns a Document or raises GgufError whose
`.name` is the Zig error name. Pinning: tests/test_gguf.py runs the
reference's own cases (gguf.zig:424-772: the wire fixture, every rejection
case, the limits, truncations, retained arrays) against this module and
against libnuq, and differential-fuzzes the two.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

# gguf.Limits (gguf.zig:13-19)
DEFAULT_LIMITS = dict(directory_bytes=64 * 1024 * 1024, metadata_count=16_384, tensor_count=100_000,
                      string_bytes=1024 * 1024, array_items=4_000_000)
RETAINED_ARRAY_ITEMS = 64  # gguf.zig:41
RETAINED_KEY_PREFIXES = ("prism.hadamard.",)  # gguf.zig:46
RETAINED_PREFIXED_ITEMS = 65_536  # gguf.zig:47

# gguf.Type (gguf.zig:21-35)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOLEAN, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", UINT64: "<Q",
           INT64: "<q", FLOAT32: "<f", FLOAT64: "<d"}
_SIZE = {UINT8: 1, INT8: 1, UINT16: 2, INT16: 2, UINT32: 4, INT32: 4, FLOAT32: 4, UINT64: 8, INT64: 8, FLOAT64: 8}

# encoding.layout (inference/src/tensor/encoding.zig:29-56): (elements per block, bytes per block)
LAYOUTS = {0: (1, 4), 1: (1, 2), 2: (32, 18), 6: (32, 22), 7: (32, 24), 8: (32, 34), 10: (256, 84),
           11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 16: (256, 66), 17: (256, 74),
           18: (256, 98), 19: (256, 50), 20: (32, 18), 21: (256, 110), 22: (256, 82), 23: (256, 136),
           29: (256, 56), 30: (1, 2), 142: (128, 34), 143: (128, 28)}

U64_MAX = (1 << 64) - 1


class GgufError(Exception):
    def __init__(self, name: str):
        super().__init__(name)
        self.name = name


@dataclass
class Value:
    kind: str  # unsigned / signed / float / boolean / string / array
    type: int
    value: object = None  # int / float / bool / bytes
    element_type: int = 0
    count: int = 0
    file_offset: int = 0
    values: list | None = None


@dataclass
class Tensor:
    name: bytes
    dimensions: tuple
    encoding_id: int
    offset: int
    bytes: int
    elements: int


@dataclass
class Document:
    version: int
    file_bytes: int
    directory_bytes: int
    data_offset: int
    alignment: int
    metadata: list = field(default_factory=list)  # (key bytes, type, Value)
    tensors: list = field(default_factory=list)

    def get(self, key: bytes):
        for k, _, v in self.metadata:
            if k == key:
                return v
        return None


@dataclass
class Rejection:
    tensor: bytes | None = None
    encoding_id: int | None = None


def _mul(a: int, b: int) -> int:
    r = a * b
    if r > U64_MAX:
        raise GgufError("Overflow")
    return r


def byte_count(layout, dims) -> int:
    """Layout.byteCount (encoding.zig:15-24)."""
    epb, bpb = layout
    if not dims or dims[0] == 0 or dims[0] % epb:
        raise GgufError("InvalidShape")
    b = _mul(dims[0] // epb, bpb)
    for d in dims[1:]:
        if d == 0:
            raise GgufError("InvalidShape")
        b = _mul(b, d)
    return b


def _validate_name(name: bytes) -> None:
    """validateName (gguf.zig:273-277)."""
    if len(name) == 0 or len(name) > 65_535:
        raise GgufError("InvalidName")
    try:
        name.decode("utf-8", errors="strict")
    except UnicodeDecodeError:
        raise GgufError("InvalidName")
    if any(b < 0x20 or b == 0x7F for b in name):
        raise GgufError("InvalidName")


class _Cursor:
    """gguf.zig:174-266."""

    def __init__(self, data: bytes, file_bytes: int, limits: dict):
        self.data, self.file_bytes, self.limits, self.position = data, file_bytes, limits, 0

    def advance(self, n: int) -> None:
        if self.position > self.file_bytes or n > self.file_bytes - self.position:
            raise GgufError("EndOfStream")
        lim = self.limits["directory_bytes"]
        if self.position > lim or n > lim - self.position:
            raise GgufError("LimitExceeded")
        self.position += n

    def take(self, n: int) -> bytes:
        start = self.position
        self.advance(n)
        if self.position > len(self.data):
            raise GgufError("EndOfStream")
        return self.data[start:self.position]

    def int(self, fmt: str) -> int:
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> bytes:
        n = self.int("<Q")
        if n > self.limits["string_bytes"]:
            raise GgufError("LimitExceeded")
        return self.take(n)

    def kind(self) -> int:
        t = self.int("<I")
        if t > FLOAT64:
            raise GgufError("InvalidMetadataType")
        return t

    def value(self, tag: int, retain: bool) -> Value:
        if tag in (UINT8, UINT16, UINT32, UINT64):
            return Value("unsigned", tag, self.int(_SCALAR[tag]))
        if tag in (INT8, INT16, INT32, INT64):
            return Value("signed", tag, self.int(_SCALAR[tag]))
        if tag in (FLOAT32, FLOAT64):
            return Value("float", tag, self.int(_SCALAR[tag]))
        if tag == BOOLEAN:
            b = self.int("<B")
            if b > 1:
                raise GgufError("InvalidBoolean")
            return Value("boolean", tag, bool(b))
        if tag == STRING:
            return Value("string", tag, self.string())
        # array
        element = self.kind()
        if element == ARRAY:
            raise GgufError("UnsupportedNestedArray")
        count = self.int("<Q")
        if count > self.limits["array_items"]:
            raise GgufError("LimitExceeded")
        arr = Value("array", tag, element_type=element, count=count, file_offset=self.position)
        if retain and count > RETAINED_PREFIXED_ITEMS:
            raise GgufError("LimitExceeded")
        if retain or (element != STRING and count <= RETAINED_ARRAY_ITEMS):
            arr.values = [self.value(element, False) for _ in range(count)]
        elif element == STRING:
            for _ in range(count):
                n = self.int("<Q")
                if n > self.limits["string_bytes"]:
                    raise GgufError("LimitExceeded")
                self.take(n)
        elif element == BOOLEAN:
            for _ in range(count):
                if self.int("<B") > 1:
                    raise GgufError("InvalidBoolean")
        else:
            self.take(_mul(count, _SIZE[element]))
        return arr


def parse(data: bytes, file_bytes: int | None = None, limits: dict | None = None,
          rejection: Rejection | None = None) -> Document:
    """gguf.parseDiagnosed (gguf.zig:311-410)."""
    lim = dict(DEFAULT_LIMITS, **(limits or {}))
    if file_bytes is None:
        file_bytes = len(data)
    data = bytes(data[:file_bytes])
    c = _Cursor(data, file_bytes, lim)
    if c.int("<I") != 0x46554747:
        raise GgufError("InvalidMagic")
    version = c.int("<I")
    if version != 3:
        raise GgufError("UnsupportedVersion")
    tensor_count = c.int("<Q")
    metadata_count = c.int("<Q")
    if tensor_count > lim["tensor_count"] or metadata_count > lim["metadata_count"]:
        raise GgufError("LimitExceeded")
    metadata, keys, alignment = [], set(), 32
    for _ in range(metadata_count):
        key = c.string()
        _validate_name(key)
        if key in keys:
            raise GgufError("DuplicateMetadata")
        keys.add(key)
        tag = c.kind()
        value = c.value(tag, any(key.startswith(p.encode()) for p in RETAINED_KEY_PREFIXES))
        metadata.append((key, tag, value))
        if key == b"general.alignment":
            if tag != UINT32:
                raise GgufError("InvalidAlignment")
            alignment = value.value
            if alignment == 0 or alignment & (alignment - 1):
                raise GgufError("InvalidAlignment")
    tensors, names = [], set()
    for _ in range(tensor_count):
        name = c.string()
        _validate_name(name)
        if name in names:
            raise GgufError("DuplicateTensor")
        names.add(name)
        rank = c.int("<I")
        if rank == 0 or rank > 4:
            if rejection is not None:
                rejection.tensor, rejection.encoding_id = name[:128], None
            raise GgufError("InvalidShape")
        dims = tuple(c.int("<Q") for _ in range(rank))
        enc = c.int("<I")
        try:
            elements = 1
            for d in dims:
                if d == 0:
                    raise GgufError("InvalidShape")
                elements = _mul(elements, d)
            if enc not in LAYOUTS:
                raise GgufError("UnsupportedTensorType")
            nbytes = byte_count(LAYOUTS[enc], dims)
        except GgufError:
            if rejection is not None:
                rejection.tensor, rejection.encoding_id = name[:128], enc
            raise
        offset = c.int("<Q")
        if offset % alignment:
            raise GgufError("InvalidAlignment")
        tensors.append(Tensor(name, dims, enc, offset, nbytes, elements))
    padding = (alignment - c.position % alignment) % alignment
    data_offset = c.position + padding
    if data_offset > file_bytes:
        raise GgufError("EndOfStream")
    previous_end = 0
    for t in sorted(tensors, key=lambda t: t.offset):
        if t.offset > file_bytes - data_offset or t.bytes > file_bytes - data_offset - t.offset:
            raise GgufError("TensorOutOfBounds")
        if t.offset < previous_end:
            raise GgufError("OverlappingTensors")
        previous_end = t.offset + t.bytes
    return Document(version, file_bytes, c.position, data_offset, alignment, metadata, tensors)


def read_array(element_type: int, count: int, file_offset: int, directory: bytes, limits: dict | None = None):
    """ArrayReader.init then next* until the end (gguf.zig:63-104): a list of
    values, or GgufError at the failing step (after the values read so far)."""
    lim = dict(DEFAULT_LIMITS, **(limits or {}))
    if len(directory) > lim["directory_bytes"] or count > lim["array_items"]:
        raise GgufError("LimitExceeded")
    if element_type not in (STRING, INT32):
        raise GgufError("InvalidMetadataType")
    if file_offset > len(directory):
        raise GgufError("EndOfStream")
    b = directory[file_offset:]
    minimum = 8 if element_type == STRING else 4
    if count > len(b) // minimum:
        raise GgufError("EndOfStream")
    out = []
    for _ in range(count):
        if element_type == STRING:
            if len(b) < 8:
                raise GgufError("EndOfStream")
            n = struct.unpack("<Q", b[:8])[0]
            if n > lim["string_bytes"]:
                raise GgufError("LimitExceeded")
            if n > len(b) - 8:
                raise GgufError("EndOfStream")
            out.append(b[8:8 + n])
            b = b[8 + n:]
        else:
            if len(b) < 4:
                raise GgufError("EndOfStream")
            out.append(struct.unpack("<i", b[:4])[0])
            b = b[4:]
    return out
