"""GGUF v3 files into device weights, over libnuq's C ABI (include/nuq_gguf.h).

Mirrors nuclis's loader surface:
  - parse(bytes, file_bytes, limits, rejection) / open(path): gguf.parse,
    gguf.parseDiagnosed (inference/src/formats/gguf.zig:311-410) and
    weights.Mapped.open (runtime/weights.zig:63-78); errors are GgufError
    whose `.name` is the Zig error name.
  - Document.get / Document.string (gguf.zig:141-153), Document.tensors.
  - ArrayReader (gguf.zig:63-104) for lazy string / int32 arrays.
  - Document.tensor_bytes / Document.host_matrix: weights.View.bytes and
    View.matrix (runtime/weights.zig:11-19) on the host mapping.
  - upload(backend, doc): the tensor-data section into one device buffer;
    DeviceWeights.matrix(name) is the device twin of View.matrix.
The parsing and the copy run in libnuq; nothing here decodes weights.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

from .backend import Matrix, _Matrix, lib

# gguf.Type (gguf.zig:21-35)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOLEAN, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)

_STATUS = {
    1: "InvalidShape", 7: "InvalidArgument", 20: "EndOfStream", 21: "InvalidMagic", 22: "UnsupportedVersion",
    23: "LimitExceeded", 24: "InvalidMetadataType", 25: "UnsupportedNestedArray", 26: "InvalidBoolean",
    27: "InvalidName", 28: "DuplicateMetadata", 29: "DuplicateTensor", 30: "InvalidAlignment", 31: "Overflow",
    32: "UnsupportedTensorType", 33: "TensorOutOfBounds", 34: "OverlappingTensors", 35: "OutOfMemory",
    36: "NotRegularFile", 37: "FileError", 38: "NotFound", 6: "DeviceError",
}
_NOT_FOUND = 38

EXPORTS = [
    "nuq_gguf_default_limits", "nuq_gguf_parse", "nuq_gguf_open", "nuq_gguf_close", "nuq_gguf_info_get",
    "nuq_gguf_metadata", "nuq_gguf_get", "nuq_gguf_array_value", "nuq_gguf_tensor_get", "nuq_gguf_find_tensor",
    "nuq_gguf_directory", "nuq_gguf_array_reader_init", "nuq_gguf_array_next_string", "nuq_gguf_array_next_int32",
    "nuq_gguf_tensor_bytes", "nuq_gguf_matrix", "nuq_gguf_data_bytes", "nuq_gguf_upload",
]


class GgufError(Exception):
    """A gguf.Error (gguf.zig:156-172); `.name` is the Zig error name."""

    def __init__(self, code: int, message: str = ""):
        self.code = code
        self.name = _STATUS.get(code, f"status {code}")
        super().__init__(message or self.name)


class _Limits(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in
                ("directory_bytes", "metadata_count", "tensor_count", "string_bytes", "array_items")]


class _Value(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_uint32), ("type", ctypes.c_uint32), ("u", ctypes.c_uint64), ("i", ctypes.c_int64),
                ("f", ctypes.c_double), ("string", ctypes.c_void_p), ("string_len", ctypes.c_uint64),
                ("element_type", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("count", ctypes.c_uint64),
                ("file_offset", ctypes.c_uint64), ("retained", ctypes.c_uint64)]


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_void_p), ("name_len", ctypes.c_uint64), ("rank", ctypes.c_uint32),
                ("encoding", ctypes.c_uint32), ("dimensions", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64),
                ("bytes", ctypes.c_uint64), ("elements", ctypes.c_uint64)]


class _Info(ctypes.Structure):
    _fields_ = [("version", ctypes.c_uint32), ("alignment", ctypes.c_uint32), ("file_bytes", ctypes.c_uint64),
                ("directory_bytes", ctypes.c_uint64), ("data_offset", ctypes.c_uint64),
                ("metadata_count", ctypes.c_uint64), ("tensor_count", ctypes.c_uint64)]


class _Rejection(ctypes.Structure):
    _fields_ = [("tensor", ctypes.c_char * 128), ("len", ctypes.c_uint32), ("has_encoding", ctypes.c_uint32),
                ("encoding", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class _ArrayReader(ctypes.Structure):
    _fields_ = [("bytes", ctypes.c_void_p), ("len", ctypes.c_uint64), ("remaining", ctypes.c_uint64),
                ("kind", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("string_bytes", ctypes.c_uint64)]


_bound = False


def _L():
    global _bound
    L = lib()
    if not _bound:
        vp, u32, u64, P = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.POINTER
        L.nuq_gguf_default_limits.argtypes = [P(_Limits)]
        L.nuq_gguf_default_limits.restype = None
        L.nuq_gguf_parse.argtypes = [vp, u64, u64, P(_Limits), P(vp), P(_Rejection)]
        L.nuq_gguf_open.argtypes = [ctypes.c_char_p, P(_Limits), P(vp), P(_Rejection)]
        L.nuq_gguf_close.argtypes = [vp]
        L.nuq_gguf_close.restype = None
        L.nuq_gguf_info_get.argtypes = [vp, P(_Info)]
        L.nuq_gguf_metadata.argtypes = [vp, u64, P(vp), P(u64), P(_Value)]
        L.nuq_gguf_get.argtypes = [vp, ctypes.c_char_p, u64, P(_Value)]
        L.nuq_gguf_array_value.argtypes = [vp, u64, u64, P(_Value)]
        L.nuq_gguf_tensor_get.argtypes = [vp, u64, P(_Tensor)]
        L.nuq_gguf_find_tensor.argtypes = [vp, ctypes.c_char_p, u64, P(u64)]
        L.nuq_gguf_directory.argtypes = [vp, P(vp), P(u64)]
        L.nuq_gguf_array_reader_init.argtypes = [P(_ArrayReader), u32, u64, u64, vp, u64, P(_Limits)]
        L.nuq_gguf_array_next_string.argtypes = [P(_ArrayReader), P(vp), P(u64), P(ctypes.c_int)]
        L.nuq_gguf_array_next_int32.argtypes = [P(_ArrayReader), P(ctypes.c_int32), P(ctypes.c_int)]
        L.nuq_gguf_tensor_bytes.argtypes = [vp, u64, P(vp), P(u64)]
        L.nuq_gguf_matrix.argtypes = [vp, u64, vp, P(_Matrix)]
        L.nuq_gguf_data_bytes.argtypes = [vp]
        L.nuq_gguf_data_bytes.restype = u64
        L.nuq_gguf_upload.argtypes = [vp, vp, vp, u64]
        _bound = True
    return L


def _check(code: int, message: str = "") -> None:
    if code != 0:
        raise GgufError(code, message)


def default_limits() -> dict:
    """gguf.Limits defaults (gguf.zig:13-19)."""
    lim = _Limits()
    _L().nuq_gguf_default_limits(ctypes.byref(lim))
    return {n: getattr(lim, n) for n, _ in _Limits._fields_}


def _limits(limits: dict | None):
    if limits is None:
        return None
    lim = _Limits()
    _L().nuq_gguf_default_limits(ctypes.byref(lim))
    for k, v in limits.items():
        setattr(lim, k, v)
    return ctypes.byref(lim)


@dataclass
class Value:
    """gguf.Value (gguf.zig:105-112) with gguf.Array's fields for arrays.
    `value` is an int, float, bool or bytes; arrays carry `values` when the
    directory retained them (else None: read them with ArrayReader)."""

    kind: str
    type: int
    value: object = None
    element_type: int = 0
    count: int = 0
    file_offset: int = 0
    values: list | None = None


_KINDS = ("unsigned", "signed", "float", "boolean", "string", "array")


def _value(v: _Value) -> Value:
    kind = _KINDS[v.kind]
    if kind == "unsigned":
        return Value(kind, v.type, v.u)
    if kind == "signed":
        return Value(kind, v.type, v.i)
    if kind == "float":
        return Value(kind, v.type, v.f)
    if kind == "boolean":
        return Value(kind, v.type, bool(v.u))
    if kind == "string":
        return Value(kind, v.type, ctypes.string_at(v.string, v.string_len) if v.string_len else b"")
    return Value(kind, v.type, None, v.element_type, v.count, v.file_offset)


@dataclass
class Tensor:
    """gguf.Tensor (gguf.zig:114-122); offset is relative to data_offset."""

    name: bytes
    dimensions: tuple
    encoding_id: int
    offset: int
    bytes: int
    elements: int


@dataclass
class Rejection:
    """gguf.Rejection (gguf.zig:287-301)."""

    tensor: bytes | None = None
    encoding_id: int | None = None


class Document:
    """A parsed directory (gguf.Document, gguf.zig:124-154). A document made
    by parse() borrows the bytes it was given and keeps a reference to them."""

    def __init__(self, handle: int, keep=None):
        self._h = handle
        self._keep = keep
        info = _Info()
        _check(_L().nuq_gguf_info_get(self._h, ctypes.byref(info)))
        self.version = info.version
        self.alignment = info.alignment
        self.file_bytes = info.file_bytes
        self.directory_bytes = info.directory_bytes
        self.data_offset = info.data_offset
        self.metadata = [self._metadata(i) for i in range(info.metadata_count)]
        self.tensors = [self._tensor(i) for i in range(info.tensor_count)]

    def _metadata(self, i: int):
        key, key_len, v = ctypes.c_void_p(), ctypes.c_uint64(), _Value()
        _check(_L().nuq_gguf_metadata(self._h, i, ctypes.byref(key), ctypes.byref(key_len), ctypes.byref(v)))
        value = _value(v)
        if value.kind == "array" and v.retained:
            items = []
            for k in range(v.retained):
                item = _Value()
                _check(_L().nuq_gguf_array_value(self._h, i, k, ctypes.byref(item)))
                items.append(_value(item))
            value.values = items
        return ctypes.string_at(key, key_len.value), v.type, value

    def _tensor(self, i: int) -> Tensor:
        t = _Tensor()
        _check(_L().nuq_gguf_tensor_get(self._h, i, ctypes.byref(t)))
        return Tensor(ctypes.string_at(t.name, t.name_len), tuple(t.dimensions[:t.rank]), t.encoding, t.offset,
                      t.bytes, t.elements)

    def close(self) -> None:
        if self._h:
            _L().nuq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def get(self, key) -> Value | None:
        key = key.encode() if isinstance(key, str) else key
        for k, _, v in self.metadata:
            if k == key:
                return v
        return None

    def string(self, key) -> bytes | None:
        v = self.get(key)
        return v.value if v is not None and v.kind == "string" else None

    def index(self, name) -> int:
        name = name.encode() if isinstance(name, str) else name
        idx = ctypes.c_uint64()
        _check(_L().nuq_gguf_find_tensor(self._h, name, len(name), ctypes.byref(idx)), f"no tensor {name!r}")
        return idx.value

    def directory(self) -> bytes:
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        _check(_L().nuq_gguf_directory(self._h, ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p, n.value) if n.value else b""

    def tensor_bytes(self, name) -> bytes:
        """weights.View.bytes (runtime/weights.zig:11-15), copied out."""
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        _check(_L().nuq_gguf_tensor_bytes(self._h, self.index(name), ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p, n.value)

    def host_matrix(self, name) -> _Matrix:
        """weights.View.matrix (runtime/weights.zig:16-19) on the host mapping."""
        m = _Matrix()
        _check(_L().nuq_gguf_matrix(self._h, self.index(name), None, ctypes.byref(m)))
        return m

    @property
    def data_bytes(self) -> int:
        return _L().nuq_gguf_data_bytes(self._h)


def parse(data, file_bytes: int | None = None, limits: dict | None = None,
          rejection: Rejection | None = None) -> Document:
    """gguf.parseDiagnosed over `data` (bytes-like) of a file `file_bytes` long."""
    buf = bytes(data)
    if file_bytes is None:
        file_bytes = len(buf)
    h = ctypes.c_void_p()
    rej = _Rejection()
    code = _L().nuq_gguf_parse(buf, len(buf), file_bytes, _limits(limits), ctypes.byref(h),
                               ctypes.byref(rej) if rejection is not None else None)
    if code != 0:
        if rejection is not None and rej.len:
            rejection.tensor = bytes(rej.tensor[:rej.len])
            rejection.encoding_id = rej.encoding if rej.has_encoding else None
        raise GgufError(code)
    return Document(h.value, keep=buf)


def open(path, limits: dict | None = None, rejection: Rejection | None = None) -> Document:  # noqa: A001
    """weights.Mapped.open (runtime/weights.zig:63-78): maps the file and parses it."""
    h = ctypes.c_void_p()
    rej = _Rejection()
    code = _L().nuq_gguf_open(str(path).encode(), _limits(limits), ctypes.byref(h),
                              ctypes.byref(rej) if rejection is not None else None)
    if code != 0:
        if rejection is not None and rej.len:
            rejection.tensor = bytes(rej.tensor[:rej.len])
            rejection.encoding_id = rej.encoding if rej.has_encoding else None
        raise GgufError(code)
    return Document(h.value)


class ArrayReader:
    """gguf.ArrayReader (gguf.zig:63-104) over a borrowed directory image."""

    def __init__(self, array: Value, directory: bytes, limits: dict | None = None):
        self._dir = bytes(directory)
        self._r = _ArrayReader()
        _check(_L().nuq_gguf_array_reader_init(ctypes.byref(self._r), array.element_type, array.count,
                                               array.file_offset, self._dir, len(self._dir), _limits(limits)))

    def next_string(self) -> bytes | None:
        p, n, has = ctypes.c_void_p(), ctypes.c_uint64(), ctypes.c_int()
        _check(_L().nuq_gguf_array_next_string(ctypes.byref(self._r), ctypes.byref(p), ctypes.byref(n),
                                               ctypes.byref(has)))
        return (ctypes.string_at(p, n.value) if n.value else b"") if has.value else None

    def next_int32(self) -> int | None:
        v, has = ctypes.c_int32(), ctypes.c_int()
        _check(_L().nuq_gguf_array_next_int32(ctypes.byref(self._r), ctypes.byref(v), ctypes.byref(has)))
        return v.value if has.value else None


class DeviceWeights:
    """A GGUF file's tensor-data section on one GPU (torch uint8 buffer).
    matrix(name) views a rank-2 tensor in place: no repacking, no copy."""

    def __init__(self, doc: Document, buffer):
        self.doc, self.buffer = doc, buffer

    def matrix(self, name) -> Matrix:
        m = _Matrix()
        _check(_L().nuq_gguf_matrix(self.doc._h, self.doc.index(name), self.buffer.data_ptr(), ctypes.byref(m)))
        start = m.bytes - self.buffer.data_ptr()
        return Matrix(m.encoding, m.rows, m.columns, self.buffer[start:start + m.byte_len], m.byte_len)


def upload(backend, doc: Document) -> DeviceWeights:
    """Copies doc's tensor data to the backend's GPU (nuq_gguf_upload), on
    torch's current stream; returns when the copy has completed."""
    torch = backend._torch
    n = doc.data_bytes
    buf = torch.empty(max(n, 1), dtype=torch.uint8, device=backend.device)
    lib().nuq_set_stream(backend._h, torch.cuda.current_stream(backend.device).cuda_stream)
    code = _L().nuq_gguf_upload(backend._h, doc._h, buf.data_ptr(), buf.numel())
    if code != 0:
        raise GgufError(code, lib().nuq_last_error(backend._h).decode())
    return DeviceWeights(doc, buf)
