"""Host-side mirror of nuclis's matmul backend over libnuq.so.

`Backend` keeps the method names, argument meaning and error behaviour of the
reference's Zig `Backend` for this path (inference/src/backends/metal/):
  matvec        ops/matvec.zig:32
  matvec_rows   ops/matvec.zig:149   (matvecRows)
  matvec_segments ops/matvec.zig:245 (matvecSegments)
  matmul        ops/matmul.zig:62
  matmul_kernel ops/matmul.zig:73    (matmulKernel)
  embed         ops/rowwise.zig:17
Errors are raised as the reference's typed errors (InvalidShape,
UnsupportedTensorEncoding, InvalidRowLength, InvalidByteLength,
NonFiniteResult). Every product runs in libnuq.so's HIP kernels; nothing here
computes. Device memory and streams come from PyTorch (plumbing only).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libnuq.so"

Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS = 8, 12, 13, 14, 23
F32, F16 = 0, 1
KERNEL_AUTO, KERNEL_ROWS, KERNEL_TILE, KERNEL_GENERIC = 0, 1, 2, 3
SEGMENT_PLAIN, SEGMENT_SILU_MUL_PAIR = 0, 1
NOALLOC_MAX_PAIR_ROWS = 1 << 20  # NUQ_NOALLOC_MAX_PAIR_ROWS (include/nuq.h)

# inference/src/tensor/encoding.zig:29-41: id -> (values per block, bytes per block)
LAYOUT = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), IQ4_XS: (256, 136)}


class NuqError(Exception):
    """Base of the typed errors; `.code` is the C status."""

    code = -1


class InvalidShape(NuqError):
    code = 1


class UnsupportedTensorEncoding(NuqError):
    code = 2


class InvalidRowLength(NuqError):
    code = 3


class InvalidByteLength(NuqError):
    code = 4


class NonFiniteResult(NuqError):
    code = 5


class DeviceError(NuqError):
    code = 6


class InvalidArgument(NuqError):
    code = 7


_ERRORS = {c.code: c for c in (InvalidShape, UnsupportedTensorEncoding, InvalidRowLength, InvalidByteLength,
                               NonFiniteResult, DeviceError, InvalidArgument)}


class _Matrix(ctypes.Structure):
    _fields_ = [("encoding", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("rows", ctypes.c_uint64),
                ("columns", ctypes.c_uint64), ("bytes", ctypes.c_void_p), ("byte_len", ctypes.c_uint64)]


class _TopKBuffers(ctypes.Structure):
    _fields_ = [("values", ctypes.c_void_p), ("indices", ctypes.c_void_p), ("sums", ctypes.c_void_p),
                ("flags", ctypes.c_void_p)]


# Backend.topk limits (backends/metal/ops/sampling.zig:15-22)
TOPK_CAPACITY, TOPK_PARTIALS, TOPK_MAX_COUNT = 256, 64, 262144


@dataclass
class TopK:
    """sampling.TopK (sampling/root.zig:154-173): the `count` best logits by
    (value descending, id ascending), Σ exp((l − max) / temperature) over every
    logit as the F64 sum of the device's F32 partial sums, and whether every
    logit was finite."""

    temperature: float
    ids: list
    values: list
    total: float
    finite: bool


class _Segment(ctypes.Structure):
    _fields_ = [("matrix", _Matrix), ("output", ctypes.c_void_p)]


_lib = None

EXPORTS = [
    "nuq_create", "nuq_destroy", "nuq_set_stream", "nuq_sync", "nuq_last_error", "nuq_set_generic_only",
    "nuq_validate_row", "nuq_embed", "nuq_dequant_range", "nuq_matvec", "nuq_matvec_rows", "nuq_matmul",
    "nuq_matmul_kernel", "nuq_matvec_segments", "nuq_argmax", "nuq_quantize_rows", "nuq_dequant_rows", "nuq_gemv",
    "nuq_gemm", "nuq_topk", "nuq_penalize", "nuq_reserve_workspace", "nuq_workspace_bytes",
    "nuq_matvec_segments_noalloc",
]


def lib() -> ctypes.CDLL:
    """Loads libnuq.so; raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, u32, u64 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64
        mp = ctypes.POINTER(_Matrix)
        L.nuq_create.argtypes = [ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]
        L.nuq_create.restype = vp
        L.nuq_destroy.argtypes = [vp]
        L.nuq_destroy.restype = None
        L.nuq_set_stream.argtypes = [vp, vp]
        L.nuq_reserve_workspace.argtypes = [vp, u64]
        L.nuq_workspace_bytes.argtypes = [vp]
        L.nuq_workspace_bytes.restype = u64
        L.nuq_sync.argtypes = [vp]
        L.nuq_last_error.argtypes = [vp]
        L.nuq_last_error.restype = ctypes.c_char_p
        L.nuq_set_generic_only.argtypes = [vp, ctypes.c_int]
        L.nuq_validate_row.argtypes = [u32, u64, u64]
        L.nuq_embed.argtypes = [vp, mp, u32, vp]
        L.nuq_dequant_range.argtypes = [vp, mp, u64, u64, vp]
        L.nuq_dequant_rows.argtypes = [vp, u32, vp, u64, u32, u32, vp]
        L.nuq_gemv.argtypes = [vp, u32, vp, u64, u32, u32, vp, vp]
        L.nuq_gemm.argtypes = [vp, u32, vp, u64, u32, u32, vp, u32, u64, vp, u64, u32]
        L.nuq_topk.argtypes = [vp, vp, u64, u32, ctypes.c_float, ctypes.POINTER(_TopKBuffers)]
        L.nuq_penalize.argtypes = [vp, vp, u64, vp, u64, ctypes.c_float, ctypes.c_float]
        L.nuq_matvec.argtypes = [vp, mp, vp, vp]
        L.nuq_matvec_rows.argtypes = [vp, mp, vp, u64, vp, u64, u32]
        L.nuq_matmul.argtypes = [vp, mp, vp, u32, u64, vp, u64, u32]
        L.nuq_matmul_kernel.argtypes = [vp, u32, mp, vp, u32, u64, vp, u64, u32]
        L.nuq_matvec_segments.argtypes = [vp, ctypes.POINTER(_Segment), u32, vp, u32]
        L.nuq_matvec_segments_noalloc.argtypes = [vp, ctypes.POINTER(_Segment), u32, vp, u32]
        L.nuq_argmax.argtypes = [vp, vp, u64, ctypes.POINTER(u32)]
        L.nuq_quantize_rows.argtypes = [u32, vp, u64, u64, vp, u64]
        _lib = L
    return _lib


def _raise(code: int, message: str = "") -> None:
    if code != 0:
        cls = _ERRORS.get(code, NuqError)
        raise cls(message or cls.__name__)


def validate_row(encoding: int, byte_count: int, element_count: int) -> None:
    """decode.validateRow (quant/decode.zig:108-120)."""
    _raise(lib().nuq_validate_row(encoding, byte_count, element_count))


def row_bytes(encoding: int, columns: int) -> int:
    values, size = LAYOUT[encoding]
    return columns // values * size


def quantize(encoding: int, weights: np.ndarray) -> np.ndarray:
    """F32 [rows][columns] -> GGUF rows (uint8 [rows][row_bytes]) on the host.

    Q8_0 is the reference's q8_0Row (quant/encode.zig:17-36); Q4_K, Q5_K, Q6_K
    and IQ4_XS use this library's own quantizers (the reference has none)."""
    w = np.ascontiguousarray(weights, dtype=np.float32)
    if w.ndim == 1:
        w = w[None, :]
    rows, columns = w.shape
    if encoding not in LAYOUT:
        raise UnsupportedTensorEncoding("UnsupportedTensorEncoding")
    if columns % LAYOUT[encoding][0]:
        raise InvalidRowLength("InvalidRowLength")
    out = np.empty((rows, row_bytes(encoding, columns)), dtype=np.uint8)
    _raise(lib().nuq_quantize_rows(encoding, w.ctypes.data, rows, columns, out.ctypes.data, out.size))
    return out


@dataclass
class Matrix:
    """cpu.Matrix (backends/cpu/root.zig:31-36) whose bytes live on the GPU.

    `bytes` is a torch uint8 CUDA tensor (or anything with data_ptr/numel);
    `byte_len` defaults to its size."""

    encoding: int
    rows: int
    columns: int
    bytes: object
    byte_len: int | None = None

    def c(self) -> _Matrix:
        n = self.byte_len if self.byte_len is not None else self.bytes.numel() * self.bytes.element_size()
        return _Matrix(self.encoding, 0, self.rows, self.columns, self.bytes.data_ptr(), n)


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


class Backend:
    """One libnuq context on one GPU, launching on torch's current stream."""

    def __init__(self, device: int = 0):
        import torch

        self._torch = torch
        self.device = device
        err = ctypes.create_string_buffer(512)
        with torch.cuda.device(device):
            self._h = lib().nuq_create(device, err, len(err))
        if not self._h:
            raise DeviceError(err.value.decode())

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().nuq_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- plumbing -----------------------------------------------------------
    def _call(self, fn, *args) -> None:
        stream = self._torch.cuda.current_stream(self.device).cuda_stream
        # a change of stream makes the new one wait for the old one's work
        # (the context's workspace is shared by its calls)
        code = lib().nuq_set_stream(self._h, stream)
        if code == 0:
            code = fn(self._h, *args)
        if code != 0:
            _raise(code, lib().nuq_last_error(self._h).decode())

    def sync(self) -> None:
        """nu_metal_commit's wait (bridge.m:279-310)."""
        self._call(lib().nuq_sync)

    def reserve_workspace(self, nbytes: int) -> None:
        """Allocates the device workspace up front (for graph capture)."""
        self._call(lib().nuq_reserve_workspace, nbytes)

    def workspace_bytes(self) -> int:
        return int(lib().nuq_workspace_bytes(self._h))

    def set_generic_only(self, enabled: bool) -> None:
        """Backend.generic_only (backends/metal/root.zig:99-102)."""
        lib().nuq_set_generic_only(self._h, int(enabled))

    # -- the reference's entry points ----------------------------------------
    def embed(self, matrix: Matrix, token: int, output) -> None:
        m = matrix.c()
        self._call(lib().nuq_embed, ctypes.byref(m), token, _ptr(output))

    def dequant_rows(self, matrix: Matrix, first: int, count: int, output) -> None:
        m = matrix.c()
        self._call(lib().nuq_dequant_range, ctypes.byref(m), first, count, _ptr(output))

    def matvec(self, matrix: Matrix, input, output) -> None:
        m = matrix.c()
        self._call(lib().nuq_matvec, ctypes.byref(m), _ptr(input), _ptr(output))

    def matvec_rows(self, matrix: Matrix, input, in_stride: int, output, out_stride: int, tokens: int) -> None:
        m = matrix.c()
        self._call(lib().nuq_matvec_rows, ctypes.byref(m), _ptr(input), in_stride, _ptr(output), out_stride, tokens)

    def matmul(self, matrix: Matrix, input, in_stride: int, output, out_stride: int, tokens: int) -> None:
        m = matrix.c()
        dtype = F16 if input.dtype == self._torch.float16 else F32
        self._call(lib().nuq_matmul, ctypes.byref(m), _ptr(input), dtype, in_stride, _ptr(output), out_stride, tokens)

    def matmul_kernel(self, kernel: int, matrix: Matrix, input, in_stride: int, output, out_stride: int,
                      tokens: int) -> None:
        m = matrix.c()
        dtype = F16 if input.dtype == self._torch.float16 else F32
        self._call(lib().nuq_matmul_kernel, kernel, ctypes.byref(m), _ptr(input), dtype, in_stride, _ptr(output),
                   out_stride, tokens)

    def matvec_segments(self, segments: list[tuple[Matrix, object]], input, mode: int = SEGMENT_PLAIN) -> None:
        arr = (_Segment * max(1, len(segments)))()
        for i, (mat, out) in enumerate(segments):
            arr[i].matrix = mat.c()
            arr[i].output = _ptr(out)
        self._call(lib().nuq_matvec_segments, arr, len(segments), _ptr(input), mode)

    def matvec_segments_noalloc(self, segments: list[tuple[Matrix, object]], input, mode: int = SEGMENT_PLAIN) -> None:
        """matvec_segments without any device allocation (no counterpart in
        the reference): the SiLU pair's second GEMV uses a fixed per-GPU
        scratch of NUQ_NOALLOC_MAX_PAIR_ROWS floats; calls that overlap on
        one GPU race on it."""
        arr = (_Segment * max(1, len(segments)))()
        for i, (mat, out) in enumerate(segments):
            arr[i].matrix = mat.c()
            arr[i].output = _ptr(out)
        self._call(lib().nuq_matvec_segments_noalloc, arr, len(segments), _ptr(input), mode)

    def penalize(self, logits, history_words, repetition: float, presence: float, count: int | None = None) -> None:
        """Backend.penalize (backends/metal/ops/sampling.zig:58-71), in place.
        `history_words` is a device uint32/int32 tensor: bit id of word id / 32."""
        n = logits.numel() if count is None else count
        self._call(lib().nuq_penalize, _ptr(logits), n, _ptr(history_words), history_words.numel(), repetition,
                   presence)

    def topk(self, logits, k: int, temperature: float, count: int | None = None) -> TopK:
        """Backend.topk (backends/metal/ops/sampling.zig:44-57) and the host's
        readback into sampling.TopK; synchronizes the stream."""
        torch = self._torch
        dev = logits.device
        values = torch.empty(max(k, 1), dtype=torch.float32, device=dev)
        indices = torch.empty(max(k, 1), dtype=torch.int32, device=dev)
        sums = torch.empty(TOPK_PARTIALS, dtype=torch.float32, device=dev)
        flags = torch.empty(TOPK_PARTIALS, dtype=torch.int32, device=dev)
        bufs = _TopKBuffers(values.data_ptr(), indices.data_ptr(), sums.data_ptr(), flags.data_ptr())
        n = logits.numel() if count is None else count
        self._call(lib().nuq_topk, _ptr(logits), n, k, temperature, ctypes.byref(bufs))
        self.sync()
        total = 0.0
        for partial in sums.cpu().tolist():  # F64, in partition order
            total += partial
        return TopK(temperature, [int(i) & 0xffffffff for i in indices.cpu().tolist()[:k]],
                    values.cpu().tolist()[:k], total, not bool(flags.cpu().any()))

    def argmax(self, logits) -> int:
        idx = ctypes.c_uint32(0)
        self._call(lib().nuq_argmax, _ptr(logits), logits.numel(), ctypes.byref(idx))
        return idx.value
