"""ctypes view of the CPU oracle (oracle/oracle.c). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker. The product path (nuclis_amd) never does.
Citations of the nuclis functions each entry restates are in oracle/oracle.h.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

OK, INVALID_SHAPE, UNSUPPORTED_ENCODING, INVALID_ROW_LENGTH, INVALID_BYTE_LENGTH, NON_FINITE = range(6)
ERROR_NAMES = {
    INVALID_SHAPE: "InvalidShape",
    UNSUPPORTED_ENCODING: "UnsupportedTensorEncoding",
    INVALID_ROW_LENGTH: "InvalidRowLength",
    INVALID_BYTE_LENGTH: "InvalidByteLength",
    NON_FINITE: "NonFiniteResult",
}

# inference/src/tensor/encoding.zig:29-41
LAYOUT = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 23: (256, 136)}


class OracleError(Exception):
    def __init__(self, code: int):
        super().__init__(ERROR_NAMES.get(code, f"error {code}"))
        self.code = code
        self.name = ERROR_NAMES.get(code, str(code))


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        c_sz, c_p = ctypes.c_size_t, ctypes.c_void_p
        L.orc_half_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_half_to_f32.restype = ctypes.c_float
        L.orc_f32_to_half.argtypes = [ctypes.c_float]
        L.orc_f32_to_half.restype = ctypes.c_uint16
        L.orc_validate_row.argtypes = [ctypes.c_uint32, c_sz, c_sz]
        L.orc_decode_row.argtypes = [ctypes.c_uint32, c_p, c_sz, c_p, c_sz]
        L.orc_q8_0_row.argtypes = [c_p, c_sz, c_p, c_sz]
        L.orc_matvec.argtypes = [ctypes.c_uint32, c_sz, c_sz, c_p, c_sz, c_p, c_sz, c_p, c_sz, ctypes.c_int]
        L.orc_matmul.argtypes = [ctypes.c_uint32, c_sz, c_sz, c_p, c_sz, c_p, c_sz, c_p, c_sz, c_sz, ctypes.c_int]
        L.orc_argmax.argtypes = [c_p, c_sz, ctypes.POINTER(ctypes.c_size_t)]
        L.orc_penalize.argtypes = [c_p, c_sz, c_p, c_sz, ctypes.c_float, ctypes.c_float, c_p]
        L.orc_topk.argtypes = [c_p, c_sz, c_sz, ctypes.c_float, c_p, c_p, ctypes.POINTER(ctypes.c_double),
                               ctypes.POINTER(ctypes.c_int)]
        _lib = L
    return _lib


def _check(code: int) -> None:
    if code != OK:
        raise OracleError(code)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def half_to_f32(bits: int) -> float:
    return lib().orc_half_to_f32(bits)


def f32_to_half(value: float) -> int:
    return lib().orc_f32_to_half(value)


def validate_row(encoding: int, byte_count: int, element_count: int) -> None:
    _check(lib().orc_validate_row(encoding, byte_count, element_count))


def decode_row(encoding: int, row: bytes | np.ndarray, elements: int) -> np.ndarray:
    buf = np.frombuffer(bytes(row), dtype=np.uint8) if not isinstance(row, np.ndarray) else row
    out = np.empty(elements, dtype=np.float32)
    _check(lib().orc_decode_row(encoding, _ptr(buf) if buf.size else None, buf.size, _ptr(out), elements))
    return out


def decode_matrix(encoding: int, weights: np.ndarray, rows: int, columns: int) -> np.ndarray:
    w = np.ascontiguousarray(weights, dtype=np.uint8).reshape(rows, -1)
    out = np.empty((rows, columns), dtype=np.float32)
    for r in range(rows):
        out[r] = decode_row(encoding, w[r], columns)
    return out


def q8_0_row(values: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    out = np.empty(v.size // 32 * 34 if v.size % 32 == 0 else 0, dtype=np.uint8)
    _check(lib().orc_q8_0_row(_ptr(v), v.size, _ptr(out), out.size))
    return out


def matvec(encoding: int, rows: int, columns: int, weights: np.ndarray, x: np.ndarray, threads: int = 0) -> np.ndarray:
    w = np.ascontiguousarray(weights, dtype=np.uint8).ravel()
    xv = np.ascontiguousarray(x, dtype=np.float32).ravel()
    y = np.empty(rows, dtype=np.float32)
    _check(lib().orc_matvec(encoding, rows, columns, _ptr(w), w.size, _ptr(xv), xv.size, _ptr(y), rows, threads))
    return y


def matmul(encoding: int, rows: int, columns: int, weights: np.ndarray, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """x: [tokens][columns] F32 (F16 inputs are widened exactly first)."""
    w = np.ascontiguousarray(weights, dtype=np.uint8).ravel()
    xm = np.ascontiguousarray(np.asarray(x).astype(np.float32))
    tokens = xm.shape[0]
    y = np.empty((tokens, rows), dtype=np.float32)
    _check(lib().orc_matmul(encoding, rows, columns, _ptr(w), w.size, _ptr(xm), xm.shape[1], _ptr(y), rows, tokens, threads))
    return y


def argmax(logits: np.ndarray) -> int:
    v = np.ascontiguousarray(logits, dtype=np.float32)
    idx = ctypes.c_size_t(0)
    _check(lib().orc_argmax(_ptr(v), v.size, ctypes.byref(idx)))
    return idx.value


def penalize(logits: np.ndarray, history_words: np.ndarray, repetition: float, presence: float) -> np.ndarray:
    v = np.ascontiguousarray(logits, dtype=np.float32)
    h = np.ascontiguousarray(history_words, dtype=np.uint32)
    out = np.empty_like(v)
    _check(lib().orc_penalize(_ptr(v), v.size, _ptr(h), h.size, repetition, presence, _ptr(out)))
    return out


def topk(logits: np.ndarray, k: int, temperature: float):
    """(ids uint32[k], values float32[k], total F64, finite)."""
    v = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.empty(k, dtype=np.uint32)
    vals = np.empty(k, dtype=np.float32)
    total = ctypes.c_double(0)
    finite = ctypes.c_int(0)
    _check(lib().orc_topk(_ptr(v), v.size, k, temperature, _ptr(ids), _ptr(vals), ctypes.byref(total),
                          ctypes.byref(finite)))
    return ids, vals, total.value, bool(finite.value)


def history_words(ids, count: int) -> np.ndarray:
    """History.writeWords layout (sampling/root.zig): bit id of word id / 32."""
    words = np.zeros((count + 31) // 32, dtype=np.uint32)
    for i in ids:
        words[i // 32] |= np.uint32(1 << (i % 32))
    return words


def default_threads() -> int:
    return lib().orc_default_threads()
