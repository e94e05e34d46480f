"""nuclis_amd: the MI355X (gfx950) quantized-weight matmul path of nuclis.

The product is libnuq.so (HIP kernels + C ABI, include/nuq.h); `backend`
mirrors the reference's Zig Backend entry points over it; `gguf` reads GGUF
files and uploads their tensor data (include/nuq_gguf.h).
"""
from .backend import (  # noqa: F401
    F16, F32, KERNEL_AUTO, KERNEL_GENERIC, KERNEL_ROWS, KERNEL_TILE, LAYOUT, IQ4_XS, Q4_K, Q5_K, Q6_K, Q8_0, SEGMENT_PLAIN,
    SEGMENT_SILU_MUL_PAIR, Backend, DeviceError, InvalidArgument, InvalidByteLength, InvalidRowLength, InvalidShape,
    Matrix, NonFiniteResult, NuqError, UnsupportedTensorEncoding, lib, quantize, row_bytes, validate_row,
)
from . import gguf  # noqa: F401,E402
