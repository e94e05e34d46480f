"""Seeded random shapes through the routed matmul entry (every encoding,
token counts across the GEMV, multi-token, verify-tile and prefill routes,
f16 and F32 activations) against the CPU oracle. Each case prints its shape
before it runs."""
import numpy as np
import pytest

import nuclis_amd as nq
from nuclis_amd.synth import gaussian
from oracle import oracle as orc
from tests.gpu_util import F16_K, F32_K, check_close, mass, to_gpu

pytestmark = pytest.mark.gpu

ENCODINGS = [8, 12, 13, 14, 23]
TOKENS = [1, 2, 3, 4, 5, 8, 9, 16, 17, 100, 129, 300]


def cases(n=30, n_prefill=8, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n + n_prefill:
        enc = int(rng.choice(ENCODINGS))
        # the last n_prefill cases take the prefill route (over 128 tokens)
        tokens = int(rng.choice(TOKENS)) if len(out) < n else int(rng.integers(129, 600))
        rows = int(rng.integers(1, 750)) * 8
        columns = int(rng.integers(1, 49)) * 256
        if rows * columns * tokens > 1.5e9:
            continue
        xdtype = "f32" if tokens == 1 else str(rng.choice(["f16", "f32"]))
        out.append((enc, rows, columns, tokens, xdtype, int(rng.integers(1 << 20))))
    return out


@pytest.fixture(scope="module")
def backend():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    b = nq.Backend(0)
    yield b
    b.close()


@pytest.mark.parametrize("encoding,rows,columns,tokens,xdtype,seed", cases())
def test_random_shape_matmul_matches_oracle(backend, encoding, rows, columns, tokens, xdtype, seed):
    import torch
    print(f"[random] enc {encoding} {rows}x{columns} tokens {tokens} {xdtype} seed {seed}", flush=True)
    w = nq.quantize(encoding, gaussian(seed, (rows, columns), 0.02))
    x32 = gaussian(seed + 1, (tokens, columns))
    xref = x32.astype(np.float16).astype(np.float32) if xdtype == "f16" else x32
    xg = to_gpu(x32.astype(np.float16)) if xdtype == "f16" else to_gpu(x32)
    out = torch.full((tokens, rows), np.nan, dtype=torch.float32, device="cuda")
    backend.matmul(nq.Matrix(encoding, rows, columns, to_gpu(w)), xg, columns, out, rows, tokens)
    backend.sync()
    want = orc.matmul(encoding, rows, columns, w, xref)
    # F32 precision: the decode GEMV and the 2-3 token rows; the tiles round
    # activations (and some weights) to f16
    k = F32_K if xdtype == "f32" and tokens <= 3 else F16_K
    check_close(out.cpu().numpy(), want, mass(encoding, w, rows, columns, xref), k, f"random {encoding} {rows}x{columns} M={tokens} {xdtype} seed {seed}")


def gemv_cases(n=24, seed=77):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        enc = int(rng.choice(ENCODINGS))
        block = 32 if enc == 8 else 256
        rows = int(rng.integers(1, 9000))
        columns = int(rng.integers(1, 80)) * block
        out.append((enc, rows, columns, int(rng.integers(1 << 20))))
    return out


@pytest.mark.parametrize("encoding,rows,columns,seed", gemv_cases())
def test_random_shape_matvec_matches_oracle(backend, encoding, rows, columns, seed):
    """The decode GEMV (any row count, any whole-block width) against the
    oracle at the plain F32 bound."""
    import torch
    print(f"[random-gemv] enc {encoding} {rows}x{columns} seed {seed}", flush=True)
    w = nq.quantize(encoding, gaussian(seed, (rows, columns), 0.02))
    x = gaussian(seed + 1, columns)
    out = torch.full((rows,), np.nan, dtype=torch.float32, device="cuda")
    backend.matvec(nq.Matrix(encoding, rows, columns, to_gpu(w)), to_gpu(x), out)
    backend.sync()
    want = orc.matvec(encoding, rows, columns, w, x)
    check_close(out.cpu().numpy()[None, :], want[None, :], mass(encoding, w, rows, columns, x[None, :]), F32_K,
                f"random-gemv {encoding} {rows}x{columns} seed {seed}")


def strided_cases(n=14, seed=4242):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        enc = int(rng.choice(ENCODINGS))
        tokens = int(rng.choice(TOKENS[1:] + [200, 257]))
        rows = int(rng.integers(2, 400)) * 8
        columns = int(rng.integers(1, 33)) * 256
        if rows * columns * tokens > 1.0e9:
            continue
        xdtype = str(rng.choice(["f16", "f32"]))
        pad_in, pad_out = 8 * int(rng.integers(1, 9)), int(rng.integers(1, 40))
        out.append((enc, rows, columns, tokens, xdtype, pad_in, pad_out, int(rng.integers(1 << 20))))
    # the F32 multi-token form (2-3 tokens, one range and K ranges), IQ4_XS,
    # and an F32 prefill
    out += [(12, 1040, 5120, 2, "f32", 8, 5, 11), (13, 528, 17408, 3, "f32", 16, 3, 12),
            (23, 640, 2560, 8, "f16", 8, 7, 13), (23, 512, 4096, 257, "f16", 24, 9, 14),
            (12, 1024, 5120, 300, "f32", 32, 8, 15)]
    return out


@pytest.mark.parametrize("encoding,rows,columns,tokens,xdtype,pad_in,pad_out,seed", strided_cases())
def test_random_strided_matmul_matches_oracle(backend, encoding, rows, columns, tokens, xdtype, pad_in, pad_out,
                                              seed):
    """Activation rows wider than the matrix (in_stride > columns) and output
    rows wider than its row count (out_stride > rows): the products match the
    oracle and the padding of every output row stays untouched."""
    import torch
    in_stride, out_stride = columns + pad_in, rows + pad_out
    print(f"[random-strided] enc {encoding} {rows}x{columns} tokens {tokens} {xdtype} "
          f"in_stride {in_stride} out_stride {out_stride} seed {seed}", flush=True)
    w = nq.quantize(encoding, gaussian(seed, (rows, columns), 0.02))
    x32 = gaussian(seed + 1, (tokens, in_stride))
    xref = x32[:, :columns].astype(np.float16).astype(np.float32) if xdtype == "f16" else x32[:, :columns]
    xg = to_gpu(x32.astype(np.float16)) if xdtype == "f16" else to_gpu(x32)
    out = torch.full((tokens, out_stride), np.nan, dtype=torch.float32, device="cuda")
    backend.matmul(nq.Matrix(encoding, rows, columns, to_gpu(w)), xg, in_stride, out, out_stride, tokens)
    backend.sync()
    got = out.cpu().numpy()
    assert np.isnan(got[:, rows:]).all(), "output padding was written"
    want = orc.matmul(encoding, rows, columns, w, np.ascontiguousarray(xref))
    k = F32_K if xdtype == "f32" and tokens <= 3 else F16_K
    check_close(got[:, :rows], want, mass(encoding, w, rows, columns, xref), k, f"strided {encoding} {rows}x{columns} M={tokens} {xdtype} seed {seed}")
