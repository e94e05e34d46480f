"""Parity of the HIP path (libnuq.so on cuda:0) with the CPU oracle.

Inputs are seeded (nuclis_amd.synth.gaussian: numpy PCG64, N(0,0.02) weights,
N(0,1) activations) and quantized by libnuq's host quantizers; the oracle and
the GPU read the same bytes. Tolerances are documented in tests/gpu_util.py.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import nuclis_amd as nq
from nuclis_amd.synth import gaussian
from oracle import oracle as orc
from tests.gpu_util import F16_K, F32_K, check_close, mass, to_gpu

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "decoder_fixtures.json").read_text())


@pytest.fixture(scope="module")
def backend():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    b = nq.Backend(0)
    yield b
    b.close()


def fixture_blocks(encoding):
    for row in GOLDEN["rows"]:
        if row["encoding"] == encoding:
            return np.frombuffer(bytes.fromhex(row["bytes_hex"]), np.uint8), \
                np.frombuffer(bytes.fromhex(row["values_f32_hex"]), np.float32)


def tiled(encoding, rows, columns):
    """metal-check.zig:284-302 (tiledMatrix): block (r*3+t) % n of the fixture."""
    raw, _ = fixture_blocks(encoding)
    n, size = nq.LAYOUT[encoding]
    blocks = raw.reshape(-1, size)
    per_row = columns // n
    idx = (np.arange(rows)[:, None] * 3 + np.arange(per_row)[None, :]) % len(blocks)
    return np.ascontiguousarray(blocks[idx].reshape(rows, per_row * size))


def tame(w, encoding):
    """metal-check.zig:329-345 (tameScales): F16 scales set to 2^-6."""
    n, size = nq.LAYOUT[encoding]
    b = w.reshape(-1, size).copy()
    positions = {12: (0, 2), 13: (0, 2), 14: (208,), 8: (0,), 23: (0,)}[encoding]
    for p in positions:
        b[:, p] = 0x00
        b[:, p + 1] = 0x24
    return b.reshape(w.shape)


def quantized(encoding, rows, columns, seed):
    return nq.quantize(encoding, gaussian(seed, (rows, columns), 0.02))


# ---------------------------------------------------------------- dequant
ALL = [8, 12, 13, 14, 23]


@pytest.mark.parametrize("encoding", ALL)
def test_embed_fixture_rows_bit_exact(backend, encoding):
    import torch
    raw, values = fixture_blocks(encoding)
    n = nq.LAYOUT[encoding][0]
    rows = values.size // n
    w = to_gpu(raw)
    m = nq.Matrix(encoding, rows, n, w)
    for token in range(rows):
        out = torch.empty(n, dtype=torch.float32, device="cuda")
        backend.embed(m, token, out)
        backend.sync()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), values[token * n:(token + 1) * n].view(np.uint32))


@pytest.mark.parametrize("encoding,rows,columns", [(8, 96, 4096), (12, 64, 5120), (14, 40, 17408), (12, 35, 17408),
                                                   (13, 48, 5120), (23, 40, 5120)])
def test_dequant_rows_bit_exact_tiled_and_random(backend, encoding, rows, columns):
    import torch
    for w in (tiled(encoding, rows, columns), quantized(encoding, rows, columns, 7)):
        out = torch.empty(rows * columns, dtype=torch.float32, device="cuda")
        backend.dequant_rows(nq.Matrix(encoding, rows, columns, to_gpu(w)), 0, rows, out)
        backend.sync()
        want = orc.decode_matrix(encoding, w, rows, columns)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.ravel().view(np.uint32))


def test_dequant_subnormal_q4_k_scales_bit_exact(backend):
    import torch
    b = np.zeros((4, 144), np.uint8)
    b[:, 0:4] = [[1, 0, 3, 0], [0xff, 0x03, 0x01, 0x80], [0, 0x04, 0x10, 0], [0x55, 0x02, 0x00, 0x01]]
    b[:, 4:16] = np.arange(12, dtype=np.uint8) * 21
    b[:, 16:] = np.arange(128, dtype=np.uint8)
    out = torch.empty(4 * 256, dtype=torch.float32, device="cuda")
    backend.dequant_rows(nq.Matrix(12, 4, 256, to_gpu(b)), 0, 4, out)
    backend.sync()
    want = orc.decode_matrix(12, b, 4, 256)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.ravel().view(np.uint32))


# ---------------------------------------------------------------- GEMV M=1
GEMV_SHAPES = [
    (8, 4096, 4096),      # config 1
    (12, 17408, 5120),    # config 2 gate/up
    (12, 5120, 17408),    # config 2 down
    (12, 1024, 5120),     # k/v
    (12, 5120, 6144),     # o
    (14, 4096, 5120),     # lm_head slice
    (14, 5120, 17408),    # prefill down shape
    (12, 35, 1280),       # ragged rows (metal-check randomized rows)
    (14, 35, 1280),
    (8, 35, 1280),
    (12, 1, 256),
    (12, 257, 1024),      # one wave set, ragged last workgroup
    (12, 100, 24576),     # 8-block lane groups on the DMA kernel
    (12, 64, 32768),      # x and the rings exceed LDS: register kernel
    (12, 5120, 17408),    # the down projection (8-block lane groups)
    (12, 37, 16640),      # 65 blocks: a partial last lane group, ragged rows
    (12, 300, 17408),
    (13, 1024, 5120),     # Q5_K and IQ4_XS
    (23, 1024, 5120),
    (13, 35, 1280),
    (23, 35, 1280),       # odd block count: the generic kernel
    (13, 512, 17408),     # 8-block lane groups
    (23, 512, 17408),
    (14, 64, 2048),       # Q6_K rows of whole 16-byte chunks
    (14, 1, 256),         # one row: the row-per-wave kernel
]


@pytest.mark.parametrize("encoding,rows,columns", GEMV_SHAPES)
def test_matvec_matches_oracle(backend, encoding, rows, columns):
    import torch
    w = quantized(encoding, rows, columns, 100 + rows % 97)
    x = gaussian(1, columns)
    out = torch.full((rows,), np.nan, dtype=torch.float32, device="cuda")
    backend.matvec(nq.Matrix(encoding, rows, columns, to_gpu(w)), to_gpu(x), out)
    backend.sync()
    want = orc.matvec(encoding, rows, columns, w, x)
    check_close(out.cpu().numpy(), want, mass(encoding, w, rows, columns, x)[0], F32_K, f"matvec {encoding}")


@pytest.mark.parametrize("encoding", ALL)
def test_matvec_tiled_fixture_blocks_and_basis_columns(backend, encoding):
    """Fixture blocks (extreme real scales) tiled into 35 x 1280; plus one-hot
    inputs that select decoded columns (cpu/root.zig:240-272)."""
    import torch
    rows, columns = 35, 1280
    w = tiled(encoding, rows, columns)
    wg = to_gpu(w)
    m = nq.Matrix(encoding, rows, columns, wg)
    x = gaussian(2, columns)
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    backend.matvec(m, to_gpu(x), out)
    backend.sync()
    check_close(out.cpu().numpy(), orc.matvec(encoding, rows, columns, w, x), mass(encoding, w, rows, columns, x)[0],
                F32_K, "tiled")
    dec = orc.decode_matrix(encoding, w, rows, columns)
    for column in (0, columns // 2 + 1, columns - 1):
        e = np.zeros(columns, np.float32)
        e[column] = 1
        backend.matvec(m, to_gpu(e), out)
        backend.sync()
        got = out.cpu().numpy()
        assert np.all(np.abs(got - dec[:, column]) <= 1e-5 * np.abs(dec[:, column])), column


@pytest.mark.parametrize("encoding", ALL)
def test_generic_control_and_misaligned_weights(backend, encoding):
    import torch
    rows, columns = 48, 1024
    w = quantized(encoding, rows, columns, 3)
    x = gaussian(4, columns)
    want = orc.matvec(encoding, rows, columns, w, x)
    mm = mass(encoding, w, rows, columns, x)[0]
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    backend.set_generic_only(True)
    try:
        backend.matvec(nq.Matrix(encoding, rows, columns, to_gpu(w)), to_gpu(x), out)
        backend.sync()
    finally:
        backend.set_generic_only(False)
    check_close(out.cpu().numpy(), want, mm, F32_K, "generic")
    # weights at an odd byte offset: routed to the generic kernel
    buf = torch.zeros(w.size + 1, dtype=torch.uint8, device="cuda")
    buf[1:] = to_gpu(w.ravel())
    backend.matvec(nq.Matrix(encoding, rows, columns, buf[1:]), to_gpu(x), out)
    backend.sync()
    check_close(out.cpu().numpy(), want, mm, F32_K, "misaligned")


def test_matvec_refusals_leave_output_untouched(backend):
    import torch
    w = to_gpu(np.zeros(68, np.uint8))
    x = to_gpu(np.zeros(32, np.float32))
    out = torch.full((2,), 123.0, device="cuda")
    with pytest.raises(nq.InvalidShape):
        backend.matvec(nq.Matrix(8, 0, 32, w), x, out)
    with pytest.raises(nq.InvalidShape):
        backend.matvec(nq.Matrix(8, 2, 32, w, 67), x, out)
    with pytest.raises(nq.InvalidByteLength):
        backend.matvec(nq.Matrix(8, 2, 32, w, 66), x, out)
    with pytest.raises(nq.InvalidRowLength):
        backend.matvec(nq.Matrix(8, 2, 16, w, 68), x, out)
    with pytest.raises(nq.UnsupportedTensorEncoding):
        backend.matvec(nq.Matrix(999, 2, 32, w), x, out)
    backend.sync()
    assert out.cpu().tolist() == [123.0, 123.0]


# ---------------------------------------------------------------- multi-token
@pytest.mark.parametrize("encoding,rows,columns", [(12, 2048, 5120), (14, 1024, 5120), (8, 512, 4096),
                                                   (12, 512, 17408), (13, 512, 5120), (23, 512, 5120)])
@pytest.mark.parametrize("tokens", [2, 3, 5, 8])
def test_matvec_rows_matches_oracle(backend, encoding, rows, columns, tokens):
    import torch
    w = quantized(encoding, rows, columns, 9)
    in_stride, out_stride = columns + 64, rows + 8
    x = np.zeros((tokens, in_stride), np.float32)
    x[:, :columns] = gaussian(10 + tokens, (tokens, columns))
    out = torch.full((tokens, out_stride), np.nan, dtype=torch.float32, device="cuda")
    backend.matvec_rows(nq.Matrix(encoding, rows, columns, to_gpu(w)), to_gpu(x), in_stride, out, out_stride, tokens)
    backend.sync()
    xs = x[:, :columns]
    want = orc.matmul(encoding, rows, columns, w, xs)
    check_close(out.cpu().numpy()[:, :rows], want, mass(encoding, w, rows, columns, xs), F32_K, "rows")


# ---------------------------------------------------------------- MFMA tile
TILE_CASES = [
    (12, 512, 5120, 8), (14, 512, 5120, 8), (8, 512, 4096, 8),
    (12, 256, 1280, 37), (14, 256, 1280, 20), (8, 256, 1280, 5),
    (12, 1024, 5120, 130), (14, 520, 17408, 64), (12, 136, 17408, 200),
    # prefill tile (tokens > 128): ragged token and row tiles
    (14, 520, 5120, 300), (8, 264, 4096, 257), (12, 512, 1280, 512),
    # 260 prefill tiles: 256 whole tiles, then 4 tiles split along K
    (12, 33064, 1024, 257),
    # Q5_K and IQ4_XS at verify, tile and prefill token counts
    (13, 512, 5120, 8), (23, 512, 5120, 8), (13, 256, 1280, 37), (23, 256, 1280, 37),
    (13, 520, 2048, 300), (23, 520, 2048, 300),
    # Q4_K / Q5_K at 17-48 tokens: verify passes of at most 16 tokens (ragged
    # last pass; K ranges and their workspace per pass), then the prefill tile
    (12, 1040, 5120, 33), (13, 1040, 17408, 48), (12, 1040, 5120, 49),
    # K not a multiple of 256 (Q8_0): the 128 x 128 tile, and the prefill
    # tile without a K split
    (8, 264, 4160, 8), (8, 264, 4160, 40),
]


@pytest.mark.parametrize("xdtype", ["f16", "f32"])
@pytest.mark.parametrize("encoding,rows,columns,tokens", TILE_CASES)
def test_tile_matches_oracle(backend, encoding, rows, columns, tokens, xdtype):
    import torch
    w = quantized(encoding, rows, columns, 20 + tokens)
    x32 = gaussian(30 + tokens, (tokens, columns))
    if xdtype == "f16":
        x16 = x32.astype(np.float16)
        xg = to_gpu(x16)
        xref = x16.astype(np.float32)
        k = F16_K
    else:
        xg = to_gpu(x32)
        xref = x32
        k = F16_K
    out = torch.full((tokens, rows), np.nan, dtype=torch.float32, device="cuda")
    backend.matmul_kernel(nq.KERNEL_TILE, nq.Matrix(encoding, rows, columns, to_gpu(w)), xg, columns, out, rows, tokens)
    backend.sync()
    want = orc.matmul(encoding, rows, columns, w, xref)
    check_close(out.cpu().numpy(), want, mass(encoding, w, rows, columns, xref), k, "tile")


# The streamed verify tile (Q4_K and Q5_K, tokens <= 16, up to 24 blocks per
# row): 2 and 3 blocks per wave, a wave whose last block is past the row
# (odd block counts), 16-row steps that end mid-step, token counts 1..16,
# row ranges shortened so the partial sums fit the LDS (13, 12000, 6144,
# 16), and the three places f16 activations go: each wave's own slot (most
# cases), all the slot-1s behind a barrier ((12, 4096, 3840, 16),
# (12, 8192, 4608, 12), (12, 8192, 6144, 8)), or no staging (16 tokens of
# 24 blocks), and rows longer than 24 blocks in K ranges. The weights enter
# the MFMAs as exact f16 integers q * sc, so only the activations are rounded.
VERIFY_DMA_CASES = [(12, 17408, 5120, 8), (12, 4104, 5120, 8), (13, 1000, 4608, 16), (12, 2000, 6144, 3),
                    (12, 808, 3840, 13), (13, 12000, 6144, 16), (12, 24, 256, 1), (13, 4104, 5120, 8),
                    (12, 4096, 3840, 16), (12, 8192, 4608, 12), (12, 8192, 6144, 8),
                    # rows longer than 24 blocks: K ranges added by a second kernel
                    (12, 5120, 17408, 8), (13, 1040, 17408, 16), (12, 2000, 12544, 5),
                    # K ranges of 17-24 Q4_K blocks: 8 waves of 3- and 2-block runs
                    (12, 1032, 11264, 8), (12, 1032, 14080, 12), (12, 4104, 17408, 3)]


@pytest.mark.parametrize("xdtype", ["f16", "f32"])
@pytest.mark.parametrize("encoding,rows,columns,tokens", VERIFY_DMA_CASES)
def test_streamed_verify_matches_oracle(backend, encoding, rows, columns, tokens, xdtype):
    import torch
    w = quantized(encoding, rows, columns, 40 + tokens)
    x32 = gaussian(50 + tokens, (tokens, columns))
    xref = x32.astype(np.float16).astype(np.float32) if xdtype == "f16" else x32
    xg = to_gpu(x32.astype(np.float16)) if xdtype == "f16" else to_gpu(x32)
    out = torch.full((tokens, rows), np.nan, dtype=torch.float32, device="cuda")
    print(f"[verify] enc {encoding} {rows}x{columns} tokens {tokens} {xdtype}", flush=True)
    backend.matmul_kernel(nq.KERNEL_TILE, nq.Matrix(encoding, rows, columns, to_gpu(w)), xg, columns, out, rows, tokens)
    backend.sync()
    want = orc.matmul(encoding, rows, columns, w, xref)
    k = F16_K
    check_close(out.cpu().numpy(), want, mass(encoding, w, rows, columns, xref), k, "verify")


@pytest.mark.parametrize("pad", [8, 64])
def test_streamed_verify_strided_activations(backend, pad):
    """f16 activation rows `pad` halves longer than K (staged through LDS in
    16-byte pieces) match the oracle; rows that are not 16-byte aligned are
    refused before any launch."""
    import torch
    encoding, rows, columns, tokens = 12, 808, 5120, 8
    w = quantized(encoding, rows, columns, 61)
    m = nq.Matrix(encoding, rows, columns, to_gpu(w))
    x = np.zeros((tokens, columns + pad), np.float16)
    x[:, :columns] = gaussian(62, (tokens, columns)).astype(np.float16)
    out = torch.full((tokens, rows), np.nan, dtype=torch.float32, device="cuda")
    backend.matmul_kernel(nq.KERNEL_TILE, m, to_gpu(x), columns + pad, out, rows, tokens)
    backend.sync()
    xref = x[:, :columns].astype(np.float32)
    want = orc.matmul(encoding, rows, columns, w, xref)
    check_close(out.cpu().numpy(), want, mass(encoding, w, rows, columns, xref), F16_K, f"pad {pad}")
    odd = to_gpu(np.zeros((tokens, columns + 4), np.float16))
    with pytest.raises(nq.InvalidShape):
        backend.matmul_kernel(nq.KERNEL_TILE, m, odd, columns + 4, out, rows, tokens)


@pytest.mark.parametrize("encoding,rows,columns,tokens", [(12, 5120, 17408, 512), (14, 2048, 5120, 1024), (12, 17408, 5120, 8),
                                                       (12, 5120, 17408, 8)])
def test_prefill_split_k_is_deterministic(backend, encoding, rows, columns, tokens):
    """Tiles split along K are summed in split order by whichever split
    finishes last: repeated launches must agree bit for bit."""
    import torch
    w = to_gpu(nq.quantize(encoding, gaussian(3, (rows, columns), 0.02)))
    x = to_gpu(gaussian(4, (tokens, columns)).astype(np.float16))
    m = nq.Matrix(encoding, rows, columns, w)
    outs = []
    for _ in range(3):
        out = torch.full((tokens, rows), np.nan, dtype=torch.float32, device="cuda")
        backend.matmul_kernel(nq.KERNEL_TILE, m, x, columns, out, rows, tokens)
        backend.sync()
        outs.append(out.cpu().numpy())
    assert np.isfinite(outs[0]).all()
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


@pytest.mark.parametrize("encoding", ALL)
def test_tile_tamed_fixture_blocks(backend, encoding):
    """metal-check.zig:4355-4436: fixture blocks with tamed scales, 40 rows,
    token counts 37/20/16/9/8/5/1, against the oracle."""
    import torch
    rows, columns = 40, 256 if encoding != 8 else 64
    w = tame(tiled(encoding, rows, columns), encoding)
    mw = nq.Matrix(encoding, rows, columns, to_gpu(w))
    for tokens in (37, 20, 16, 9, 8, 5, 1):
        x = gaussian(tokens, (tokens, columns))
        out = torch.full((tokens, rows), np.nan, dtype=torch.float32, device="cuda")
        backend.matmul_kernel(nq.KERNEL_TILE, mw, to_gpu(x), columns, out, rows, tokens)
        backend.sync()
        want = orc.matmul(encoding, rows, columns, w, x)
        check_close(out.cpu().numpy(), want, mass(encoding, w, rows, columns, x), F16_K, f"tamed {tokens}")


@pytest.mark.parametrize("tokens", [1, 2, 3, 8, 64])
def test_matmul_routing_matches_oracle(backend, tokens):
    import torch
    rows, columns = 256, 5120
    w = quantized(12, rows, columns, 5)
    x = gaussian(6, (tokens, columns))
    out = torch.empty((tokens, rows), dtype=torch.float32, device="cuda")
    backend.matmul(nq.Matrix(12, rows, columns, to_gpu(w)), to_gpu(x), columns, out, rows, tokens)
    backend.sync()
    want = orc.matmul(12, rows, columns, w, x)
    check_close(out.cpu().numpy(), want, mass(12, w, rows, columns, x), F16_K, "matmul")


def test_matmul_refusals(backend):
    import torch
    w = to_gpu(quantized(12, 16, 256, 1).ravel())
    x = torch.zeros((4, 256), device="cuda")
    out = torch.zeros((4, 16), device="cuda")
    with pytest.raises(nq.InvalidShape):   # rows % 8
        backend.matmul(nq.Matrix(12, 12, 256, w[: 12 * 144]), x, 256, out, 16, 4)
    with pytest.raises(nq.InvalidShape):   # tokens 0
        backend.matmul(nq.Matrix(12, 16, 256, w), x, 256, out, 16, 0)
    with pytest.raises(nq.InvalidShape):   # in_stride < columns
        backend.matmul(nq.Matrix(12, 16, 256, w), x, 128, out, 16, 4)
    with pytest.raises(nq.InvalidShape):   # rows tile kernel limit
        backend.matmul_kernel(nq.KERNEL_ROWS, nq.Matrix(12, 16, 256, w), x, 256, out, 16, 9)


# ---------------------------------------------------------------- segments / argmax
def test_segments_plain_and_silu_pair(backend):
    import torch
    segments_plain(backend, [(12, 1024), (12, 512), (14, 256), (8, 128)])
    segments_plain(backend, [(13, 512), (23, 256), (12, 256)])
    columns = 5120
    x = gaussian(41, columns)
    xg = to_gpu(x)
    # gate/up pair: out = silu(gate x) * (up x)
    gate, up = quantized(12, 1024, columns, 50), quantized(12, 1024, columns, 51)
    pair_out = torch.full((1024,), np.nan, device="cuda")
    backend.matvec_segments([(nq.Matrix(12, 1024, columns, to_gpu(gate)), pair_out),
                             (nq.Matrix(12, 1024, columns, to_gpu(up)), pair_out)], xg, nq.SEGMENT_SILU_MUL_PAIR)
    backend.sync()
    g = orc.matvec(12, 1024, columns, gate, x).astype(np.float64)
    u = orc.matvec(12, 1024, columns, up, x).astype(np.float64)
    want = g / (1 + np.exp(-g)) * u
    got = pair_out.cpu().numpy()
    mg, mu = mass(12, gate, 1024, columns, x)[0], mass(12, up, 1024, columns, x)[0]
    # first-order propagation of the two F32 bounds through silu(g)*u (|silu'| <= 1.1)
    bound = 1.1 * np.abs(u) * (F32_K * mg + 1e-6) + np.abs(g) * (F32_K * mu + 1e-6) + 1e-6
    assert np.all(np.abs(got - want) <= bound)


@pytest.mark.parametrize("rows", [4096, 17408])
def test_silu_pair_large_runs_as_two_gemvs(backend, rows):
    """From 4096 rows the pair runs as two decode GEMVs plus the epilogue:
    the integer-dot bound (F32 plus the x-rounding term) propagated through
    silu(g) * u (|silu'| <= 1.1, |silu(g)| <= |g|), and the result equal to
    the epilogue applied to the two GEMVs alone."""
    import torch
    columns = 5120
    x = gaussian(42, columns)
    xg = to_gpu(x)
    gate, up = quantized(12, rows, columns, 52), quantized(12, rows, columns, 53)
    mg_, mu_ = nq.Matrix(12, rows, columns, to_gpu(gate)), nq.Matrix(12, rows, columns, to_gpu(up))
    pair_out = torch.full((rows,), np.nan, device="cuda")
    backend.matvec_segments([(mg_, pair_out), (mu_, pair_out)], xg, nq.SEGMENT_SILU_MUL_PAIR)
    gd, ud = torch.empty(rows, device="cuda"), torch.empty(rows, device="cuda")
    backend.matvec(mg_, xg, gd)
    backend.matvec(mu_, xg, ud)
    backend.sync()
    got = pair_out.cpu().numpy().astype(np.float64)
    gg, uu = gd.cpu().numpy().astype(np.float64), ud.cpu().numpy().astype(np.float64)
    assert np.allclose(got, gg / (1 + np.exp(-gg)) * uu, rtol=1e-6, atol=1e-12)
    g = orc.matvec(12, rows, columns, gate, x).astype(np.float64)
    u = orc.matvec(12, rows, columns, up, x).astype(np.float64)
    want = g / (1 + np.exp(-g)) * u
    eg = F32_K * mass(12, gate, rows, columns, x)[0] + 1e-6
    eu = F32_K * mass(12, up, rows, columns, x)[0] + 1e-6
    bound = 1.1 * np.abs(u) * eg + (np.abs(g) + eg) * eu + 1e-6 * np.abs(want) + 1e-6
    assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) - bound)


@pytest.mark.parametrize("encoding,columns,rows", [
    (12, 5120, (6144, 1024, 1024)),   # config-3 q/k/v
    (12, 5120, (17408,)),
    (12, 17408, (512, 16, 1040, 2048)),
    (13, 5120, (1024, 48)),
    (14, 8192, (512, 256)),
    (8, 4096, (4096, 1024, 32)),
    (23, 5120, (2048, 1024, 16)),
])
def test_segments_one_encoding_run_as_one_gemv(backend, encoding, columns, rows):
    """Segments of one encoding and row stride run as one launch of the decode
    GEMV: every output equals the matrix's own matvec bit for bit (the same
    per-row arithmetic), and stays within the integer-dot bound of the oracle."""
    import torch
    ws = [quantized(encoding, r, columns, 70 + i) for i, r in enumerate(rows)]
    x = gaussian(71, columns)
    xg = to_gpu(x)
    mats = [nq.Matrix(encoding, r, columns, to_gpu(w)) for r, w in zip(rows, ws)]
    outs = [torch.full((r,), np.nan, device="cuda") for r in rows]
    singles = [torch.full((r,), np.nan, device="cuda") for r in rows]
    backend.matvec_segments(list(zip(mats, outs)), xg, nq.SEGMENT_PLAIN)
    for m, o in zip(mats, singles):
        backend.matvec(m, xg, o)
    backend.sync()
    for r, w, o, one in zip(rows, ws, outs, singles):
        got = o.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), one.cpu().numpy().view(np.uint32))
        want = orc.matvec(encoding, r, columns, w, x).astype(np.float64)
        bound = F32_K * mass(encoding, w, r, columns, x)[0] + 1e-6
        assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) - bound)


def test_segments_fall_back_when_the_gemv_does_not_fit(backend):
    """At K = 32768 the decode GEMV's x slices and rings exceed the LDS, so
    one-encoding segments run on the merged row kernel (F32 bound)."""
    segments_plain(backend, [(12, 64, 32768), (12, 32, 32768)])


def segments_plain(backend, shapes):
    import torch
    columns = shapes[0][2] if len(shapes[0]) > 2 else 5120
    shapes = [s_[:2] for s_ in shapes]
    ws = [quantized(e, r, columns, 40 + i) for i, (e, r) in enumerate(shapes)]
    x = gaussian(41, columns)
    xg = to_gpu(x)
    outs = [torch.full((r,), np.nan, device="cuda") for _, r in shapes]
    segs = [(nq.Matrix(e, r, columns, to_gpu(w)), o) for (e, r), w, o in zip(shapes, ws, outs)]
    backend.matvec_segments(segs, xg, nq.SEGMENT_PLAIN)
    backend.sync()
    for (e, r), w, o in zip(shapes, ws, outs):
        check_close(o.cpu().numpy(), orc.matvec(e, r, columns, w, x), mass(e, w, r, columns, x)[0], F32_K, "segment")


def test_argmax_first_maximum(backend):
    import torch
    v = gaussian(60, 151936)
    v[77777] = 50.0
    v[99999] = 50.0
    assert backend.argmax(to_gpu(v)) == orc.argmax(v) == 77777
    v[5] = np.inf
    with pytest.raises(nq.NonFiniteResult):
        backend.argmax(to_gpu(v))
    assert backend.argmax(torch.tensor([3.0], device="cuda")) == 0


def test_workspace_is_allocated_lazily():
    """nuq_create allocates no workspace; decode GEMVs never take one; the
    first prefill that splits K (or verify tile with K ranges) allocates what
    its plan needs, and results match a context that reserved it up front."""
    import torch
    b = nq.Backend(0)
    try:
        assert b.workspace_bytes() == 0
        rows, columns = 2048, 5120
        w = to_gpu(quantized(12, rows, columns, 11))
        m = nq.Matrix(12, rows, columns, w)
        y = torch.empty(rows, device="cuda")
        b.matvec(m, to_gpu(gaussian(12, columns)), y)
        b.sync()
        assert b.workspace_bytes() == 0
        tokens = 8
        x = to_gpu(gaussian(13, (tokens, 17408)).astype(np.float16))
        wd = to_gpu(quantized(12, 1024, 17408, 14))
        md = nq.Matrix(12, 1024, 17408, wd)
        out = torch.empty((tokens, 1024), device="cuda")
        b.matmul(md, x, 17408, out, 1024, tokens)   # verify tile in K ranges
        b.sync()
        lazy = b.workspace_bytes()
        assert 0 < lazy <= 4 << 20, lazy
        b2 = nq.Backend(0)
        try:
            b2.reserve_workspace(64 << 20)
            assert b2.workspace_bytes() >= 64 << 20
            out2 = torch.empty_like(out)
            b2.matmul(md, x, 17408, out2, 1024, tokens)
            b2.sync()
            assert torch.equal(out, out2)
        finally:
            b2.close()
    finally:
        b.close()


def test_captured_workspace_survives_growth():
    """A graph captured with the context's workspace (the verify tile's K
    ranges) still replays correctly after a later eager call has grown the
    workspace: the captured buffer is kept until the context is destroyed,
    not freed on growth, so its memory cannot be handed to a new allocation
    (filled with garbage here) while the graph still writes to it."""
    import torch
    b = nq.Backend(0)
    try:
        tokens, rows, columns = 8, 1024, 17408
        md = nq.Matrix(12, rows, columns, to_gpu(quantized(12, rows, columns, 140)))
        x = to_gpu(gaussian(141, (tokens, columns)).astype(np.float16))
        eager = torch.empty((tokens, rows), device="cuda")
        b.matmul(md, x, columns, eager, rows, tokens)
        b.sync()
        small = b.workspace_bytes()
        assert 0 < small <= 4 << 20
        out = torch.full((tokens, rows), np.nan, device="cuda")
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                b.matmul(md, x, columns, out, rows, tokens)
        torch.cuda.synchronize()
        # an eager prefill that splits K grows the workspace past the captured one
        pm = nq.Matrix(12, 17408, 5120, to_gpu(quantized(12, 17408, 5120, 142)))
        xp = to_gpu(gaussian(143, (4096, 5120)).astype(np.float16))
        yp = torch.empty((4096, 17408), device="cuda")
        b.matmul(pm, xp, 5120, yp, 17408, 4096)
        b.sync()
        assert b.workspace_bytes() > small
        junk = [torch.full((small // 4,), 7.0, device="cuda") for _ in range(4)]
        for _ in range(3):
            out.fill_(np.nan)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int32), eager.view(torch.int32))
            assert all(bool((j == 7.0).all()) for j in junk)
        del graph
    finally:
        b.close()


def test_stream_change_orders_work():
    """Calls from two torch streams on one context: the second stream waits
    for the first one's work, so the shared workspace is not raced."""
    import torch
    rows, columns, tokens = 4096, 17408, 8
    w = quantized(12, rows, columns, 15)
    m = nq.Matrix(12, rows, columns, to_gpu(w))
    xs = [to_gpu(gaussian(16 + i, (tokens, columns)).astype(np.float16)) for i in range(2)]
    b = nq.Backend(0)
    try:
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        outs = [torch.empty((tokens, rows), device="cuda") for _ in range(2)]
        torch.cuda.synchronize()
        with torch.cuda.stream(s1):
            b.matmul(m, xs[0], columns, outs[0], rows, tokens)
        with torch.cuda.stream(s2):
            b.matmul(m, xs[1], columns, outs[1], rows, tokens)
        torch.cuda.synchronize()
        for i in range(2):
            ref = torch.empty_like(outs[i])
            b.matmul(m, xs[i], columns, ref, rows, tokens)
            b.sync()
            assert torch.equal(outs[i], ref)
    finally:
        b.close()


@pytest.mark.parametrize("encoding", [8, 12, 13, 14, 23])
def test_matvec_wide_range_activations(backend, encoding):
    """Activations spread over twelve binary decades inside every 32-value
    slice (the decode GEMV's fixed-point slices are scaled by the slice
    maximum): the plain F32 bound still holds, as it does for an F32 FMA
    chain, whose accumulator carries the large terms the same way."""
    import torch
    rows, columns = 1024, 5120
    w = quantized(encoding, rows, columns, 90)
    rng = np.random.default_rng(91)
    x = (gaussian(92, columns) * np.exp2(rng.uniform(-6, 6, columns))).astype(np.float32)
    out = torch.full((rows,), np.nan, device="cuda")
    backend.matvec(nq.Matrix(encoding, rows, columns, to_gpu(w)), to_gpu(x), out)
    backend.sync()
    want = orc.matvec(encoding, rows, columns, w, x)
    check_close(out.cpu().numpy(), want, mass(encoding, w, rows, columns, x)[0], F32_K, f"widerange {encoding}")


@pytest.mark.parametrize("encoding", [8, 12, 14])
def test_matvec_nan_activation_poisons_rows(backend, encoding):
    """A NaN activation makes every output NaN, as in the oracle's F64 sum."""
    import torch
    rows, columns = 256, 5120
    w = quantized(encoding, rows, columns, 93)
    x = gaussian(94, columns)
    x[1234] = np.nan
    out = torch.zeros(rows, device="cuda")
    backend.matvec(nq.Matrix(encoding, rows, columns, to_gpu(w)), to_gpu(x), out)
    backend.sync()
    assert np.isnan(orc.matvec(encoding, rows, columns, w, x)).all()
    assert np.isnan(out.cpu().numpy()).all()


# Decode GEMV shapes of every M=1 route the integer-dot kernels take: the
# DMA kernel (K = 5120 and 17408), the Q6_K odd-block tail workgroup (K =
# 1280, 5 blocks per row) and the register kernel past the DMA kernel's LDS
# (Q4_K, K = 24576).
DECODE_ROUTES = [(8, 256, 5120), (12, 256, 5120), (13, 256, 5120), (14, 256, 5120), (23, 256, 5120),
                 (12, 64, 17408), (14, 64, 17408), (14, 257, 1280), (12, 64, 24576)]


@pytest.mark.parametrize("encoding,rows,columns", DECODE_ROUTES)
@pytest.mark.parametrize("exp2", [-120, -100, 100])
def test_matvec_extreme_activation_magnitudes(backend, encoding, rows, columns, exp2):
    """x = N(0,1) * 2^exp2: the fixed-point slices use a power-of-two scale,
    so small and large activations keep their relative precision. Checked
    without the absolute 1e-6 allowance (it would hide any result at 2^-100):
    per output |d| <= 4e-6 * sum|w*x|, and normwise <= 2e-3."""
    import torch
    w = quantized(encoding, rows, columns, 120)
    x = (gaussian(121, columns) * np.float32(2.0 ** exp2)).astype(np.float32)
    assert np.all(np.isfinite(x)) and np.abs(x).max() > 0
    print(f"[extreme] enc {encoding} {rows}x{columns} x*2^{exp2}", flush=True)
    out = torch.full((rows,), np.nan, device="cuda")
    backend.matvec(nq.Matrix(encoding, rows, columns, to_gpu(w)), to_gpu(x), out)
    backend.sync()
    got = out.cpu().numpy().astype(np.float64)
    want = orc.matvec(encoding, rows, columns, w, x).astype(np.float64)
    m = mass(encoding, w, rows, columns, x)[0]
    assert np.all(np.isfinite(got))
    err = np.abs(got - want)
    worst = int(np.argmax(err / m))
    assert np.all(err <= F32_K * m), f"row {worst}: |d|={err[worst]:.3e} mass {m[worst]:.3e}"
    assert err.max() / np.abs(want).max() <= 2e-3


def _class_pattern(v):
    """+1 for +Inf, -1 for -Inf, 2 for NaN, 0 for finite."""
    v = np.asarray(v, np.float64)
    return np.where(np.isnan(v), 2, np.where(np.isposinf(v), 1, np.where(np.isneginf(v), -1, 0)))


INF_CASES = {
    "pos": {1234: np.inf},
    "neg": {77: -np.inf},
    "both": {5: np.inf, 4000: -np.inf},
    "same_slice": {64: np.inf, 65: np.inf, 95: -np.inf},
    "inf_nan": {300: np.inf, 301: np.nan},
}


@pytest.mark.parametrize("encoding,rows,columns", DECODE_ROUTES)
@pytest.mark.parametrize("case", sorted(INF_CASES))
def test_matvec_infinite_activations_match_reference(backend, encoding, rows, columns, case):
    """cpu.matvec multiplies each weight by its activation in F64
    (backends/cpu/root.zig:144-152): an infinite activation makes a row +-Inf
    by the sign of its weight, NaN where that weight is 0 or where products of
    both signs meet; NaN stays NaN. The GPU output has the oracle's class in
    every row (+Inf, -Inf, NaN), and its finite rows stay within the F32
    bound."""
    import torch
    w = quantized(encoding, rows, columns, 130)
    if encoding == 12 and case == "pos":
        # make some weights of column 1234 exactly zero: group 4 of block 4
        # gets scale 0 and minimum 0 in a few rows (bytes 4..15 hold them)
        blk = w.reshape(rows, -1, 144)
        blk[:8, 4, 4:16] = 0
    x = gaussian(131, columns)
    for c, v in INF_CASES[case].items():
        x[c % columns] = v
    print(f"[inf] enc {encoding} {rows}x{columns} {case}", flush=True)
    out = torch.zeros(rows, device="cuda")
    backend.matvec(nq.Matrix(encoding, rows, columns, to_gpu(w)), to_gpu(x), out)
    backend.sync()
    got = out.cpu().numpy()
    want = orc.matvec(encoding, rows, columns, w, x)
    np.testing.assert_array_equal(_class_pattern(got), _class_pattern(want))
    assert not np.all(np.isfinite(want))
    if encoding == 12 and case == "pos":
        assert np.isnan(want[:8]).all() and np.isinf(want[8:]).all()  # the planted zeros reach NaN
    fin = np.isfinite(want)
    if fin.any():
        xf = np.where(np.isfinite(x), x, 0).astype(np.float32)
        check_close(got[fin], want[fin], mass(encoding, w, rows, columns, xf)[0][fin], F32_K, f"inf {encoding}")


# Multi-token GEMV at F32 precision on the matrix cores (Q4_K / Q5_K, 2..3
# F32 token rows): each token's activations enter the MFMAs as three f16
# parts holding every bit of x, so the plain F32 bound applies.
# (From four tokens the f16 tile takes over, as the reference's half tiles
# do from four tokens, ops/matmul.zig:86-108.)
MULTI_TOKEN_CASES = [(e, r, c, t) for (e, r, c) in [(12, 17408, 5120), (12, 5120, 17408), (13, 17408, 5120),
                                                    (13, 1040, 5120), (12, 40, 1280), (12, 1000, 4608),
                                                    (13, 520, 17408)]
                     for t in (2, 3)]


@pytest.mark.parametrize("encoding,rows,columns,tokens", MULTI_TOKEN_CASES)
def test_multi_token_f32_matches_oracle(backend, encoding, rows, columns, tokens):
    import torch
    w = quantized(encoding, rows, columns, 95 + tokens)
    rng = np.random.default_rng(96 + tokens)
    x = gaussian(97 + tokens, (tokens, columns))
    x[-1] *= np.exp2(rng.uniform(-6, 6, columns)).astype(np.float32)  # wide range inside each run
    in_stride, out_stride = columns + 4, rows + 8
    xs = np.zeros((tokens, in_stride), np.float32)
    xs[:, :columns] = x
    print(f"[multi-token] enc {encoding} {rows}x{columns} T={tokens}", flush=True)
    m = nq.Matrix(encoding, rows, columns, to_gpu(w))
    out = torch.full((tokens, out_stride), np.nan, device="cuda")
    backend.matmul(m, to_gpu(xs), in_stride, out, out_stride, tokens)
    out2 = torch.full((tokens, out_stride), np.nan, device="cuda")
    backend.matvec_rows(m, to_gpu(xs), in_stride, out2, out_stride, tokens)
    backend.sync()
    want = orc.matmul(encoding, rows, columns, w, x)
    got = out.cpu().numpy()[:, :rows]
    check_close(got, want, mass(encoding, w, rows, columns, x), F32_K, f"multitoken {encoding}")
    assert np.array_equal(got.view(np.uint32), out2.cpu().numpy()[:, :rows].view(np.uint32))


# Four F32 token rows in one launch of the multi-token MFMA form (matvecRows;
# the parts go through the staging two tokens at a time): the plain F32 bound,
# with one token spread over twelve binary decades inside each run.
@pytest.mark.parametrize("encoding,rows,columns", sorted({(e, r, c) for (e, r, c, _) in MULTI_TOKEN_CASES}))
def test_matvec_rows_four_tokens_f32(backend, encoding, rows, columns):
    import torch
    tokens = 4
    w = quantized(encoding, rows, columns, 99)
    rng = np.random.default_rng(98)
    x = gaussian(100, (tokens, columns))
    x[2] *= np.exp2(rng.uniform(-6, 6, columns)).astype(np.float32)
    in_stride, out_stride = columns + 4, rows + 8
    xs = np.zeros((tokens, in_stride), np.float32)
    xs[:, :columns] = x
    print(f"[rows-4] enc {encoding} {rows}x{columns}", flush=True)
    m = nq.Matrix(encoding, rows, columns, to_gpu(w))
    out = torch.full((tokens, out_stride), np.nan, device="cuda")
    backend.matvec_rows(m, to_gpu(xs), in_stride, out, out_stride, tokens)
    backend.sync()
    want = orc.matmul(encoding, rows, columns, w, x)
    got = out.cpu().numpy()
    check_close(got[:, :rows], want, mass(encoding, w, rows, columns, x), F32_K, f"rows-4 {encoding}")
    assert np.isnan(got[:, rows:]).all()


# A NaN in one token's activations: that token's rows are all NaN, as the
# oracle's F64 sums are, and the other tokens of the same launch are unaffected.
@pytest.mark.parametrize("tokens", [2, 4])
def test_matvec_rows_nan_token_stays_in_its_rows(backend, tokens):
    import torch
    encoding, rows, columns = 12, 1040, 5120
    w = quantized(encoding, rows, columns, 101)
    x = gaussian(102, (tokens, columns))
    x[tokens - 1, 777] = np.nan
    print(f"[rows-nan] T={tokens}", flush=True)
    m = nq.Matrix(encoding, rows, columns, to_gpu(w))
    out = torch.zeros((tokens, rows), device="cuda")
    backend.matvec_rows(m, to_gpu(x), columns, out, rows, tokens)
    backend.sync()
    got = out.cpu().numpy()
    assert np.isnan(got[tokens - 1]).all()
    want = orc.matmul(encoding, rows, columns, w, x[:tokens - 1])
    check_close(got[:tokens - 1], want, mass(encoding, w, rows, columns, x[:tokens - 1]), F32_K, "rows-nan")


# Graph replays of the streamed kernels: the matmul routes (decode GEMV,
# F32 multi-token, verify tile with register-staged or ringed steps, K ranges
# with their reduce, prefill) captured in a HIP graph, replayed with eager
# work between replays, must equal the eager result bit for bit. Copies or
# loads read before they land would show up here as replay differences.
GRAPH_CASES = [(12, 2048, 5120, 1, "f32"), (12, 4104, 5120, 8, "f16"), (12, 4104, 5120, 8, "f32"),
               (12, 17408, 5120, 2, "f32"), (13, 4104, 5120, 3, "f32"), (13, 4104, 5120, 8, "f16"),
               (12, 1040, 17408, 8, "f16"), (12, 1024, 5120, 512, "f16")]


@pytest.mark.parametrize("encoding,rows,columns,tokens,xdtype", GRAPH_CASES)
def test_matmul_graph_replays_match_eager(backend, encoding, rows, columns, tokens, xdtype):
    import torch
    w = quantized(encoding, rows, columns, 110 + tokens)
    x = gaussian(111 + tokens, (tokens, columns))
    xg = to_gpu(x.astype(np.float16)) if xdtype == "f16" else to_gpu(x)
    m = nq.Matrix(encoding, rows, columns, to_gpu(w))
    print(f"[graph] enc {encoding} {rows}x{columns} tokens {tokens} {xdtype}", flush=True)
    eager = torch.full((tokens, rows), np.nan, device="cuda")
    backend.matmul(m, xg, columns, eager, rows, tokens)  # also sizes the lazy workspace
    backend.sync()
    out = torch.full((tokens, rows), np.nan, device="cuda")
    other = torch.empty((tokens, rows), device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            backend.matmul(m, xg, columns, out, rows, tokens)
    torch.cuda.synchronize()
    for _ in range(3):
        out.fill_(np.nan)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32))
        backend.matmul(m, xg, columns, other, rows, tokens)  # eager work between replays
        backend.sync()
        assert torch.equal(other.view(torch.int32), eager.view(torch.int32))


# matvecRows with 4..8 F32 token rows (Q4_K / Q5_K) runs as launches of the
# F32 multi-token MFMA form over at most 4 tokens: within the plain F32 bound,
# and each chunk's tokens bit-identical to the same tokens served alone.
@pytest.mark.parametrize("encoding,rows,columns", [(12, 4104, 5120), (13, 1040, 5120), (12, 1040, 17408)])
@pytest.mark.parametrize("tokens", [4, 5, 8])
def test_matvec_rows_in_chunks_matches_oracle(backend, encoding, rows, columns, tokens):
    import torch
    w = quantized(encoding, rows, columns, 120 + tokens)
    x = gaussian(121 + tokens, (tokens, columns))
    m = nq.Matrix(encoding, rows, columns, to_gpu(w))
    xg = to_gpu(x)
    print(f"[rows-chunks] enc {encoding} {rows}x{columns} T={tokens}", flush=True)
    out = torch.full((tokens, rows), np.nan, device="cuda")
    backend.matvec_rows(m, xg, columns, out, rows, tokens)
    out2 = torch.full((tokens, rows), np.nan, device="cuda")
    backend.matmul_kernel(nq.KERNEL_ROWS, m, xg, columns, out2, rows, tokens)
    first = 3 if tokens == 4 else 4  # (4 tokens: the first three alone)
    alone = torch.full((first, rows), np.nan, device="cuda")
    backend.matvec_rows(m, xg[:first].contiguous(), columns, alone, rows, first)
    backend.sync()
    want = orc.matmul(encoding, rows, columns, w, x)
    got = out.cpu().numpy()
    m_ = mass(encoding, w, rows, columns, x)
    check_close(got, want, m_, F32_K, f"rows-chunks {encoding}")
    # KERNEL_ROWS forces the register-dequant GEMV: the same F32 bound
    check_close(out2.cpu().numpy(), want, m_, F32_K, f"rows-register {encoding}")
    assert np.array_equal(got[:first].view(np.uint32), alone.cpu().numpy().view(np.uint32))


# f16 token rows on the automatic route run on the streamed verify tile for
# Q4_K / Q5_K (exact f16 activations times exact f16 integers q * sc), and
# KERNEL_ROWS forces the register-dequant GEMV: both within the plain F32
# bound.
@pytest.mark.parametrize("encoding,rows,columns", [(12, 2056, 5120), (13, 1040, 5120), (12, 1040, 17408)])
@pytest.mark.parametrize("tokens", [2, 3, 8])
def test_matvec_rows_f16_matches_oracle(backend, encoding, rows, columns, tokens):
    import torch
    w = quantized(encoding, rows, columns, 140 + tokens)
    x16 = gaussian(141 + tokens, (tokens, columns)).astype(np.float16)
    m = nq.Matrix(encoding, rows, columns, to_gpu(w))
    xg = to_gpu(x16)
    print(f"[rows-f16] enc {encoding} {rows}x{columns} T={tokens}", flush=True)
    out = torch.full((tokens, rows), np.nan, device="cuda")
    backend.matmul_kernel(nq.KERNEL_ROWS, m, xg, columns, out, rows, tokens)
    auto = torch.full((tokens, rows), np.nan, device="cuda")
    backend.matmul(m, xg, columns, auto, rows, tokens)
    backend.sync()
    x = x16.astype(np.float32)
    want = orc.matmul(encoding, rows, columns, w, x)
    m_ = mass(encoding, w, rows, columns, x)
    check_close(out.cpu().numpy(), want, m_, F32_K, f"rows-f16 {encoding}")
    check_close(auto.cpu().numpy(), want, m_, F32_K, f"auto-f16 {encoding}")


# The K-split register-dequant kernel behind KERNEL_ROWS for Q4_K with f16
# activations (1..8 tokens): one K range up to 32 blocks, K ranges (and the
# range reduce) beyond; rows that are not whole 4-row steps; rows with fewer
# blocks than a wave's 4; padded activation and output strides. Every product
# is exact (f16 activations times the exact f16 integer q * sc), so the plain
# F32 bound holds.
RD_SHAPES = [(17408, 5120), (5120, 17408), (1000, 256), (40, 1280), (264, 12288), (520, 8448)]


@pytest.mark.parametrize("rows,columns", RD_SHAPES)
@pytest.mark.parametrize("tokens", [1, 2, 3, 5, 8])
def test_register_rows_kernel_f16_matches_oracle(backend, rows, columns, tokens):
    import torch
    w = quantized(12, rows, columns, 150 + tokens)
    in_stride, out_stride = columns + 8, rows + 4
    x16 = np.zeros((tokens, in_stride), np.float16)
    x16[:, :columns] = gaussian(151 + tokens, (tokens, columns)).astype(np.float16)
    m = nq.Matrix(12, rows, columns, to_gpu(w))
    print(f"[rows-dma] {rows}x{columns} T={tokens}", flush=True)
    out = torch.full((tokens, out_stride), np.nan, device="cuda")
    backend.matmul_kernel(nq.KERNEL_ROWS, m, to_gpu(x16), in_stride, out, out_stride, tokens)
    backend.sync()
    got = out.cpu().numpy()
    assert np.isnan(got[:, rows:]).all(), "output padding was written"
    x = x16[:, :columns].astype(np.float32)
    want = orc.matmul(12, rows, columns, w, x)
    check_close(got[:, :rows], want, mass(12, w, rows, columns, x), F32_K,
                f"rows-dma {rows}x{columns} T={tokens}")


@pytest.mark.parametrize("rows,columns,tokens", [(5120, 17408, 8), (17408, 5120, 3)])
def test_register_rows_kernel_graph_replays_match_eager(backend, rows, columns, tokens):
    """The register-dequant kernel captured in a HIP graph (its K ranges and
    range reduce included) replays bit-identically to the eager call, with
    eager work between the replays."""
    import torch
    w = quantized(12, rows, columns, 160)
    xg = to_gpu(gaussian(161, (tokens, columns)).astype(np.float16))
    m = nq.Matrix(12, rows, columns, to_gpu(w))
    print(f"[rows-dma graph] {rows}x{columns} T={tokens}", flush=True)
    eager = torch.full((tokens, rows), np.nan, device="cuda")
    backend.matmul_kernel(nq.KERNEL_ROWS, m, xg, columns, eager, rows, tokens)  # sizes the workspace
    backend.sync()
    out = torch.full((tokens, rows), np.nan, device="cuda")
    other = torch.empty((tokens, rows), device="cuda")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            backend.matmul_kernel(nq.KERNEL_ROWS, m, xg, columns, out, rows, tokens)
    torch.cuda.synchronize()
    for _ in range(3):
        out.fill_(np.nan)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32))
        backend.matmul_kernel(nq.KERNEL_ROWS, m, xg, columns, other, rows, tokens)
        backend.sync()
        assert torch.equal(other.view(torch.int32), eager.view(torch.int32))


@pytest.mark.parametrize("encoding,rows,columns", [(12, 17408, 5120), (12, 4096, 4096), (8, 4096, 4096),
                                                    (13, 17408, 5120), (14, 20000, 5120), (23, 17408, 5120),
                                                    (12, 333, 5120), (12, 1, 5120), (12, 5, 5120), (12, 129, 5120),
                                                    (8, 3, 4096), (14, 17, 5120), (12, 2049, 2560)])
def test_matvec_repeats_bit_identically(backend, encoding, rows, columns):
    """Within a workgroup of the DMA GEMV, the waves of one K range claim row
    steps at run time, so which wave computes a row changes from launch to
    launch; a row's sum must not. Five launches, with another matrix's GEMV
    between them, give the same bits as the first (and match the oracle)."""
    import torch
    w = quantized(encoding, rows, columns, 170)
    xh = gaussian(171, columns)
    m = nq.Matrix(encoding, rows, columns, to_gpu(w))
    other = nq.Matrix(encoding, 2048, columns, to_gpu(quantized(encoding, 2048, columns, 172)))
    x = to_gpu(xh)
    print(f"[repeat] enc {encoding} {rows}x{columns}", flush=True)
    first = torch.empty(rows, device="cuda")
    backend.matvec(m, x, first)
    sink = torch.empty(2048, device="cuda")
    for _ in range(5):
        backend.matvec(other, x, sink)
        again = torch.full((rows,), np.nan, device="cuda")
        backend.matvec(m, x, again)
        backend.sync()
        assert torch.equal(again.view(torch.int32), first.view(torch.int32))
    want = orc.matvec(encoding, rows, columns, w, xh)
    check_close(first.cpu().numpy(), want, mass(encoding, w, rows, columns, xh)[0], F32_K,
                f"repeat {encoding} {rows}x{columns}")
