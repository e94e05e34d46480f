"""The benchmark configurations (BASELINE.json `configs`) at their full
shapes and stated seeds, through the C-ABI library on cuda:0, against the
CPU oracle.

  configs[0]  Q8_0 4096 x 4096 GEMV, W seed 0, x seed 1
  configs[1]  Q4_K GEMV 17408 x 5120 (gate/up) and 5120 x 17408 (down)
  configs[3]  M=8 verify on both Q4_K matrices: the register GEMV
              (KERNEL_ROWS) and the MFMA tile (KERNEL_TILE)
  configs[4]  prefill at M=512 and M=4096: Q4_K 17408 x 5120 and
              Q6_K 5120 x 17408, f16 activations

configs[2] (the layer stack) is tests/test_gpu_layer.py. For the prefill
cases every output row is checked on a token subsample that holds the first
and the last token of every 256-token tile, so every 256 x 256 output tile
(whole, or split along K and reduced) is compared with the oracle's
per-token matvec (metal-check.zig:4410-4424 checks its tiles the same way).
"""
import numpy as np
import pytest

import nuclis_amd as nq
from nuclis_amd.synth import CONFIGS, X_SEED_GEMV, X_SEED_PREFILL, X_SEED_VERIFY, gaussian
from oracle import oracle as orc
from tests.gpu_util import F16_K, F32_K, check_close, mass, to_gpu

pytestmark = pytest.mark.gpu

_W = {}


def weights(name):
    if name not in _W:
        enc, rows, cols, seed = CONFIGS[name]
        _W[name] = nq.quantize(enc, gaussian(seed, (rows, cols), 0.02))
    return _W[name]


@pytest.fixture(scope="module")
def backend():
    b = nq.Backend(0)
    yield b
    b.close()


@pytest.mark.parametrize("name", ["c1_q8_0", "c2_gate", "c2_down"])
def test_config_gemv(backend, name):
    import torch
    enc, rows, cols, _ = CONFIGS[name]
    w = weights(name)
    x = gaussian(X_SEED_GEMV, cols)
    print(f"[config gemv] {name} enc {enc} {rows}x{cols}", flush=True)
    out = torch.full((rows,), np.nan, device="cuda")
    backend.matvec(nq.Matrix(enc, rows, cols, to_gpu(w)), to_gpu(x), out)
    backend.sync()
    want = orc.matvec(enc, rows, cols, w, x)
    check_close(out.cpu().numpy(), want, mass(enc, w, rows, cols, x)[0], F32_K, f"gemv {name}")


@pytest.mark.parametrize("kernel", ["rows", "tile"])
@pytest.mark.parametrize("name", ["c2_gate", "c2_down"])
def test_config_verify_m8(backend, name, kernel):
    import torch
    enc, rows, cols, _ = CONFIGS[name]
    w = weights(name)
    x16 = gaussian(X_SEED_VERIFY, (8, cols)).astype(np.float16)
    print(f"[config verify] {name} {kernel} {rows}x{cols} M=8", flush=True)
    out = torch.full((8, rows), np.nan, device="cuda")
    kid = nq.KERNEL_ROWS if kernel == "rows" else nq.KERNEL_TILE
    backend.matmul_kernel(kid, nq.Matrix(enc, rows, cols, to_gpu(w)), to_gpu(x16), cols, out, rows, 8)
    backend.sync()
    xref = x16.astype(np.float32)
    want = orc.matmul(enc, rows, cols, w, xref)
    # the register GEMV computes in F32 (the f16 activations widen exactly)
    k = F32_K if kernel == "rows" else F16_K
    check_close(out.cpu().numpy(), want, mass(enc, w, rows, cols, xref), k, f"verify_{kernel} {name}")


def token_sample(tokens):
    """First and last token of every 256-token tile, plus a seeded spread."""
    t = set()
    for start in range(0, tokens, 256):
        t.add(start)
        t.add(min(start + 255, tokens - 1))
    rng = np.random.default_rng(tokens)
    t.update(rng.choice(tokens, size=min(8, tokens), replace=False).tolist())
    return np.array(sorted(t))


@pytest.mark.parametrize("tokens", [512, 4096])
@pytest.mark.parametrize("name", ["c5_gate", "c5_down"])
def test_config_prefill(backend, name, tokens):
    import torch
    enc, rows, cols, _ = CONFIGS[name]
    w = weights(name)
    x16 = gaussian(X_SEED_PREFILL, (tokens, cols)).astype(np.float16)
    print(f"[config prefill] {name} enc {enc} {rows}x{cols} M={tokens}", flush=True)
    out = torch.full((tokens, rows), np.nan, device="cuda")
    backend.matmul(nq.Matrix(enc, rows, cols, to_gpu(w)), to_gpu(x16), cols, out, rows, tokens)
    backend.sync()
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    sel = token_sample(tokens)
    xref = x16[sel].astype(np.float32)
    want = orc.matmul(enc, rows, cols, w, xref)
    check_close(got[sel], want, mass(enc, w, rows, cols, xref), F16_K, f"prefill {name} M={tokens}")
