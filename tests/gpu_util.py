"""Helpers of the GPU parity tests: device upload and the tolerance checks.

Tolerances (stated where they are used):
  * dequantisation: bit-exact against the oracle decoder;
  * F32-arithmetic products (GEMV, multi-token GEMV, generic control):
    |gpu - ref| <= 4e-6 * sum|w*x| + 1e-6 per output, the reference's bound
    for its matvecs (metal-check.zig:3976), and normwise
    max|gpu - ref| / max|ref| <= 2e-3 (the stated max relative error);
  * the integer-dot decode GEMV holds the same F32 bound: it carries x as
    fixed point with 23 significant bits relative to each 32-value slice's
    maximum (power-of-two slice scale) into an exact integer dot, with no
    extra term;
  * f16 MFMA tiles (verify, 128x128 and prefill): weights (and F32
    activations) are rounded to f16, so each term carries at most 2^-11
    relative error per rounded operand; the bound is the reference's own for
    its half tiles, |gpu - ref| <= 2e-4 * sum|w*x| + 1e-6 per output
    (metal-check.zig:3779, 3826, 4424), plus the same 2e-3 normwise bound.

check_close records the worst observed |gpu - ref| / sum|w*x| per label
family and bound, with the full label (encoding, shape, tokens) of the case
that set it; conftest prints the table at the end of the session, so the
margin under each bound, and where it is smallest, is visible in the test
log.
"""
import numpy as np

from oracle import oracle as orc


def to_gpu(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def mass(encoding, w_bytes, rows, columns, x):
    """sum_c |w[r,c] * x[t,c]| for every token t and row r (F64)."""
    dec = orc.decode_matrix(encoding, w_bytes, rows, columns).astype(np.float64)
    return np.abs(np.atleast_2d(x).astype(np.float64)) @ np.abs(dec).T


F32_K = 4e-6   # F32 arithmetic (metal-check.zig:3976)
F16_K = 2e-4   # half tiles (metal-check.zig:4424)

WORST = {}   # (first word of the label, k) -> (worst |d| / mass, k, full label of that case)


def check_close(got, want, mass_, k, label="", extra=0.0):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{label}: non-finite output"
    err = np.abs(got - want)
    bound = k * mass_ + extra + 1e-6
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), (f"{label}: |d|={err[worst]:.3e} > bound {bound[worst]:.3e} at {worst} "
                                  f"(got {got[worst]}, want {want[worst]})")
    m = np.asarray(mass_, np.float64)
    ratio = float(np.max(np.where(m > 0, err / np.where(m > 0, m, 1.0), 0.0))) if err.size else 0.0
    key = (label.split(" ")[0] if label else "unlabelled", k)
    if ratio >= WORST.get(key, (-1.0, k, ""))[0]:
        WORST[key] = (ratio, k, label)
    normwise = err.max() / max(np.abs(want).max(), 1e-30)
    assert normwise <= 2e-3, f"{label}: normwise {normwise:.3e}"
    return normwise
