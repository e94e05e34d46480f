"""CPU-side checks of libnuq.so: it loads, exports every symbol include/*.h
declares, validates rows as decode.validateRow does, and its host quantizers
write blocks the oracle decodes (Q8_0 bit-identical to the reference encoder).
No compute is launched: this file runs without a GPU."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import nuclis_amd as nq
from nuclis_amd.synth import gaussian
from oracle import oracle as orc

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = "".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    return sorted(set(re.findall(r"^(?:const\s+)?\w+\s*\*?\s*(nuq_\w+)\(", text, re.M)))


def test_header_and_python_binding_agree():
    assert declared_functions() == sorted(nq.backend.EXPORTS + nq.gguf.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(nq.backend.LIB_PATH))
    for name in declared_functions():
        assert hasattr(lib, name), name


@pytest.mark.parametrize("encoding", [8, 12, 13, 14, 23])
def test_validate_row_matches_oracle(encoding):
    n, size = nq.LAYOUT[encoding]
    cases = [(0, 0), (size, n), (size - 1, n), (size + 1, n), (size, 2 * n), (2 * size, n), (size, n - 1),
             (3 * size, 3 * n), (size, n + 1)]
    for byte_count, elements in cases:
        try:
            orc.validate_row(encoding, byte_count, elements)
            want = None
        except orc.OracleError as e:
            want = e.name
        try:
            nq.validate_row(encoding, byte_count, elements)
            got = None
        except nq.NuqError as e:
            got = type(e).__name__
        assert got == want, (byte_count, elements)
    with pytest.raises(nq.UnsupportedTensorEncoding):
        nq.validate_row(999, 1, 1)


def test_q8_0_quantizer_is_the_reference_encoder():
    w = gaussian(0, (64, 4096), 0.02)
    w[0, :32] = 0
    w[1, :32] *= 1e6
    w[2, 5] = np.nan
    got = nq.quantize(8, w)
    for r in range(w.shape[0]):
        assert np.array_equal(got[r], orc.q8_0_row(w[r])), r


@pytest.mark.parametrize("encoding,tol", [(12, 0.6), (14, 0.55)])
def test_k_quantizers_round_trip(encoding, tol):
    """Own Q4_K/Q6_K quantizers: decode(quantize(w)) is within `tol` of the
    group's quantization step of w (their bytes are unpinned by design; parity
    of whatever bytes they write is checked by decoding them)."""
    w = gaussian(3, (16, 1024), 0.02)
    q = nq.quantize(encoding, w)
    assert q.shape == (16, nq.row_bytes(encoding, 1024))
    back = orc.decode_matrix(encoding, q, 16, 1024)
    err = np.abs(back - w)
    group = 32 if encoding == 12 else 16
    spread = w.reshape(16, -1, group)
    step = (spread.max(-1) - np.minimum(spread.min(-1), 0)) / 15 if encoding == 12 else np.abs(spread).max(-1) / 31
    # scale quantization (6 or 8 bits) widens the step by a few percent
    assert np.all(err.reshape(16, -1, group) <= step[..., None] * tol + 1e-7)
    rel = np.linalg.norm(back - w) / np.linalg.norm(w)
    assert rel < (0.1 if encoding == 12 else 0.03)


def test_q5_k_quantizer_round_trip():
    """Own Q5_K quantizer: within a small fraction of the 31-level group step."""
    w = gaussian(4, (16, 1024), 0.02)
    q = nq.quantize(13, w)
    assert q.shape == (16, nq.row_bytes(13, 1024))
    back = orc.decode_matrix(13, q, 16, 1024)
    spread = w.reshape(16, -1, 32)
    step = (spread.max(-1) - np.minimum(spread.min(-1), 0)) / 31
    assert np.all(np.abs(back - w).reshape(16, -1, 32) <= step[..., None] * 0.6 + 1e-7)
    assert np.linalg.norm(back - w) / np.linalg.norm(w) < 0.05


def test_iq4_xs_quantizer_round_trip():
    """Own IQ4_XS quantizer: every value is the nearest of the 16 code values
    at its group's stored scale, and the row error is that of a 4-bit code."""
    w = gaussian(5, (16, 1024), 0.02)
    q = nq.quantize(23, w)
    assert q.shape == (16, nq.row_bytes(23, 1024))
    back = orc.decode_matrix(23, q, 16, 1024)
    table = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)
    blocks = q.reshape(-1, 136)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    high = blocks[:, 2].astype(np.int32) | (blocks[:, 3].astype(np.int32) << 8)
    for b in range(blocks.shape[0]):
        for g in range(8):
            low = (blocks[b, 4 + g // 2] >> (4 * (g % 2))) & 15
            mul = d[b] * ((low | (((high[b] >> (2 * g)) & 3) << 4)) - 32)
            vals = w.reshape(-1, 256)[b, g * 32:(g + 1) * 32]
            best = np.min(np.abs(vals[:, None] - mul * table[None, :]), axis=1)
            got = np.abs(vals - back.reshape(-1, 256)[b, g * 32:(g + 1) * 32])
            assert np.all(got <= best + 1e-9)
    assert np.linalg.norm(back - w) / np.linalg.norm(w) < 0.12


def test_quantizer_refusals():
    with pytest.raises(nq.InvalidRowLength):
        nq.quantize(12, np.zeros((2, 100), np.float32))
    with pytest.raises(nq.UnsupportedTensorEncoding):
        nq.quantize(3, np.zeros((2, 256), np.float32))


def test_c_abi_host_checks_from_c():
    """tests/c_abi/nuq_check.c's host-only part (GGUF parsing through the C
    header), linked against libnuq.so without touching a GPU."""
    import subprocess
    exe = ROOT / "tests" / "c_abi" / "_build" / "nuq_check"
    assert exe.exists(), "run __graft_entry__.build()"
    r = subprocess.run([str(exe), "--host-only"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "host OK" in r.stdout, r.stdout + r.stderr


def test_gguf_reader_survives_corruption_under_sanitizers():
    """tests/c_abi/gguf_fuzz.c: the GGUF reader (host C++) built on its own
    with AddressSanitizer and UBSan, fed every truncation, every byte/u32/u64
    patch and 200,000 random edits of the reference's wire fixture
    (gguf.zig:617-650). Any overread, leak or undefined behaviour fails."""
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("no host C++ compiler")
    d = ROOT / "tests" / "c_abi"
    subprocess.run(["make", "-s", "-C", str(d), "fuzz"], check=True, capture_output=True, timeout=300)
    r = subprocess.run([str(d / "_build" / "gguf_fuzz")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "gguf_fuzz: OK" in r.stdout, r.stdout + r.stderr


def test_gemv_asm_loads_are_not_read_before_their_waits():
    """The decode GEMV's activation loads are inline asm waited for by a
    later inline-asm s_waitcnt; the compiled gfx950 code must not read (or
    copy) their destination registers in between (tests/isa/asm_hazard.py)."""
    import subprocess
    import tempfile
    from tests.isa.asm_hazard import hazards
    root = Path(__file__).resolve().parents[1]
    with tempfile.TemporaryDirectory() as d:
        out = Path(d) / "gemv_int.s"
        subprocess.run(["/opt/rocm/bin/hipcc", "-x", "hip", "--offload-arch=gfx950", "-O3", "-std=c++17",
                        "-I", str(root / "include"), "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                        "-fno-gpu-flush-denormals-to-zero", "--cuda-device-only", "-S",
                        str(root / "nuclis_amd" / "csrc" / "gemv_int.hip"), "-o", str(out)],
                       check=True, capture_output=True)
        count, found = hazards(out.read_text())
    assert count >= 10, count
    assert not found, found[:5]


def test_asm_hazard_checker_catches_planted_races():
    """The static checker itself: reads and writes of an in-flight load's
    registers before its wait are reported, vmcnt(N) retires only the older
    loads, and a load at the bottom of a loop is checked against the top."""
    from tests.isa.asm_hazard import hazards

    def run(body):
        asm = "_ZN3nuq15gemv_dma_kernelX:  ; @k\n" + "\n".join(body) + "\n.Lfunc_end0:\n"
        return hazards(asm)[1]

    load_a = "global_load_dwordx4 v[0:3], v[20:21], off"
    load_b = "global_load_dwordx4 v[4:7], v[22:23], off"
    assert run([load_a, "s_waitcnt vmcnt(0)", "v_add_u32_e32 v8, v0, v1"]) == []
    assert run([load_a, "v_add_u32_e32 v8, v0, v1", "s_waitcnt vmcnt(0)"])        # read before the wait
    assert run([load_a, "v_mov_b32_e32 v2, 0", "s_waitcnt vmcnt(0)"])             # write before the wait
    assert run([load_a, load_b, "s_waitcnt vmcnt(1)", "v_add_u32_e32 v8, v0, v1"]) == []
    assert run([load_a, load_b, "s_waitcnt vmcnt(1)", "v_add_u32_e32 v8, v4, v1"])  # b still in flight
    assert run([load_a, "global_load_lds_dwordx4 v[20:21], off", "s_waitcnt vmcnt(1)",
                "v_add_u32_e32 v8, v0, v1"]) == []                                  # the copy writes no VGPR
    assert run([".LBB0_1:", "v_add_u32_e32 v8, v0, v1", "s_waitcnt vmcnt(0)", load_a,
                "s_cbranch_scc1 .LBB0_1", "s_waitcnt vmcnt(0)"])                     # loop back edge
