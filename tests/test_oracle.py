"""Pins the CPU oracle before anything is checked against it.

Sources of truth, none of them a retyping of the oracle's formulas:
  * llama.cpp 7620399f decoder outputs the reference holds
    (inference/src/quant/fixtures/*.json -> tests/golden/decoder_fixtures.json),
    decoded from an unaligned copy as decode.zig:706-724 does;
  * the reference's known-answer tests (decode.zig:455-473, :566-585,
    :692-704, :726-737, :754-779; encode.zig:40-71; cpu/root.zig:171-298);
  * numpy's IEEE float16 for both half conversions, exhaustively/randomly;
  * brute-force F64 sums for matvec.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as orc

GOLDEN = json.loads((Path(__file__).parent / "golden" / "decoder_fixtures.json").read_text())


def fixture(encoding):
    for row in GOLDEN["rows"]:
        if row["encoding"] == encoding:
            return bytes.fromhex(row["bytes_hex"]), np.frombuffer(bytes.fromhex(row["values_f32_hex"]), np.float32)
    raise KeyError(encoding)


def test_fixture_revision():
    assert GOLDEN["revision"] == "7620399f58aebfd2196b74021f9581bcf7218cb9"


ALL = [8, 12, 13, 14, 23]


@pytest.mark.parametrize("encoding", ALL)
def test_decoders_match_llama_cpp_fixtures_from_unaligned_storage(encoding):
    raw, values = fixture(encoding)
    buf = np.zeros(len(raw) + 1, np.uint8)
    buf[1:] = np.frombuffer(raw, np.uint8)
    got = orc.decode_row(encoding, buf[1:], values.size)
    assert got.view(np.uint32).tolist() == values.view(np.uint32).tolist()


def test_half_widening_matches_numpy_for_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.half_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # NaN stays NaN with its sign; whether a signalling payload is quieted
    # depends on the widening instruction, so only the sign is compared
    assert np.array_equal(got[nan].view(np.uint32) >> 31, want[nan].view(np.uint32) >> 31)


def test_half_narrowing_rounds_to_nearest_even_like_numpy():
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 65536, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -26,
                  3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, np.inf, -np.inf], np.float32),
        (np.arange(1, 4096, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -24),  # subnormal ties
    ])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_half(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def test_half_edges_from_reference_test():
    # decode.zig:438-452
    assert orc.half_to_f32(0x8000) == 0.0 and np.signbit(orc.half_to_f32(0x8000))
    assert orc.half_to_f32(0x0001) == 2.0 ** -24
    assert orc.half_to_f32(0x3e00) == 1.5
    assert orc.half_to_f32(0x7bff) == 65504
    assert np.isposinf(orc.half_to_f32(0x7c00))
    assert np.isnan(orc.half_to_f32(0x7e00))


def test_q8_0_signed_extremes_and_independent_scales():
    # decode.zig:455-473
    b = np.zeros(68, np.uint8)
    b[1] = 0x38; b[2] = 0x80; b[3] = 0xFF; b[4] = 0x7F; b[35] = 0xC0; b[36] = 3; b[67] = 0xFE
    want = np.zeros(64, np.float32)
    want[0], want[1], want[2], want[32], want[63] = -64, -0.5, 63.5, -6, 4
    assert np.array_equal(orc.decode_row(8, b, 64), want)


def test_q6_k_signed_scale_extremes_and_quarter_order():
    # decode.zig:692-704
    b = np.full(210, 0xF0, np.uint8)
    b[128:192] = 0xE4
    scales = [-128, 127, -1, 0, 1, 2, -3, 4, 5, -6, 7, -8, 9, -10, 11, -12]
    b[192:208] = np.array(scales, np.int8).view(np.uint8)
    b[208], b[209] = 0, 0x38
    codes = [-32, -16, 15, 31]
    want = np.array([0.5 * scales[i // 16] * codes[(i // 32) % 4] for i in range(256)], np.float32)
    assert np.array_equal(orc.decode_row(14, b, 256), want)


def test_q4_k_six_bit_coefficients_for_every_group():
    # decode.zig:754-764
    b = np.full(144, 0xA3, np.uint8)
    b[0:4] = [0, 0x38, 0, 0x34]
    b[4:16] = [0xC1, 0x82, 0x43, 4, 0x45, 0x86, 0xC7, 8, 0x91, 0xA2, 0xB3, 0xC4]
    expected = [0.25, 8.5, 2.75, 18, 67.25, 159.5, 13.75, 17]
    want = np.array([expected[i // 32] for i in range(256)], np.float32)
    assert np.array_equal(orc.decode_row(12, b, 256), want)


def test_q5_k_high_bit_plane_selects_group_and_column():
    # decode.zig:766-779: d = 1, group scales 1 and minima 0; codes 3 (low
    # nibble) and 10 (high); high-plane byte c has bit c % 8 set, so value i
    # gains 16 exactly when column i % 32 has bit (i / 32) set
    b = np.zeros(176, np.uint8)
    b[1] = 0x3C
    b[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
    b[48:] = 0xA3
    b[16:48] = [1 << (c % 8) for c in range(32)]
    want = np.array([(3 if (i // 32) % 2 == 0 else 10) + (16 if i % 8 == i // 32 else 0) for i in range(256)],
                    np.float32)
    assert np.array_equal(orc.decode_row(13, b, 256), want)


def test_iq4_xs_six_bit_signed_scales_and_half_row_order():
    # decode.zig:726-737: d = 0.5; packed scale bytes give the eight signed
    # group scales below; every code byte 0xF0 puts table entry 0 (-127) in the
    # first 16 values of a group and entry 15 (113) in the last 16
    b = np.full(136, 0xF0, np.uint8)
    b[0:8] = [0, 0x38, 0xE4, 0xE4, 0x10, 0x32, 0x54, 0xFE]
    scales = [-32, -15, 2, 19, -28, -11, 14, 31]
    want = np.array([0.5 * scales[i // 32] * (-127 if i % 32 < 16 else 113) for i in range(256)], np.float32)
    assert np.array_equal(orc.decode_row(23, b, 256), want)


def test_q4_k_subnormal_scales_stay_exact():
    # metal-check.zig:4632: subnormal F16 scales must not flush to zero
    b = np.zeros(144, np.uint8)
    b[0:4] = [1, 0, 3, 0]        # d = 2^-24, dmin = 3 * 2^-24
    b[4:16] = 0x3F                # every scale / minimum 63 (groups 4..7 too)
    b[16:144] = 0xF5              # codes 5 (low) and 15 (high)
    got = orc.decode_row(12, b, 256)
    d, dmin = np.float32(2.0 ** -24), np.float32(3 * 2.0 ** -24)
    lo = np.float32(d * np.float32(63)) * np.float32(5) - np.float32(dmin * np.float32(63))
    assert got[0] == lo and got[0] != 0


@pytest.mark.parametrize("encoding", [0, 1] + ALL)
def test_invalid_rows_are_refused(encoding):
    # decode.zig:566-585
    n, size = orc.LAYOUT[encoding]
    with pytest.raises(orc.OracleError, match="InvalidRowLength"):
        orc.validate_row(encoding, 0, 0)
    for bad_bytes, elements in [(size - 1, n), (size + 1, n), (size, 2 * n), (2 * size, n)]:
        with pytest.raises(orc.OracleError, match="InvalidByteLength"):
            orc.validate_row(encoding, bad_bytes, elements)
    if n > 1:
        with pytest.raises(orc.OracleError, match="InvalidRowLength"):
            orc.validate_row(encoding, size, n - 1)
    with pytest.raises(orc.OracleError, match="UnsupportedTensorEncoding"):
        orc.validate_row(999, 0, 1)


def reference_q8_0(values):
    """q8_0Row written independently in numpy: round half away from zero in
    F64 after the F32 division."""
    v = np.asarray(values, np.float32).reshape(-1, 32)
    out = np.zeros((v.shape[0], 34), np.uint8)
    amax = np.max(np.where(np.isnan(v), 0, np.abs(v)), axis=1)
    d = (amax / np.float32(127)).astype(np.float32).astype(np.float16)
    out[:, 0:2] = d.reshape(-1, 1).view(np.uint8).reshape(-1, 2)
    scale = d.astype(np.float32)[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        r = (v / scale).astype(np.float64)
    q = np.sign(r) * np.floor(np.abs(r) + 0.5)
    q = np.clip(q, -127, 127)
    ok = (scale != 0) & np.isfinite(scale) & ~np.isnan(v)
    q = np.where(ok, q, 0).astype(np.int8)
    out[:, 2:] = q.view(np.uint8)
    return out.ravel()


def test_q8_0_encoder_matches_independent_numpy_restatement():
    rng = np.random.default_rng(11)
    vals = rng.standard_normal(32 * 2000).astype(np.float32) * np.float32(0.02)
    vals[:32] *= 1e6  # large scales
    vals[64:96] = 0
    vals[96:128] = np.float32(70000)  # d overflows F16 -> infinite -> zero codes
    assert np.array_equal(orc.q8_0_row(vals), reference_q8_0(vals))


def test_q8_0_encoder_known_answers():
    # encode.zig:56-71
    x = np.zeros(64, np.float32)
    x[0], x[1], x[2], x[40] = -2.54, 2.54, 0.01, np.nan
    b = orc.q8_0_row(x)
    assert b[2].view(np.int8) == -127 and b[3].view(np.int8) == 127 and b[4] == 0
    assert b[34] == 0 and b[35] == 0 and not b[36:].any()
    with pytest.raises(orc.OracleError):
        orc.q8_0_row(x[:48])


def test_q8_0_round_trip_within_half_a_step():
    # encode.zig:40-53
    rng = np.random.default_rng(0x38)
    x = (rng.random(96, dtype=np.float32) - 0.5) * np.repeat(np.array([4, 0.002, 300], np.float32), 32)
    b = orc.q8_0_row(x)
    y = orc.decode_row(8, b, 96)
    for k in range(3):
        d = np.frombuffer(b[k * 34:k * 34 + 2].tobytes(), np.float16)[0].astype(np.float32)
        assert np.all(np.abs(x[k * 32:(k + 1) * 32] - y[k * 32:(k + 1) * 32]) <= d / 2 + np.abs(x[k * 32:(k + 1) * 32]) * 1e-6)


def f32_bytes(values):
    return np.asarray(values, np.float32).view(np.uint8)


def test_matvec_rectangular_f32_and_f16():
    # cpu/root.zig:171-182
    y = orc.matvec(0, 2, 3, f32_bytes([1, 2, 3, -4, 5, -6]), np.array([2, -1, 0.5], np.float32))
    assert y.tolist() == [1.5, -16]
    y = orc.matvec(1, 1, 2, np.array([0, 0x38, 0, 0xC0], np.uint8), np.array([-4, 3], np.float32))
    assert y.tolist() == [-8]


def test_matvec_f64_accumulation_keeps_small_terms():
    # cpu/root.zig:184-192
    y = orc.matvec(0, 1, 3, f32_bytes([2.0 ** 24, 1, -2.0 ** 24]), np.ones(3, np.float32))
    assert y[0] == 1.0


def test_matvec_q8_two_blocks():
    # cpu/root.zig:194-204
    b = np.ones(136, np.uint8)
    for i, s in enumerate([0x3800, 0x4000, 0xBC00, 0x3400]):
        b[i * 34] = s & 0xFF
        b[i * 34 + 1] = s >> 8
    x = np.ones(64, np.float32)
    x[32:] = -2
    assert orc.matvec(8, 2, 64, b, x).tolist() == [-112, -48]


def test_matvec_refusals_leave_output_untouched():
    # cpu/root.zig:206-238
    b = np.zeros(68, np.uint8)
    x = np.zeros(32, np.float32)
    with pytest.raises(orc.OracleError, match="InvalidShape"):
        orc.matvec(8, 0, 32, b, x)
    with pytest.raises(orc.OracleError, match="InvalidByteLength"):
        orc.matvec(8, 2, 32, b[:67], x)
    with pytest.raises(orc.OracleError, match="InvalidByteLength"):
        orc.matvec(8, 2, 32, b[:66], x)
    with pytest.raises(orc.OracleError, match="InvalidRowLength"):
        orc.matvec(8, 2, 16, b[:34], x[:16])
    with pytest.raises(orc.OracleError, match="UnsupportedTensorEncoding"):
        orc.matvec(999, 2, 32, b, x)


@pytest.mark.parametrize("encoding", ALL)
def test_basis_vectors_select_fixture_columns(encoding):
    # cpu/root.zig:240-272
    raw, values = fixture(encoding)
    columns = orc.LAYOUT[encoding][0]
    rows = values.size // columns
    w = np.frombuffer(raw, np.uint8)
    for column in [0, columns // 2 + 1, columns - 1]:
        x = np.zeros(columns, np.float32)
        x[column] = 1
        y = orc.matvec(encoding, rows, columns, w, x)
        assert np.array_equal(y, values.reshape(rows, columns)[:, column])


def test_matvec_split_across_tasks_is_bit_identical():
    # cpu/root.zig:274-298
    rng = np.random.default_rng(19)
    rows, columns = 300, 512
    b = rng.integers(0, 256, rows * 16 * 34, dtype=np.uint8)
    sc = (rng.random(rows * 16, dtype=np.float32) - 0.5).astype(np.float16).view(np.uint8).reshape(-1, 2)
    b.reshape(-1, 34)[:, 0:2] = sc
    x = (rng.random(columns, dtype=np.float32) * 2 - 1).astype(np.float32)
    serial = orc.matvec(8, rows, columns, b, x, threads=1)
    for t in (2, 3, 8):
        assert np.array_equal(orc.matvec(8, rows, columns, b, x, threads=t).view(np.uint32), serial.view(np.uint32))


@pytest.mark.parametrize("encoding", ALL)
def test_matvec_equals_f64_sum_of_decoded_rows(encoding):
    """Closed form: y = f32(sum_c f64(w) f64(x)), checked with math.fsum
    (exactly rounded) so only the reference's one final rounding differs."""
    import math
    rng = np.random.default_rng(encoding)
    raw, _ = fixture(encoding)
    columns = orc.LAYOUT[encoding][0] * 2
    blocks = np.frombuffer(raw, np.uint8).reshape(-1, orc.LAYOUT[encoding][1])
    rows = 5
    w = np.concatenate([blocks[(r * 3 + t) % len(blocks)] for r in range(rows) for t in range(2)])
    x = rng.standard_normal(columns).astype(np.float32)
    y = orc.matvec(encoding, rows, columns, w, x)
    dec = orc.decode_matrix(encoding, w, rows, columns).astype(np.float64)
    for r in range(rows):
        exact = math.fsum(dec[r] * x.astype(np.float64))
        assert abs(float(y[r]) - exact) <= 1e-12 * np.sum(np.abs(dec[r] * x)) + abs(exact) * 2 ** -23


def test_argmax_first_maximum_and_non_finite():
    # sampling/root.zig:226-239
    assert orc.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert orc.argmax(np.array([-5], np.float32)) == 0
    with pytest.raises(orc.OracleError, match="NonFinite"):
        orc.argmax(np.array([1, np.inf], np.float32))
    with pytest.raises(orc.OracleError, match="NonFinite"):
        orc.argmax(np.array([np.nan, 1], np.float32))


# -- device sampling oracles (penalize, top-k) ------------------------------------------


def test_penalize_oracle_hand_computed_cases():
    """sampling/root.zig:541-611: history {1, 3} over [1.0, 2.0, 1.5, -1.0]."""
    logits = np.array([1.0, 2.0, 1.5, -1.0], np.float32)
    words = orc.history_words([1, 3], 4)
    assert words[0] == (1 << 1) | (1 << 3)
    assert orc.penalize(logits, words, 1.0, 1.0).tolist() == [1.0, 1.0, 1.5, -2.0]   # presence 1.0
    assert orc.penalize(logits, words, 1.0, 0.5).tolist() == [1.0, 1.5, 1.5, -1.5]   # presence 0.5
    assert orc.penalize(logits, words, 2.0, 0.0).tolist() == [1.0, 1.0, 1.5, -2.0]   # repetition 2.0
    # repetition first, then presence: 2/4 - 1 = -0.5 and -1*4 - 1 = -5
    assert orc.penalize(logits, words, 4.0, 1.0).tolist() == [1.0, -0.5, 1.5, -5.0]
    only3 = orc.history_words([3], 4)
    assert orc.penalize(logits, only3, 1.0, -5.0).tolist() == [1.0, 2.0, 1.5, 4.0]   # rewarding presence
    tiny = orc.history_words([0], 2)
    assert np.isinf(orc.penalize(np.array([1e30, 0], np.float32), tiny, 1e-40, 0.0)[0])
    with pytest.raises(orc.OracleError):
        orc.penalize(logits, np.zeros(0, np.uint32), 1.0, 0.0)


def test_history_words_layout():
    """History.writeWords (sampling/root.zig:133-140, test :530-531)."""
    assert orc.history_words([3, 9], 16)[0] == (1 << 3) | (1 << 9)
    w = orc.history_words([31, 32, 95], 96)
    assert w.tolist() == [1 << 31, 1, 1 << 31]


def _lexsort_topk(v, k):
    """Independent restatement: numpy's lexsort on (id, -value) over the
    non-NaN entries, padded with (-inf, 0xffffffff)."""
    ids = np.arange(v.size)
    keep = ~np.isnan(v)
    order = np.lexsort((ids[keep], -v[keep].astype(np.float64)))
    top = ids[keep][order][:k]
    vals = v[top]
    pad = k - top.size
    return (np.concatenate([top, np.full(pad, 0xffffffff)]).astype(np.uint32),
            np.concatenate([vals, np.full(pad, -np.inf, np.float32)]).astype(np.float32))


@pytest.mark.parametrize("seed", range(6))
def test_topk_oracle_matches_an_independent_sort_and_fsum(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(300, 5000))
    v = (rng.standard_normal(n) * 3).astype(np.float32)
    v[rng.integers(0, n, 40)] = 2.5                          # ties
    v[rng.integers(0, n, 5)] = 0.0
    v[rng.integers(0, n, 5)] = -0.0                          # -0 ties with +0
    v[rng.integers(0, n, 3)] = -np.inf
    if seed % 2:
        v[rng.integers(0, n, 7)] = np.nan
    k = int(rng.integers(1, 257))
    t = float(rng.choice([0.7, 1.0, 1.5]))
    ids, vals, total, finite = orc.topk(v, k, t)
    want_ids, want_vals = _lexsort_topk(v, k)
    assert ids.tolist() == want_ids.tolist()
    assert vals.view(np.uint32).tolist() == want_vals.view(np.uint32).tolist()
    m = float(vals[0])
    exact = math.fsum(math.exp((float(x) - m) / t) for x in v.astype(np.float64))
    if finite:
        assert abs(total - exact) <= 1e-12 * exact
    else:
        assert math.isnan(total) or not np.all(np.isfinite(v))
    assert finite == bool(np.all(np.isfinite(v)))


def test_topk_oracle_pads_when_nan_leaves_fewer_than_k():
    v = np.array([np.nan, 1.0, np.nan, -np.inf], np.float32)
    ids, vals, _, finite = orc.topk(v, 4, 1.0)
    assert ids.tolist() == [1, 3, 0xffffffff, 0xffffffff]
    assert vals[:2].tolist() == [1.0, -np.inf] and np.all(np.isneginf(vals[2:]))
    assert not finite
