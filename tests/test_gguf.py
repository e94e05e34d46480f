"""GGUF directory reader: libnuq's C++ parser (nuclis_amd.gguf) against the
reference's own tests (inference/src/formats/gguf.zig:424-772,
runtime/weights.zig:87-103) and against the independent Python restatement
in oracle/gguf_oracle.py, case by case and over the reference's corruption
families. Host only: no GPU work."""
import random
import struct

import pytest

import nuclis_amd as nq
from nuclis_amd import gguf
from oracle import gguf_oracle as og
from tests.gguf_fixture import FIRST_TAG, array_i32, array_str, fixture, gstr, header, pad32, write_model

U64_MAX = (1 << 64) - 1


def outcome_product(data, file_bytes=None, limits=None):
    try:
        doc = gguf.parse(data, file_bytes, limits)
    except gguf.GgufError as e:
        return ("error", e.name)
    with doc:
        return ("ok", summary(doc))


def outcome_oracle(data, file_bytes=None, limits=None):
    try:
        doc = og.parse(data, file_bytes, limits)
    except og.GgufError as e:
        return ("error", e.name)
    return ("ok", summary(doc))


def _val(v):
    vals = None if v.values is None else tuple(_val(x) for x in v.values)
    return (v.kind, v.type, v.value, v.element_type, v.count, v.file_offset, vals)


def summary(doc):
    return (doc.version, doc.alignment, doc.directory_bytes, doc.data_offset,
            tuple((k, t, _val(v)) for k, t, v in doc.metadata),
            tuple((t.name, tuple(t.dimensions), t.encoding_id, t.offset, t.bytes, t.elements) for t in doc.tensors))


def both(data, file_bytes=None, limits=None):
    a, b = outcome_product(data, file_bytes, limits), outcome_oracle(data, file_bytes, limits)
    assert a == b, (a, b)
    return a


# -- gguf.zig:512-523 ------------------------------------------------------------
def test_read_metadata_and_tensor_ranges_without_consuming_weights():
    data = fixture()
    kind, s = both(data)
    assert kind == "ok"
    with gguf.parse(data) as doc:
        assert doc.string("general.architecture") == b"fixture"
        assert doc.tensors[0].bytes == 16
        assert doc.get("tokenizer.ggml.tokens").count == 2
        assert doc.directory_bytes < doc.data_offset
        # the directory ends right after the second tensor descriptor
        descriptor = len(gstr("second")) + 4 + 8 + 4 + 8
        assert data.index(b"second") - 8 + descriptor == doc.directory_bytes
        assert doc.data_offset % 32 == 0 and len(data) - doc.data_offset == 64


# -- gguf.zig:473-502 ------------------------------------------------------------
def test_a_rejected_tensor_is_named_for_the_caller_that_asks():
    for opts, err, enc in (({"encoding_id": 999}, "UnsupportedTensorType", 999),
                           ({"encoding_id": 12, "dimension": 100}, "InvalidShape", 12),
                           ({"encoding_id": 0, "dimension": 0}, "InvalidShape", 0)):
        data = fixture(**opts)
        for mod in (gguf, og):
            rej = mod.Rejection()
            with pytest.raises(mod.GgufError) as e:
                mod.parse(data, rejection=rej)
            assert e.value.name == err
            assert rej.tensor == b"first" and rej.encoding_id == enc
    with pytest.raises(gguf.GgufError) as e:
        gguf.parse(fixture(encoding_id=999))
    assert e.value.name == "UnsupportedTensorType"
    assert gguf.Rejection().tensor is None


def test_rank_rejection_names_the_tensor_without_an_encoding():
    data = bytearray(fixture())
    rank_at = data.index(b"first") + len(b"first")
    struct.pack_into("<I", data, rank_at, 5)
    for mod in (gguf, og):
        rej = mod.Rejection()
        with pytest.raises(mod.GgufError) as e:
            mod.parse(bytes(data), rejection=rej)
        assert e.value.name == "InvalidShape" and rej.tensor == b"first" and rej.encoding_id is None


# -- gguf.zig:525-547 ------------------------------------------------------------
def test_lazy_array_access_bounds_offsets_counts_strings_and_element_types():
    b = b"\x01\x00\x00\x00\x00\x00\x00\x00a"
    desc = gguf.Value("array", 9, None, gguf.STRING, 1, 0)
    r = gguf.ArrayReader(desc, b)
    assert r.next_string() == b"a"
    assert r.next_string() is None
    with pytest.raises(gguf.GgufError) as e:
        r.next_int32()
    assert e.value.name == "InvalidMetadataType"
    for n in range(len(b)):
        try:
            t = gguf.ArrayReader(desc, b[:n])
        except gguf.GgufError as err:
            assert err.name == "EndOfStream"
        else:
            with pytest.raises(gguf.GgufError) as e:
                t.next_string()
            assert e.value.name == "EndOfStream"
    limited = gguf.ArrayReader(desc, b, {"string_bytes": 0})
    with pytest.raises(gguf.GgufError) as e:
        limited.next_string()
    assert e.value.name == "LimitExceeded"
    for lim in ({"array_items": 0}, {"directory_bytes": 8}):
        with pytest.raises(gguf.GgufError) as e:
            gguf.ArrayReader(desc, b, lim)
        assert e.value.name == "LimitExceeded"
    with pytest.raises(gguf.GgufError) as e:
        gguf.ArrayReader(gguf.Value("array", 9, None, gguf.STRING, 0, U64_MAX), b)
    assert e.value.name == "EndOfStream"
    signed = gguf.ArrayReader(gguf.Value("array", 9, None, gguf.INT32, 1, 0), b"\xff\xff\xff\xff")
    assert signed.next_int32() == -1
    assert signed.next_int32() is None
    with pytest.raises(gguf.GgufError) as e:
        signed.next_string()
    assert e.value.name == "InvalidMetadataType"
    # the oracle's reader agrees on the same inputs
    assert og.read_array(og.STRING, 1, 0, b) == [b"a"]
    assert og.read_array(og.INT32, 1, 0, b"\xff\xff\xff\xff") == [-1]


def test_lazy_token_array_reads_back_through_the_directory():
    data = fixture()
    with gguf.parse(data) as doc:
        tokens = doc.get("tokenizer.ggml.tokens")
        assert tokens.values is None  # string arrays outside the retained prefixes stay lazy
        r = gguf.ArrayReader(tokens, doc.directory())
        got = []
        while (s := r.next_string()) is not None:
            got.append(s)
    assert got == [b"a", "unicode: λ".encode()]
    assert og.read_array(og.STRING, 2, tokens.file_offset, data) == got


# -- gguf.zig:549-566 ------------------------------------------------------------
def test_truncated_directory_and_tensor_payloads_fail_cleanly():
    data = fixture()
    with gguf.parse(data) as doc:
        required = doc.data_offset + 48
    for n in range(required):
        kind, name = both(data[:n], n)
        assert kind == "error" and name in ("EndOfStream", "TensorOutOfBounds"), (n, name)


# -- gguf.zig:568-590 ------------------------------------------------------------
@pytest.mark.parametrize("opts,expected", [
    ({"version": 2}, "UnsupportedVersion"),
    ({"alignment": 0}, "InvalidAlignment"),
    ({"alignment": 3}, "InvalidAlignment"),
    ({"duplicate_metadata": True}, "DuplicateMetadata"),
    ({"duplicate_tensor": True}, "DuplicateTensor"),
    ({"dimension": 0}, "InvalidShape"),
    ({"dimension": U64_MAX}, "Overflow"),
    ({"encoding_id": 999}, "UnsupportedTensorType"),
    ({"encoding_id": 12}, "InvalidShape"),
    ({"second_offset": 1}, "InvalidAlignment"),
    ({"second_offset": 0}, "OverlappingTensors"),
    ({"second_offset": 1024}, "TensorOutOfBounds"),
])
def test_reject_unsupported_containers_duplicates_invalid_layouts_and_ranges(opts, expected):
    assert both(fixture(**opts)) == ("error", expected)


# -- gguf.zig:592-615 ------------------------------------------------------------
def test_hostile_lengths_and_counts_are_rejected_before_allocating():
    data = fixture()
    for lim in ({"tensor_count": 1}, {"metadata_count": 1}, {"directory_bytes": 24}, {"string_bytes": 4},
                {"array_items": 1}):
        assert both(data, limits=lim) == ("error", "LimitExceeded"), lim
    hostile = bytearray(data)
    struct.pack_into("<Q", hostile, 24, U64_MAX)
    assert both(bytes(hostile)) == ("error", "LimitExceeded")


# -- gguf.zig:658-670, 672-684 -------------------------------------------------------
def test_reject_bad_magic_and_unknown_metadata_tags():
    data = bytearray(fixture())
    data[0] = ord("X")
    assert both(bytes(data)) == ("error", "InvalidMagic")
    data[0] = ord("G")
    struct.pack_into("<I", data, FIRST_TAG, 99)
    assert both(bytes(data)) == ("error", "InvalidMetadataType")


def test_invalid_boolean_values_and_nested_arrays_are_explicit_errors():
    data = bytearray(fixture())
    struct.pack_into("<I", data, FIRST_TAG, 7)
    data[FIRST_TAG + 4] = 2
    assert both(bytes(data)) == ("error", "InvalidBoolean")
    struct.pack_into("<II", data, FIRST_TAG, 9, 9)
    assert both(bytes(data)) == ("error", "UnsupportedNestedArray")


# -- gguf.zig:686-709 ------------------------------------------------------------
def test_retain_small_numeric_arrays_while_leaving_large_arrays_as_descriptors():
    body = header(0, 2) + array_i32("sections", [i - 1 for i in range(4)]) + array_i32("large", [i - 1 for i in range(65)])
    data = pad32(body)
    assert both(data)[0] == "ok"
    with gguf.parse(data) as doc:
        sections = doc.get("sections")
        assert sections.values[0].value == -1 and sections.values[3].value == 2
        assert doc.get("large").values is None
        r = gguf.ArrayReader(doc.get("large"), doc.directory())
        assert [r.next_int32() for _ in range(65)] == [i - 1 for i in range(65)] and r.next_int32() is None


# -- gguf.zig:711-745 ------------------------------------------------------------
def test_arrays_under_a_retained_key_prefix_keep_every_value_strings_included():
    body = header(0, 3) + array_i32("prism.hadamard.sign_values", [1 if i % 2 == 0 else -1 for i in range(65)])
    body += array_str("prism.hadamard.weight_names", ["output.weight", "blk.0.ffn_up.weight"])
    body += array_str("other.names", ["skipped"])
    data = pad32(body)
    assert both(data)[0] == "ok"
    with gguf.parse(data) as doc:
        signs = doc.get("prism.hadamard.sign_values").values
        assert len(signs) == 65 and signs[1].value == -1
        assert doc.get("prism.hadamard.weight_names").values[1].value == b"blk.0.ffn_up.weight"
        assert doc.get("other.names").values is None


def test_retained_prefix_arrays_have_their_own_limit():
    body = header(0, 1) + gstr("prism.hadamard.big") + struct.pack("<IIQ", 9, 5, 65_537)
    body += bytes(4 * 65_537)
    assert both(pad32(body)) == ("error", "LimitExceeded")


# -- gguf.zig:756-772: the fuzz seed ------------------------------------------------
def test_fuzz_seed_parses():
    seed = header(1, 1) + gstr("general.alignment") + struct.pack("<II", 4, 32)
    seed += gstr("w") + struct.pack("<IQIQ", 1, 4, 0, 0) + bytes(6) + bytes([0x3F]) * 16
    kind, s = both(seed)
    assert kind == "ok"
    for short in (header(1, 1), b"GGUF"):
        assert both(short)[0] == "error"


# -- gguf.zig:617-650: corruption families, product vs oracle -------------------------
def test_corrupted_files_agree_with_the_oracle():
    good = fixture()
    n = len(good)
    for k in range(n):
        for claimed in (k, n, U64_MAX):
            both(good[:k], claimed)
    for at in range(n):
        for v in (0, 1, 0x7F, 0x80, 0xFF):
            b = bytearray(good)
            b[at] = v
            both(bytes(b))
        if at + 4 <= n:
            for v in ((1 << 32) - 1, 1 << 31, 13):
                b = bytearray(good)
                struct.pack_into("<I", b, at, v)
                both(bytes(b))
        if at + 8 <= n:
            for v in (U64_MAX, 1 << 63, 1 << 32, 100_000, 100_001):
                b = bytearray(good)
                struct.pack_into("<Q", b, at, v)
                both(bytes(b))
    rng = random.Random(0x6767_7566)
    for _ in range(1000):
        b = bytearray(good)
        for _ in range(rng.randint(1, 4)):
            b[rng.randrange(n)] = rng.randrange(256)
        both(bytes(b))


def test_truncation_and_directory_limit_are_judged_in_the_reference_order():
    # Cursor.advance (gguf.zig:180-188) checks the file's end before the
    # directory limit: a read past both is EndOfStream.
    good = fixture()
    for k in range(0, 120, 3):
        for lim in (8, 24, 30, 40, 64, 100):
            both(good[:k], k, {"directory_bytes": lim})
    assert both(good[:30], 30, {"directory_bytes": 24}) == ("error", "EndOfStream")
    assert both(good, None, {"directory_bytes": 24}) == ("error", "LimitExceeded")


def test_names_must_be_valid_utf8_without_control_bytes():
    for name in (b"ok.name", "λ.weight".encode(), b"bad\x01", b"bad\x7f", b"\xc0\x80", b"\xed\xa0\x80",
                 b"\xf4\x90\x80\x80", b"\xe2\x82", b""):
        body = header(0, 1) + gstr(name) + struct.pack("<IB", 0, 1)
        both(pad32(body))


# -- runtime/weights.zig: Mapped.open, View.bytes / View.matrix -----------------------
def test_mapped_open_views_tensor_bytes_and_matrices(tmp_path):
    rng = random.Random(5)
    q4 = bytes(rng.randrange(256) for _ in range(3 * 144))
    f32 = struct.pack("<4f", 1.0, 2.0, -3.0, 0.5)
    path = tmp_path / "m.gguf"
    write_model(path, [("blk.0.w", (256, 3), 12, list(q4)), ("norm", (4,), 0, list(f32))])
    with gguf.open(path) as doc:
        parsed = gguf.parse(path.read_bytes())
        assert summary(doc) == summary(parsed)
        assert summary(doc) == summary(og.parse(path.read_bytes()))
        assert doc.tensor_bytes("blk.0.w") == q4 and doc.tensor_bytes("norm") == f32
        m = doc.host_matrix("blk.0.w")
        assert (m.encoding, m.rows, m.columns, m.byte_len) == (12, 3, 256, 3 * 144)
        with pytest.raises(gguf.GgufError) as e:
            doc.host_matrix("norm")
        assert e.value.name == "InvalidShape"
        with pytest.raises(gguf.GgufError) as e:
            doc.index("missing")
        assert e.value.name == "NotFound"
        assert doc.data_bytes == path.stat().st_size - doc.data_offset
        parsed.close()
    empty = tmp_path / "empty.gguf"
    empty.write_bytes(b"")
    for p, name in ((empty, "LimitExceeded"), (tmp_path, "NotRegularFile"), (tmp_path / "none", "FileError")):
        with pytest.raises(gguf.GgufError) as e:
            gguf.open(p)
        assert e.value.name == name


def test_default_limits_match_the_reference():
    assert gguf.default_limits() == og.DEFAULT_LIMITS


def test_layouts_agree_with_the_oracle_table():
    # every id 0..255 either sizes like encoding.layout or is refused
    for enc in range(256):
        dims = 256 * 128
        data = pad32(header(1, 0) + gstr("t") + struct.pack("<IQIQ", 1, dims, enc, 0)) + bytes(2 * dims * 4)
        r = both(data)
        if enc in og.LAYOUTS:
            epb, bpb = og.LAYOUTS[enc]
            assert r[0] == "ok" and r[1][5][0][4] == dims // epb * bpb
        else:
            assert r == ("error", "UnsupportedTensorType")
    assert set(og.LAYOUTS) >= set(nq.LAYOUT)
