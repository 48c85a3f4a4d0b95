"""The validating safetensors reader (liblrm_hip.so, lrm_st_*) and the deterministic writer, after the reference's
tests (tests/Lrm.Tensor.Tests/SafetensorsTests.fs:14-420): the writer's known-answer vector S1 (byte count and
SHA-256 pinned there), order independence, Python ensure_ascii escaping, the reader on S1, every committed tiny
golden rewritten byte for byte against its manifest SHA-256, OpenVerified, the malformed-file matrix (each refused by
validate and by open, whose message names the file), escaped names, unaligned headers, the writer's refusals, the
atomic replace and a seeded round trip. CPU only: the reader runs no GPU code.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from conftest import TINY
from rosylnalive_amd import safetensors_io as st
from rosylnalive_amd.safetensors_io import IntegrityError, SafetensorsFormatError

# ---- S1 (SafetensorsTests.fs:14-37)
S1_NAME = "é\U0001F600"
S1_VALUE = '"q"\\\n\x7f\t'
S1_META = [("lrm.test", "saïtensors!"), ("a", S1_VALUE)]
S1_TENSORS = [("x", "F32", np.array([1.0, -2.0], np.float32)), (S1_NAME, "BF16", np.array([[0x3F80]], np.uint16)),
              ("b", "I64", np.array(7, np.int64)), ("e", "U8", np.zeros(0, np.uint8))]
S1_HEADER = ('{"__metadata__":{"a":"\\"q\\"\\\\\\n\\u007f\\t","lrm.test":"sa\\u00eftensors!"},'
             '"b":{"dtype":"I64","shape":[],"data_offsets":[0,8]},'
             '"e":{"dtype":"U8","shape":[0],"data_offsets":[8,8]},'
             '"x":{"dtype":"F32","shape":[2],"data_offsets":[8,16]},'
             '"\\u00e9\\ud83d\\ude00":{"dtype":"BF16","shape":[1,1],"data_offsets":[16,18]}}' + " " * 7)
S1_SHA256 = "49fc00c6aa63a8f23a5488fe2bd49a8768779e8f5b943a166013f4b2140666ce"


def s1_bytes():
    return st.to_bytes(S1_TENSORS, S1_META)


def raw_file(header, data: bytes) -> bytes:
    h = header.encode("utf-8") if isinstance(header, str) else header
    return len(h).to_bytes(8, "little") + h + data


def esc(hex4):
    """The six characters of a JSON \\uXXXX escape."""
    return "\\u" + hex4


def entry(dtype, shape, b, e):
    return f'{{"dtype":"{dtype}","shape":{shape},"data_offsets":[{b},{e}]}}'


def expect_format_error(tmp_path, label, data: bytes):
    with pytest.raises(SafetensorsFormatError):
        st.SafetensorsFile.validate(data)
    p = tmp_path / "t.safetensors"
    p.write_bytes(data)
    with pytest.raises(SafetensorsFormatError) as e:
        st.SafetensorsFile.open(str(p))
    assert os.path.realpath(str(p)) in str(e.value), f"{label}: the message names the file"


def test_writer_known_answer_vector_s1():
    b = s1_bytes()
    assert int.from_bytes(b[:8], "little") == 312, "header length, padded to 8"
    assert b[8:320].decode("ascii") == S1_HEADER
    assert len(b) == 338
    assert hashlib.sha256(b).hexdigest() == S1_SHA256


def test_writer_output_is_independent_of_input_order():
    assert st.to_bytes(list(reversed(S1_TENSORS)), list(reversed(S1_META))) == s1_bytes()


def test_json_strings_escape_like_python_ensure_ascii():
    s = "\x00\x1f\x7f\x80￿" + "\U0010FFFF"
    assert st.json_string(s) == '"\\u0000\\u001f\\u007f\\u0080\\uffff\\udbff\\udfff"'
    assert st.json_string('a"b\\c\n\r\t\b\f~ ') == '"a\\"b\\\\c\\n\\r\\t\\b\\f~ "'


def test_reader_opens_s1(tmp_path):
    p = tmp_path / "s1.safetensors"
    p.write_bytes(s1_bytes())
    with st.SafetensorsFile.open(str(p)) as f:
        assert f.header_length == 312 and f.data_offset == 320 and f.length == 338
        assert f.names == ["b", "e", "x", S1_NAME], "names in code point order"
        assert f.metadata == sorted(S1_META)
        assert f.read("x").tolist() == [1.0, -2.0]
        assert f.read(S1_NAME, "BF16").tolist() == [[0x3F80]]
        assert f.read("b").shape == () and int(f.read("b")) == 7
        assert f.read("e").size == 0
        assert f.is_aligned
        assert f.rebuild_header() == f.header_bytes()
        with pytest.raises(TypeError):
            f.read("x", "F64")


def test_every_tiny_golden_file_is_rebuilt_byte_for_byte():
    manifest = json.load(open(os.path.join(TINY, "manifest.json")))
    by_path = {os.path.relpath(e["path"], "goldens/tiny/g1"): e for e in manifest["files"]}
    checked = 0
    for root, _, files in os.walk(TINY):
        for name in sorted(files):
            if not name.endswith(".safetensors"):
                continue
            rel = os.path.relpath(os.path.join(root, name), TINY)
            pin = by_path[rel]
            with st.SafetensorsFile.open_verified(os.path.join(root, name), pin["bytes"], pin["sha256"]) as f:
                assert f.is_aligned, rel
                tensors = [(e.name, e.dtype, f.read(e.name)) for e in f.entries]
                again = st.to_bytes(tensors, f.metadata)
                assert hashlib.sha256(again).hexdigest() == pin["sha256"], rel + " rewritten"
                checked += 1
    assert checked >= 9
    with st.SafetensorsFile.open(os.path.join(TINY, "model", "model.safetensors")) as m:
        assert (len(m.entries), m.header_length) == (24, 2480), "tiny model: 24 tensors, N = 2,480"
        assert m.metadata == [("format", "pt")]
        assert all(e.dtype == "BF16" for e in m.entries)
        assert "lm_head.weight" not in m, "no lm_head (tied)"


def test_open_verified_checks_size_and_sha256_before_parsing(tmp_path):
    b = s1_bytes()
    p = tmp_path / "v.safetensors"
    p.write_bytes(b)
    st.SafetensorsFile.open_verified(str(p), len(b), S1_SHA256).close()
    with pytest.raises(IntegrityError):
        st.SafetensorsFile.open_verified(str(p), len(b) + 1, S1_SHA256)
    with pytest.raises(IntegrityError):
        st.SafetensorsFile.open_verified(str(p), len(b), hashlib.sha256(b"x").hexdigest())
    junk = tmp_path / "junk.safetensors"
    junk.write_bytes(b"\xff" * 64)
    with pytest.raises(IntegrityError):  # the hash is checked before the garbage header is parsed
        st.SafetensorsFile.open_verified(str(junk), 64, hashlib.sha256(b"x").hexdigest())


OK = entry("F32", "[1]", 0, 4)
D4 = bytes(4)
MALFORMED = [
    ("not JSON", '{"a":', D4),
    ("not an object", "[1, 2]", D4),
    ("leading space", " {}", b""),
    ("duplicate name", '{"a":' + OK + ',"a":' + OK + "}", D4),
    ("unknown dtype", '{"a":' + entry("BOOL", "[4]", 0, 4) + "}", D4),
    ("negative dimension", '{"a":' + entry("U8", "[-4]", 0, 4) + "}", D4),
    ("fractional dimension", '{"a":' + entry("U8", "[4.0]", 0, 4) + "}", D4),
    ("size mismatch", '{"a":' + entry("F32", "[2]", 0, 4) + "}", D4),
    ("end beyond the data", '{"a":' + entry("U8", "[8]", 0, 8) + "}", D4),
    ("reversed offsets", '{"a":' + entry("U8", "[0]", 4, 0) + "}", D4),
    ("hole", '{"a":' + entry("U8", "[2]", 2, 4) + "}", D4),
    ("overlap", '{"a":' + entry("U8", "[3]", 0, 3) + ',"b":' + entry("U8", "[2]", 2, 4) + "}", D4),
    ("trailing bytes", '{"a":' + entry("U8", "[2]", 0, 2) + "}", D4),
    ("offsets not a pair", '{"a":{"dtype":"U8","shape":[4],"data_offsets":[0]}}', D4),
    ("missing field", '{"a":{"dtype":"U8","shape":[4]}}', D4),
    ("unknown field", '{"a":{"dtype":"U8","shape":[4],"data_offsets":[0,4],"x":1}}', D4),
    ("empty name", '{"":' + OK + "}", D4),
    ("metadata not strings", '{"__metadata__":{"k":1},"a":' + OK + "}", D4),
    ("metadata not an object", '{"__metadata__":[],"a":' + OK + "}", D4),
    ("lone high surrogate in a name", '{"' + esc("d800") + '":' + OK + "}", D4),
    ("lone low surrogate in a name", '{"a' + esc("dc00") + 'b":' + OK + "}", D4),
    ("high surrogate without its low half", '{"' + esc("d83d") + esc("0041") + '":' + OK + "}", D4),
    ("lone surrogate in a metadata key", '{"__metadata__":{"' + esc("dc00") + '":"v"},"a":' + OK + "}", D4),
    ("lone surrogate in a metadata value", '{"__metadata__":{"k":"' + esc("dc00") + '"},"a":' + OK + "}", D4),
    ("lone surrogate in a dtype", '{"a":' + entry("U" + esc("d800"), "[4]", 0, 4) + "}", D4),
    ("lone surrogate in a field name",
     '{"a":{"dtype":"U8","shape":[4],"data_offsets":[0,4],"' + esc("d800") + '":1}}', D4),
    ("invalid UTF-8 in a name", b'{"a' + b"\xff" + ('":' + OK + "}").encode(), D4),
    ("invalid UTF-8 in a metadata value",
     b'{"__metadata__":{"k":"v' + b"\xc3" + ('"},"a":' + OK + "}").encode(), D4),
    ("a UTF-8 encoded surrogate (CESU-8)", b'{"a' + b"\xed\xa0\x80" + ('":' + OK + "}").encode(), D4),
    ("an overlong UTF-8 encoding", b'{"' + b"\xc1\x81" + ('":' + OK + "}").encode(), D4),
    ("nesting deeper than 8", '{"__metadata__":' + "[" * 8 + "]" * 8 + "}", b""),
    ("a trailing comma", '{"a":' + OK + ",}", D4),
]


@pytest.mark.parametrize("label,header,data", MALFORMED, ids=[m[0] for m in MALFORMED])
def test_the_reader_rejects_malformed_headers(tmp_path, label, header, data):
    expect_format_error(tmp_path, label, raw_file(header, data))


def test_the_reader_rejects_bad_lengths(tmp_path):
    expect_format_error(tmp_path, "short", bytes([1, 2]))
    expect_format_error(tmp_path, "N", (100).to_bytes(8, "little") + bytes(8))
    expect_format_error(tmp_path, "cap", (100_000_001).to_bytes(8, "little") + bytes(8))


def test_the_reader_decodes_escaped_names_that_are_valid_unicode():
    header = ('{"' + esc("d83d") + esc("de00") + '":' + entry("U8", "[2]", 0, 2) + ',"' + esc("0041") + '":'
              + entry("U8", "[2]", 2, 4) + "}")
    f = st.SafetensorsFile.validate(raw_file(header, bytes(4)))
    assert f.names == ["A", "\U0001F600"], "decoded, in code point order"


def test_the_reader_accepts_any_header_length_and_records_alignment(tmp_path):
    header = '{"a":' + entry("U8", "[4]", 0, 4) + "}"
    p = tmp_path / "u.safetensors"
    p.write_bytes(raw_file(header, bytes([1, 2, 3, 4])))
    with st.SafetensorsFile.open(str(p)) as f:
        assert f.header_length == len(header) and len(header) % 8 != 0
        assert not f.is_aligned, "data start not a multiple of 8"
        assert f.read("a").tolist() == [1, 2, 3, 4]


def test_the_writer_rejects_duplicate_reserved_and_invalid_names_and_short_data():
    def t(n):
        return (n, "U8", np.zeros(1, np.uint8))

    for bad in ([t("a"), t("a")], [t("__metadata__")], [t("")], [t("\ud800")]):
        with pytest.raises(ValueError):
            st.to_bytes(bad)
    with pytest.raises(ValueError):  # two bytes cannot hold two F32 values
        st.header([], [("a", "F32", (2,), 1)])
    with pytest.raises(ValueError):
        st.to_bytes([], [("k", "1"), ("k", "2")])


def test_save_replaces_the_target_atomically_and_leaves_no_temporary_file(tmp_path):
    p = tmp_path / "w.safetensors"
    p.write_text("old")
    st.save(str(p), S1_TENSORS, S1_META)
    assert hashlib.sha256(p.read_bytes()).hexdigest() == S1_SHA256
    assert os.listdir(tmp_path) == ["w.safetensors"]


@pytest.mark.parametrize("seed", range(12))
def test_round_trip_write_read_rewrite(tmp_path, seed):
    """SafetensorsTests.fs:393-420 on seeded samples: random dtypes, ranks 0..3, dims 0..4, names with characters that
    need escaping and astral characters, 0..2 metadata pairs."""
    r = np.random.default_rng(seed)
    names = list(st.DTYPES)
    tensors = []
    for i in range(int(r.integers(0, 12))):
        dt = names[int(r.integers(0, len(names)))]
        shape = tuple(int(x) for x in r.integers(0, 5, int(r.integers(0, 4))))
        raw = r.integers(0, 256, int(np.prod(shape)) * np.dtype(st.DTYPES[dt][1]).itemsize, dtype=np.uint8)
        name = f"t{i}" + ("\U0001F600" if i % 3 == 0 else "") + ('"' if i % 4 == 1 else "")
        tensors.append((name, dt, raw.view(st.DTYPES[dt][1]).reshape(shape)))
    meta = [(f"k{i}", f"v{i}\n") for i in range(int(r.integers(0, 3)))]
    b = st.to_bytes(tensors, meta)
    f = st.SafetensorsFile.validate(b)
    assert f.header_length % 8 == 0 and len(f.entries) == len(tensors) and f.metadata == sorted(meta)
    p = tmp_path / "r.safetensors"
    p.write_bytes(b)
    with st.SafetensorsFile.open(str(p)) as g:
        for name, dt, a in tensors:
            e = g.entry(name)
            assert e.dtype == dt and e.shape == a.shape
            assert g.read(name).tobytes() == a.tobytes()
        again = st.to_bytes([(e.name, e.dtype, g.read(e.name)) for e in g.entries], g.metadata)
        assert again == b and g.rebuild_header() == g.header_bytes()


def test_the_qwen3_0_6b_layout_header_matches_the_real_checkpoint():
    """The writer's header for the Qwen3-0.6B layout (311 BF16 entries: 28 layers x 11, the embedding, the final norm
    and the stored copy of the tied lm_head, metadata format=pt) is as long as the real checkpoint's: N = 35,552, data
    at 35,560 (tests/Lrm.Tensor.Tests/ModelTests.fs:16-29, where the reference's writer rebuilds that header byte for
    byte). Names, shapes, dtypes and order all enter the length."""
    import math

    from rosylnalive_amd.qwen import QwenConfig

    shapes = QwenConfig.qwen3_0_6b().weight_shapes()
    shapes["lm_head.weight"] = shapes["model.embed_tokens.weight"]
    h = st.header([("format", "pt")], [(n, "BF16", s, 2 * math.prod(s)) for n, s in shapes.items()])
    assert len(shapes) == 311
    assert int.from_bytes(h[:8], "little") == 35_552 and len(h) == 35_560
    assert shapes["lm_head.weight"] == (151_936, 1024)
