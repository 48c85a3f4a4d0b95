"""The Qwen3 tokenizer (liblrm_hip.so, lrm_tok_*), after the reference's tokenizer tests
(tests/Lrm.Tokenizer.Tests: PreTokenizerTests.fs, UnicodeTests.fs, ToyTests.fs, CorpusTests.fs). CPU only.

The Qwen3-0.6B tokenizer.json (151,643 tokens, 151,387 merges) is not in the reference or in this image, as it is not
on the reference's CI runners, where its corpus tests skip. What pins the tokenizer here:
- the Split pre-tokenizer: vectors P1-P18 and the oracle's 4,000 split cases (tests/golden/tokenizer/split-cases.jsonl,
  from HF tokenizers 0.23.3);
- the Unicode data: every scalar's Split class and contraction letter against the oracle's probe
  (unicode-oracle.json), and the NFC against the oracle's digests of its probe families F1-F9 over every scalar, K over
  every canonical decomposition and P over every pair of reordering marks;
- BPE, added tokens, decoding and the loader: the reference's toy tokenizer.json (263 tokens, 7 merges, 3 added) and its
  known answers;
- the corpus (goldens/tokenizer/g1/cases.jsonl, the rows that need no vocabulary, corpus-subset.jsonl): 350 decode
  cases whose ids are single bytes, added tokens or rows with no token, on a tokenizer with Qwen3's byte ids and added
  tokens; where the added tokens fall in 438 encode cases; EncodeBytes' replacement of ill-formed UTF-8 in 141 cases;
  the refusal of 8 lone surrogates.
BPE merge ranks of the real vocabulary and the ids of ordinary text stay unpinned without tokenizer.json.
"""
import hashlib
import json
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from conftest import GOLDEN
from rosylnalive_amd import tokenizer as T
from rosylnalive_amd.tokenizer import QwenTokenizer, TokenizerDataError

TOK = os.path.join(GOLDEN, "tokenizer")
ORACLE = json.load(open(os.path.join(TOK, "unicode-oracle.json")))
SPLIT_CASES = [json.loads(l) for l in open(os.path.join(TOK, "split-cases.jsonl"), encoding="utf-8")]
SCALARS = [c for c in range(0x110000) if not 0xD800 <= c <= 0xDFFF]


def hexs(s):
    return " ".join("%x" % ord(x) for x in s)


# ---------------------------------------------------------------- the Split pre-tokenizer (PreTokenizerTests.fs)

SPLIT_VECTORS = [  # P1 .. P18 (PreTokenizerTests.fs:11-33)
    ("Hello world", ["Hello", " world"]),
    ("it's", ["it", "'s"]),
    ("WE'RE 'Sa", ["WE", "'RE", " '", "Sa"]),
    ("x'ſa", ["x", "'ſ", "a"]),
    ("  hi", [" ", " hi"]),
    ("a  \n\n  b", ["a", "  \n\n", " ", " b"]),
    ("end   ", ["end", "   "]),
    ("12345", ["1", "2", "3", "4", "5"]),
    ("x½Ⅻ", ["x", "½", "Ⅻ"]),
    (" !!\r\n\r\nx", [" !!\r\n\r\n", "x"]),
    ("\tfoo", ["\tfoo"]),
    ("　中文", ["　中文"]),
    ("\U0001D400\U0001D401", ["\U0001D400\U0001D401"]),
    ("a\r\nb", ["a", "\r\n", "b"]),
    ("x ́y", ["x", " ́", "y"]),
    ("'ll've", ["'ll", "'ve"]),
    ("don't'", ["don", "'t", "'"]),
    ("\U0001D7CE\U0001D7CF", ["\U0001D7CE", "\U0001D7CF"]),
]


@pytest.mark.parametrize("text,pieces", SPLIT_VECTORS)
def test_split_vectors(text, pieces):
    assert T.pre_split(text) == pieces


def test_every_oracle_split_case_and_the_pieces_tile_the_text():
    assert len(SPLIT_CASES) >= 4000
    bad = [(c["text"], T.pre_split(c["text"]), c["pieces"]) for c in SPLIT_CASES if T.pre_split(c["text"]) != c["pieces"]]
    assert not bad, bad[:5]
    for c in SPLIT_CASES:
        assert "".join(T.pre_split(c["text"])) == c["text"]
    assert T.pre_split("") == []


def test_the_byte_map_vector_b1_and_bijection():
    for b, c in [(0x00, "Ā"), (0x09, "ĉ"), (0x0A, "Ċ"), (0x20, "Ġ"), (0x21, "!"), (0x7E, "~"),
                 (0x7F, "ġ"), (0xA0, "ł"), (0xA1, "¡"), (0xAC, "¬"), (0xAD, "Ń"),
                 (0xFF, "ÿ")]:
        assert T.byte_char(b) == c, hex(b)
    chars = [T.byte_char(b) for b in range(256)]
    assert len(set(chars)) == 256
    assert sorted(c for c in chars if c >= "Ā") == [chr(c) for c in range(0x100, 0x144)]


# ---------------------------------------------------------------- Unicode data (UnicodeTests.fs)

@pytest.fixture(scope="module")
def tables():
    return T.scalar_tables()


def test_every_scalars_class_equals_the_oracles(tables):
    cls, _, _ = tables
    code = {"L": 0, "N": 1, "S": 2, "O": 3}
    want = np.empty(0x110000, np.uint8)
    runs = ORACLE["classes"]
    for i, (start, k) in enumerate(runs):
        end = runs[i + 1][0] if i + 1 < len(runs) else 0x110000
        want[start:end] = code.get(k, 3)
    s = np.array(SCALARS)
    bad = s[cls[s] != want[s]]
    assert bad.size == 0, [hex(c) for c in bad[:20]]


def test_every_scalars_class_agrees_with_the_regex_module(tables):
    """Pins the compiled class table by something other than the probe file it was generated from: Python's regex
    module (its own Unicode 17.0 tables) classifies every scalar as \\p{L}, \\p{N}, \\s or other; the compiled
    table (Unicode 16.0, the tokenizer specification's) may differ from it only on scalars that Python's unicodedata
    (Unicode 13.0) leaves unassigned, i.e. on letters and numbers added after 13.0. A class moved between two assigned
    scalars, a dropped run or a shifted run boundary fails here."""
    import unicodedata

    regex = pytest.importorskip("regex")
    cls, _, _ = tables
    L, N, S = regex.compile(r"\p{L}"), regex.compile(r"\p{N}"), regex.compile(r"\s")
    differ = []
    for c in SCALARS:
        ch = chr(c)
        theirs = 0 if L.match(ch) else 1 if N.match(ch) else 2 if S.match(ch) else 3
        if int(cls[c]) != theirs:
            differ.append(c)
    assigned = [hex(c) for c in differ if unicodedata.category(chr(c)) != "Cn"]
    assert not assigned, assigned[:20]
    # the Unicode 14.0-16.0 additions the two versions disagree on are a few thousand scalars, not a whole plane
    assert len(differ) < 20000, len(differ)
    # and the well-known members of each class
    for c, k in ((ord("a"), 0), (0x4E00, 0), (ord("7"), 1), (0x0663, 1), (ord(" "), 2), (0x3000, 2), (ord("!"), 3)):
        assert int(cls[c]) == k, hex(c)


def test_the_contraction_group_matches_exactly_the_oracles_letters(tables):
    _, con, _ = tables
    want = {}
    for key, cps in ORACLE["contraction_letters"].items():
        for c in cps:
            letters = key.split(" ")[0].split("|")
            want.setdefault(c, set()).update(letters)
    got = {c: chr(con[c]) for c in SCALARS if con[c]}
    assert set(got) == set(want)
    for c, letter in got.items():
        assert letter in want[c], hex(c)
    assert ORACLE["apostrophes"] == [0x27]
    # only U+0027 opens a contraction, on every BMP scalar
    opens = [c for c in range(0x10000) if not 0xD800 <= c <= 0xDFFF
             and T.pre_split("x" + chr(c) + "sa") == ["x", chr(c) + "s", "a"]]
    assert opens == [0x27]


FAMILIES = [("F1", lambda ch: ch), ("F2", lambda ch: "a" + ch + "̴"), ("F3", lambda ch: "aͅ" + ch),
            ("F5", lambda ch: ch + "́"), ("F6", lambda ch: "a" + ch), ("F7", lambda ch: ch + "̈"),
            ("F8", lambda ch: "ᄀ" + ch), ("F9", lambda ch: "가" + ch)]


def _digest(lines):
    h = hashlib.sha256()
    for line in lines:
        h.update(line.encode("utf-8"))
    return len(lines), h.hexdigest()


@pytest.mark.parametrize("name,build", FAMILIES, ids=[f[0] for f in FAMILIES])
def test_nfc_family_equals_the_oracles_nfc_on_every_scalar(name, build):
    inputs = [build(chr(c)) for c in SCALARS]
    outs = T.nfc_many(inputs)
    lines = ["%s %x %s\n" % (name, c, hexs(o)) for c, i, o in zip(SCALARS, inputs, outs) if o != i]
    want = ORACLE["nfc"][name]
    assert _digest(lines) == (want["count"], want["sha256"])


def test_nfc_family_k_every_canonical_decomposition_recomposed():
    seqs = ["".join(chr(int(x, 16)) for x in s.split()) for s in ORACLE["composition_inputs"]]
    outs = T.nfc_many(seqs)
    lines = ["K %d %s\n" % (i, hexs(o)) for i, (s, o) in enumerate(zip(seqs, outs)) if o != s]
    assert _digest(lines) == (ORACLE["nfc"]["K"]["count"], ORACLE["nfc"]["K"]["sha256"])


def test_nfc_family_p_every_pair_of_reordering_marks():
    marks = [c for a, b in ORACLE["marks"] for c in range(a, b + 1)]
    h = hashlib.sha256()
    n = 0
    for m1 in marks:
        inputs = ["a" + chr(m1) + chr(m2) for m2 in marks]
        for m2, i, o in zip(marks, inputs, T.nfc_many(inputs)):
            if o != i:
                h.update(("P %x %x %s\n" % (m1, m2, hexs(o))).encode("utf-8"))
                n += 1
    assert (n, h.hexdigest()) == (ORACLE["nfc"]["P"]["count"], ORACLE["nfc"]["P"]["sha256"])


def test_nfc_split_points_and_the_scalars_newer_than_the_oracles_tables(tables):
    _, _, spl = tables
    want = np.zeros(0x110000, np.uint8)
    for a, b in ORACLE["split_points"]:
        want[a:b + 1] = 1
    assert want[0xFFFE] == 1
    assert np.array_equal(spl[np.array(SCALARS)], want[np.array(SCALARS)])
    assert T.nfc("é￾ä") == "é￾ä", "NFC on both sides of U+FFFE"
    assert T.nfc("a̴߽") == "a̴߽", "U+07FD (Unicode 11) is inert in the oracle: no reordering"
    assert T.nfc("é") == "é" and T.nfc("각") == "각"


# ---------------------------------------------------------------- the toy tokenizer (ToyTests.fs)

TOY_MERGES = [(" ", "t"), ("h", "e"), (" t", "he"), ("a", "a"), ("b", "c"), ("a", "b"), ("aa", "aa")]
TOY_ADDED = [("<|a|>", True), ("<|ab|>", True), ("<x>", False)]
SPLIT_PATTERN = ("(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\\r\\n\\p{L}\\p{N}]?\\p{L}+|\\p{N}| ?[^\\s\\p{L}\\p{N}]+[\\r\\n]*|"
                 "\\s*[\\r\\n]+|\\s+(?!\\S)|\\s+")


def bl(s):
    return T.byte_level(s.encode("utf-8"))


def byte_level_step():
    return {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": False, "use_regex": False}


def toy_json(edit=None, vocab=None, merges=None, added=None):
    """The reference's toy tokenizer.json (ToyTests.fs:35-96): 256 byte tokens, 7 merges, 3 added tokens."""
    if vocab is None:
        vocab = {T.byte_char(b): b for b in range(256)}
        for i, (l, r) in enumerate(TOY_MERGES):
            vocab[bl(l) + bl(r)] = 256 + i
    if merges is None:
        merges = [[bl(l), bl(r)] for l, r in TOY_MERGES]
    if added is None:
        added = [{"id": len(vocab) + i, "content": c, "single_word": False, "lstrip": False, "rstrip": False,
                  "normalized": False, "special": sp} for i, (c, sp) in enumerate(TOY_ADDED)]
    root = {
        "version": "1.0", "truncation": None, "padding": None, "normalizer": {"type": "NFC"},
        "pre_tokenizer": {"type": "Sequence", "pretokenizers": [
            {"type": "Split", "pattern": {"Regex": SPLIT_PATTERN}, "behavior": "Isolated", "invert": False},
            byte_level_step()]},
        "post_processor": byte_level_step(), "decoder": byte_level_step(), "added_tokens": added,
        "model": {"type": "BPE", "dropout": None, "unk_token": None, "continuing_subword_prefix": "",
                  "end_of_word_suffix": "", "fuse_unk": False, "byte_fallback": False, "ignore_merges": False,
                  "vocab": vocab, "merges": merges},
    }
    if edit:
        edit(root)
    return json.dumps(root).encode("utf-8")


@pytest.fixture(scope="module")
def toy():
    return QwenTokenizer.parse(toy_json())


def test_toy_bpe_merges_the_lowest_rank_first_and_the_leftmost_among_equal_ranks(toy):
    idof = lambda s: toy.id_of(bl(s))
    assert toy.encode(" the") == [idof(" the")]
    assert toy.encode("abc") == [idof("a"), idof("bc")], "'bc' (rank 4) before 'ab' (rank 5)"
    assert toy.encode("aaa") == [idof("aa"), idof("a")]
    assert toy.encode("aaaa") == [idof("aaaa")]
    assert toy.encode("aaaaa") == [idof("aaaa"), idof("a")]
    assert toy.encode("") == []
    ids = toy.encode("a" * 100_001)  # one long piece
    assert len(ids) == 25_001 and set(ids[:25_000]) == {idof("aaaa")} and ids[-1] == idof("a")
    assert toy.encode(" the" * 30_000) == [idof(" the")] * 30_000
    assert toy.encode(" the aa") == [idof(" the"), idof(" "), idof("aa")]


def byte_ids(toy, s):
    return [toy.id_of(T.byte_char(b)) for b in s.encode("utf-8")]


def test_toy_added_tokens_match_first_leftmost_longest_on_the_raw_text(toy):
    assert toy.encode("<|ab|>") == [264]
    assert toy.encode("<|a|><|ab|>") == [263, 264]
    assert toy.encode("x<x>y") == byte_ids(toy, "x") + [265] + byte_ids(toy, "y")
    assert toy.encode("<|a") == byte_ids(toy, "<|a")
    assert toy.encode("<<x>") == byte_ids(toy, "<") + [265]


def test_toy_nfc_runs_on_each_stretch_between_added_tokens(toy):
    assert toy.encode("é") == byte_ids(toy, "é")
    assert toy.encode("e<x>́") == byte_ids(toy, "e") + [265] + byte_ids(toy, "́")


def test_toy_lone_surrogates_are_refused_and_pairs_encoded(toy):
    for h in ["d800", "0061dc00", "0061d800d8000062", "dfff0061"]:
        with pytest.raises(ValueError):
            toy.encode(bytes.fromhex(h).decode("utf-16-be", "surrogatepass"))
    assert toy.encode("\U0001F600") == byte_ids(toy, "\U0001F600")


def test_toy_encode_bytes_replaces_each_maximal_ill_formed_subpart(toy):
    assert toy.encode_bytes(b"\x80") == byte_ids(toy, "�")
    assert toy.encode_bytes(b"\xe4\xb8") == byte_ids(toy, "�")
    assert toy.encode_bytes(b"a\xf0\x80b") == byte_ids(toy, "a��b")


def test_toy_decode(toy):
    idof = lambda s: toy.id_of(bl(s))
    assert toy.decode_bytes([idof(" the")]) == b" the"
    assert toy.decode([263, 265]) == "<|a|><x>"
    assert toy.decode_bytes([]) == b""
    assert toy.decode_bytes([toy.vocab_size, 151_935]) == b"", "rows with no token add nothing"
    zhong = byte_ids(toy, "中")
    assert toy.decode([zhong[0], 151_700, zhong[1], zhong[2]]) == "中"
    assert toy.decode([zhong[0]]) == "�"
    assert toy.decode([zhong[0], zhong[1], idof("a")]) == "�a"
    for bad in [-1, T.MODEL_ROWS, 2**31 - 1]:
        with pytest.raises(Exception) as e:
            toy.decode_bytes([bad])
        assert "outside the model" in str(e.value)


def test_toy_id_of_and_token_of(toy):
    assert toy.id_of("<|ab|>") == 264
    assert toy.id_of(bl(" the")) == 258
    assert toy.id_of(" the") is None
    assert toy.token_of(258) == bl(" the")
    assert toy.token_of(265) == "<x>"
    assert toy.token_of(266) is None
    assert toy.vocab_size == 266 and toy.merge_count == 7
    assert [a.special for a in toy.added_tokens] == [True, True, False]


def _pre(r):
    return r["pre_tokenizer"]["pretokenizers"]


REFUSALS = [  # ToyTests.fs:231-256
    ("another regex", lambda r: _pre(r)[0]["pattern"].__setitem__("Regex", "\\p{L}+|\\s+")),
    ("behaviour Removed", lambda r: _pre(r)[0].__setitem__("behavior", "Removed")),
    ("ByteLevel with use_regex", lambda r: _pre(r)[1].__setitem__("use_regex", True)),
    ("ByteLevel without use_regex", lambda r: _pre(r)[1].pop("use_regex")),
    ("add_prefix_space", lambda r: _pre(r)[1].__setitem__("add_prefix_space", True)),
    ("NFKC", lambda r: r["normalizer"].__setitem__("type", "NFKC")),
    ("dropout", lambda r: r["model"].__setitem__("dropout", 0.1)),
    ("byte fallback", lambda r: r["model"].__setitem__("byte_fallback", True)),
    ("ignore_merges", lambda r: r["model"].__setitem__("ignore_merges", True)),
    ("an unknown token", lambda r: r["model"].__setitem__("unk_token", "<unk>")),
    ("a normalized added token", lambda r: r["added_tokens"][0].__setitem__("normalized", True)),
    ("an lstrip added token", lambda r: r["added_tokens"][1].__setitem__("lstrip", True)),
    ("an added token id gap", lambda r: r["added_tokens"][2].__setitem__("id", 300)),
    ("a merge of an unknown token", lambda r: r["model"]["merges"].append(["zz", "a"])),
    ("a merge whose result is missing", lambda r: r["model"]["merges"].append(["b", "b"])),
    ("a vocabulary id gap", lambda r: r["model"]["vocab"].__setitem__(bl(" the"), 999)),
    ("a decoder that is not ByteLevel", lambda r: r["decoder"].__setitem__("type", "WordPiece")),
    ("a model that is not BPE", lambda r: r["model"].__setitem__("type", "Unigram")),
]


@pytest.mark.parametrize("name,edit", REFUSALS, ids=[r[0] for r in REFUSALS])
def test_toy_loader_refuses(name, edit):
    with pytest.raises(TokenizerDataError):
        QwenTokenizer.parse(toy_json(edit))


def test_toy_merges_as_strings_and_the_sha256_pin(toy, tmp_path):
    t = QwenTokenizer.parse(toy_json(merges=[bl(l) + " " + bl(r) for l, r in TOY_MERGES]))
    assert t.encode(" the aaaaa") == toy.encode(" the aaaaa")
    p = tmp_path / "tokenizer.json"
    p.write_bytes(toy_json())
    assert QwenTokenizer.load(str(p), hashlib.sha256(toy_json()).hexdigest()).vocab_size == 266
    with pytest.raises(TokenizerDataError):
        QwenTokenizer.load(str(p), "00" * 32)


def test_toy_decoding_the_encoding_gives_the_nfc_text_back_and_threads_agree(toy):
    texts = [c["text"] for c in SPLIT_CASES]
    seq = [toy.encode(s) for s in texts]
    for s, ids in zip(texts, seq):
        assert toy.decode(ids) == T.nfc(s)
    with ThreadPoolExecutor(8) as ex:
        par = list(ex.map(toy.encode, texts))
    assert par == seq


# ---------------------------------------------------------------- the corpus (CorpusTests.fs), without the vocabulary

def gpt2_byte_order():
    """Bytes in the order of their vocabulary ids in GPT-2-style byte-level vocabularies such as Qwen's: the printable
    bytes (0x21..0x7E, 0xA1..0xAC, 0xAE..0xFF), then the others, each in increasing order; so byte 0x00 is id 188."""
    printable = [b for b in range(256) if 0x21 <= b <= 0x7E or 0xA1 <= b <= 0xAC or 0xAE <= b <= 0xFF]
    return printable + [b for b in range(256) if b not in printable]


@pytest.fixture(scope="module")
def qwen_skeleton():
    """Qwen3's ids for the 256 byte tokens and its 26 added tokens (corpus manifest), the other 151,387 vocabulary
    ids filled with tokens no text reaches, no merges."""
    manifest = json.load(open(os.path.join(TOK, "corpus-manifest.json")))
    vocab = {T.byte_char(b): i for i, b in enumerate(gpt2_byte_order())}
    for i in range(256, 151_643):
        vocab[T.byte_level(b"\xff\xfe" + i.to_bytes(3, "big"))] = i
    added = [{"id": a["id"], "content": a["content"], "single_word": False, "lstrip": False, "rstrip": False,
              "normalized": False, "special": a["special"]} for a in manifest["added_tokens"]]
    t = QwenTokenizer.parse(toy_json(vocab=vocab, merges=[], added=added))
    assert t.vocab_size == 151_669
    return t


CORPUS = [json.loads(l) for l in open(os.path.join(TOK, "corpus-subset.jsonl"), encoding="utf-8")]


def test_corpus_decode_cases_of_bytes_and_added_tokens(qwen_skeleton):
    rows = [r for r in CORPUS if r["kind"] == "decode" and all(i < 256 or i >= 151_643 for i in r["ids"])]
    assert len(rows) == 350
    for r in rows:
        assert qwen_skeleton.decode_bytes(r["ids"]).hex() == r["bytes"], r["id"]
        assert qwen_skeleton.decode(r["ids"]) == r["text"], r["id"]


def test_corpus_added_tokens_fall_where_the_oracle_puts_them(qwen_skeleton):
    rows = [r for r in CORPUS if r["kind"] == "encode"]
    assert len(rows) == 438
    for r in rows:
        got = [i for i in qwen_skeleton.encode(r["text"]) if i >= 151_643]
        assert got == [i for i in r["ids"] if i >= 151_643], r["id"]


def test_corpus_encode_bytes_replaces_as_the_oracle(qwen_skeleton):
    rows = [r for r in CORPUS if r["kind"] == "encode_bytes"]
    assert len(rows) == 141
    for r in rows:
        ids = qwen_skeleton.encode_bytes(bytes.fromhex(r["bytes"]))
        assert qwen_skeleton.decode(ids) == T.nfc(r["text"]), r["id"]


def test_corpus_lone_surrogates_are_refused(qwen_skeleton):
    rows = [r for r in CORPUS if r["kind"] == "encode_reject"]
    assert len(rows) == 8
    for r in rows:
        with pytest.raises(ValueError, match="lone surrogate"):
            qwen_skeleton.encode(bytes.fromhex(r["utf16"]).decode("utf-16-be", "surrogatepass"))
