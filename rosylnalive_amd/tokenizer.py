"""The Qwen3 byte-level BPE tokenizer of liblrm_hip.so (csrc/tokenizer.cpp), with the interface of the reference's
QwenTokenizer (src/Lrm.Tokenizer/QwenTokenizer.fs): parse, encode, encode_bytes, decode_bytes, decode, id_of, token_of,
vocab_size, merge_count, added_tokens. Encode runs added tokens on the raw text (leftmost-longest), then for each
stretch between them the oracle's NFC, the Split pre-tokenizer and byte-level BPE; it adds no BOS or EOS.

The stages are exposed alone for their tests: pre_split (PreTokenizer.pieces), nfc (Nfc.normalize), scalar_tables
(the Split classes, the contraction letters and NFC's split points per scalar) and byte_char (ByteLevel.charOf).
"""
from __future__ import annotations

import ctypes as C
import hashlib
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np

from ._native import LrmError, TokenizerDataError, check, lib

__all__ = ["QwenTokenizer", "AddedToken", "TokenizerDataError", "pre_split", "nfc", "nfc_many", "scalar_tables",
           "byte_char", "byte_level", "MODEL_ROWS"]

MODEL_ROWS = 151_936  # Qwen3's embedding / lm_head rows (QwenTokenizer.ModelRows)


@dataclass(frozen=True)
class AddedToken:
    id: int
    content: str
    special: bool


def _utf8(text: str) -> bytes:
    """UTF-8 of `text`; a lone surrogate is refused as the reference refuses it (QwenTokenizer.fs:49-66)."""
    try:
        return text.encode("utf-8")
    except UnicodeEncodeError as e:
        raise ValueError(f"the text holds a lone surrogate U+{ord(text[e.start]):04X} at index {e.start}; only "
                         "Unicode scalar values can be encoded") from None


def _buf(data: bytes):
    return C.create_string_buffer(data, max(1, len(data)))


def _call_sized(fn, elem, first_cap):
    """fn(out, cap, count_ptr) with the size rule of the lrm_tok_* entry points: retry once with the size it needs."""
    count = C.c_uint64()
    cap = max(1, first_cap)
    out = (elem * cap)()
    check(fn(out, cap, C.byref(count)))
    if count.value > cap:
        cap = count.value
        out = (elem * cap)()
        check(fn(out, cap, C.byref(count)))
    return out, count.value


class QwenTokenizer:
    def __init__(self, handle: C.c_void_p, sha256: str):
        self._h = handle
        self.sha256 = sha256
        v, m, a = C.c_int32(), C.c_int32(), C.c_int32()
        check(lib().lrm_tok_info(self._h, C.byref(v), C.byref(m), C.byref(a)))
        self.vocab_size, self.merge_count = v.value, m.value
        self.added_tokens: List[AddedToken] = [self._added(i) for i in range(a.value)]

    @classmethod
    def parse(cls, json_bytes: bytes) -> "QwenTokenizer":
        """A tokenizer from tokenizer.json bytes, structure checked (QwenTokenizer.parse); TokenizerDataError for a
        configuration other than Qwen3's."""
        h = C.c_void_p()
        check(lib().lrm_tok_parse(_buf(json_bytes), len(json_bytes), C.byref(h)))
        return cls(h, hashlib.sha256(json_bytes).hexdigest())

    @classmethod
    def load(cls, path: str, sha256: Optional[str] = None) -> "QwenTokenizer":
        """Reads tokenizer.json; with `sha256` the file must have that SHA-256 before it is parsed (QwenTokenizer.load
        pins the Qwen3-0.6B file)."""
        data = open(path, "rb").read()
        got = hashlib.sha256(data).hexdigest()
        if sha256 is not None and got != sha256.lower():
            raise TokenizerDataError(8, f"{path} has SHA-256 {got}, but the pin is {sha256.lower()}")
        return cls.parse(data)

    def _added(self, i: int) -> AddedToken:
        tid, n, sp = C.c_int32(), C.c_int32(), C.c_int32()
        check(lib().lrm_tok_added(self._h, i, C.byref(tid), None, 0, C.byref(n), C.byref(sp)))
        b = C.create_string_buffer(max(1, n.value))
        check(lib().lrm_tok_added(self._h, i, C.byref(tid), b, n.value, C.byref(n), C.byref(sp)))
        return AddedToken(tid.value, b.raw[:n.value].decode("utf-8"), bool(sp.value))

    def encode(self, text: str) -> List[int]:
        data = _utf8(text)
        src = _buf(data)
        out, n = _call_sized(lambda o, c, k: lib().lrm_tok_encode(self._h, src, len(data), o, c, k), C.c_int32,
                             len(data) + 16)
        return list(out[:n])

    def encode_bytes(self, data: bytes) -> List[int]:
        """EncodeBytes: each maximal ill-formed UTF-8 subpart becomes one U+FFFD first."""
        src = _buf(data)
        out, n = _call_sized(lambda o, c, k: lib().lrm_tok_encode_bytes(self._h, src, len(data), o, c, k),
                             C.c_int32, 3 * len(data) + 16)
        return list(out[:n])

    def decode_bytes(self, ids: Sequence[int]) -> bytes:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        out, n = _call_sized(lambda o, c, k: lib().lrm_tok_decode_bytes(self._h, a.ctypes.data, a.size, o, c, k),
                             C.c_uint8, 8 * a.size + 16)
        return bytes(out[:n])

    def decode(self, ids: Sequence[int]) -> str:
        """decode_bytes as UTF-8, one U+FFFD per maximal ill-formed subpart (errors="replace")."""
        return self.decode_bytes(ids).decode("utf-8", errors="replace")

    def id_of(self, token: str) -> Optional[int]:
        data = token.encode("utf-8", errors="surrogatepass")
        r = C.c_int32()
        check(lib().lrm_tok_id_of(self._h, _buf(data), len(data), C.byref(r)))
        return None if r.value < 0 else r.value

    def token_of(self, tid: int) -> Optional[str]:
        n = C.c_int32()
        check(lib().lrm_tok_token_of(self._h, int(tid), None, 0, C.byref(n)))
        if n.value < 0:
            return None
        b = C.create_string_buffer(max(1, n.value))
        check(lib().lrm_tok_token_of(self._h, int(tid), b, n.value, C.byref(n)))
        return b.raw[:n.value].decode("utf-8")

    def close(self) -> None:
        if getattr(self, "_h", None):
            check(lib().lrm_tok_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pre_split(text: str) -> List[str]:
    """The Split pre-tokenizer's pieces of `text` (PreTokenizer.pieces)."""
    data = _utf8(text)
    src = _buf(data)
    out, n = _call_sized(lambda o, c, k: lib().lrm_tok_pre_split(src, len(data), o, c, k), C.c_uint64,
                         len(data) + 2)
    b = list(out[:n])
    return [data[b[i]:b[i + 1]].decode("utf-8") for i in range(len(b) - 1)]


def nfc(text: str) -> str:
    """The oracle's NFC (Nfc.normalize)."""
    data = _utf8(text)
    src = _buf(data)
    out, n = _call_sized(lambda o, c, k: lib().lrm_tok_nfc(src, len(data), o, c, k), C.c_uint8, 3 * len(data) + 16)
    return bytes(out[:n]).decode("utf-8")


def nfc_many(texts: Sequence[str]) -> List[str]:
    """nfc of each text, in one call."""
    enc = [_utf8(t) for t in texts]
    offsets = np.zeros(len(enc) + 1, np.uint64)
    np.cumsum([len(b) for b in enc], out=offsets[1:])
    data = b"".join(enc)
    src = _buf(data)
    cap = 3 * len(data) + 16
    out = (C.c_uint8 * cap)()
    out_offsets = np.zeros(len(enc) + 1, np.uint64)
    n = C.c_uint64()
    check(lib().lrm_tok_nfc_many(src, offsets.ctypes.data, len(enc), out, cap, out_offsets.ctypes.data, C.byref(n)))
    if n.value > cap:
        raise LrmError(4, "NFC grew a batch beyond three times its bytes")
    raw = bytes(out[:n.value])
    return [raw[int(out_offsets[i]):int(out_offsets[i + 1])].decode("utf-8") for i in range(len(enc))]


def scalar_tables():
    """Per scalar 0 .. 0x10FFFF: the Split class (0 letter, 1 number, 2 space, 3 other), the contraction letter (its
    ASCII code, 0 for none) and 1 where NFC splits the text."""
    cls = np.zeros(0x110000, np.uint8)
    con = np.zeros(0x110000, np.uint8)
    spl = np.zeros(0x110000, np.uint8)
    check(lib().lrm_tok_scalar_tables(cls.ctypes.data, con.ctypes.data, spl.ctypes.data))
    return cls, con, spl


def byte_char(b: int) -> str:
    """The character that stands for byte b in the byte-level alphabet (ByteLevel.charOf)."""
    c = C.c_uint32()
    check(lib().lrm_tok_byte_char(int(b), C.byref(c)))
    return chr(c.value)


def byte_level(data: bytes) -> str:
    """The byte-level string of `data` (ByteLevel.encode)."""
    return "".join(byte_char(b) for b in data)
