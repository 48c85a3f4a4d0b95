"""safetensors files: the validating reader of liblrm_hip.so and the deterministic writer.

The reader is SafetensorsFile (src/Lrm.Tensor/Safetensors.fs:504-727) in the library (csrc/safetensors.cpp, through
the lrm_st_* entry points): it maps the file read-only and checks the header length, the JSON, every dtype, shape and
offset range and that the tensors tile the data section exactly before anything is returned; a malformed file raises
SafetensorsFormatError, a size or SHA-256 that differs from a pinned one IntegrityError. bf16 tensors stay as their
bits (numpy uint16), which is what the kernels consume.

The writer is Safetensors.header / toBytes / writeFile (Safetensors.fs:113-255): "__metadata__" first, then the
tensors, each in code point order of the names, as compact ASCII JSON with strings escaped as Python's
json.dumps(ensure_ascii=True) escapes them, padded with spaces to a multiple of 8 bytes, the data in the same order
with no gaps. The same inputs in any order give the same bytes.
"""
from __future__ import annotations

import ctypes as C
import json
import math
import os
import struct
import uuid
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

import numpy as np

from . import _native as N
from ._native import IntegrityError, SafetensorsFormatError, check, lib

__all__ = ["SafetensorsFile", "SafetensorsFormatError", "IntegrityError", "Entry", "DTYPES", "load", "json_string",
           "header", "to_bytes", "save", "MAX_HEADER_BYTES"]

MAX_HEADER_BYTES = 100_000_000
# safetensors dtype name -> (library DType code, numpy dtype of the values; BF16 as raw bits)
DTYPES = {
    "F32": (1, np.float32),
    "BF16": (2, np.uint16),
    "F16": (3, np.float16),
    "I32": (4, np.int32),
    "U32": (5, np.uint32),
    "U8": (6, np.uint8),
    "F64": (7, np.float64),
    "I64": (8, np.int64),
}
_BY_CODE = {code: (name, dt) for name, (code, dt) in DTYPES.items()}


class Entry:
    """One tensor: name, safetensors dtype name, shape, and byte offsets [begin, end) in the data section."""

    __slots__ = ("name", "dtype", "shape", "begin", "end")

    def __init__(self, name, dtype, shape, begin, end):
        self.name, self.dtype, self.shape, self.begin, self.end = name, dtype, shape, begin, end

    @property
    def nbytes(self) -> int:
        return self.end - self.begin

    def __repr__(self):
        return f"Entry({self.name!r}, {self.dtype}, {self.shape}, [{self.begin}, {self.end}))"


def _decode(raw: bytes) -> str:
    return raw.decode("utf-8")


class SafetensorsFile:
    """A mapped, validated file (open / open_verified) or validated bytes (validate)."""

    def __init__(self, handle: C.c_void_p, keep=None):
        self._h = handle
        self._keep = keep
        hl, do, ne, nm, al, ln = C.c_int64(), C.c_int64(), C.c_int32(), C.c_int32(), C.c_int32(), C.c_uint64()
        check(lib().lrm_st_info(self._h, C.byref(hl), C.byref(do), C.byref(ne), C.byref(nm), C.byref(al),
                                C.byref(ln)))
        self.header_length, self.data_offset, self.length = hl.value, do.value, ln.value
        self.is_aligned = bool(al.value)
        self.entries: List[Entry] = [self._entry(i) for i in range(ne.value)]
        self.metadata: List[Tuple[str, str]] = [self._meta(i) for i in range(nm.value)]
        self._index = {e.name: i for i, e in enumerate(self.entries)}

    @classmethod
    def open(cls, path: str) -> "SafetensorsFile":
        h = C.c_void_p()
        check(lib().lrm_st_open(os.fsencode(path), C.byref(h)))
        return cls(h)

    @classmethod
    def open_verified(cls, path: str, nbytes: int, sha256_hex: str) -> "SafetensorsFile":
        h = C.c_void_p()
        check(lib().lrm_st_open_verified(os.fsencode(path), int(nbytes), sha256_hex.encode(), C.byref(h)))
        return cls(h)

    @classmethod
    def validate(cls, data: bytes) -> "SafetensorsFile":
        buf = (C.c_uint8 * max(1, len(data))).from_buffer_copy(data if data else b"\0")
        h = C.c_void_p()
        check(lib().lrm_st_validate(buf, len(data), C.byref(h)))
        return cls(h, keep=buf)

    def _entry(self, i: int) -> Entry:
        nlen, dt, rank, b, e = C.c_int32(), C.c_uint32(), C.c_int32(), C.c_int64(), C.c_int64()
        check(lib().lrm_st_entry(self._h, i, None, 0, C.byref(nlen), None, C.byref(rank), None, 0, None, None))
        name = C.create_string_buffer(max(1, nlen.value))
        dims = (C.c_int64 * max(1, rank.value))()
        check(lib().lrm_st_entry(self._h, i, name, nlen.value, C.byref(nlen), C.byref(dt), C.byref(rank), dims,
                                 rank.value, C.byref(b), C.byref(e)))
        return Entry(_decode(name.raw[:nlen.value]), _BY_CODE[dt.value][0], tuple(dims[k] for k in range(rank.value)),
                     b.value, e.value)

    def _meta(self, i: int) -> Tuple[str, str]:
        kl, vl = C.c_int32(), C.c_int32()
        check(lib().lrm_st_metadata(self._h, i, None, 0, C.byref(kl), None, 0, C.byref(vl)))
        k, v = C.create_string_buffer(max(1, kl.value)), C.create_string_buffer(max(1, vl.value))
        check(lib().lrm_st_metadata(self._h, i, k, kl.value, C.byref(kl), v, vl.value, C.byref(vl)))
        return _decode(k.raw[:kl.value]), _decode(v.raw[:vl.value])

    @property
    def names(self) -> List[str]:
        return [e.name for e in self.entries]

    def __contains__(self, name: str) -> bool:
        return name in self._index

    def entry(self, name: str) -> Entry:
        if name not in self._index:
            raise KeyError(f"no tensor {name!r}")
        return self.entries[self._index[name]]

    def try_metadata(self, key: str) -> Optional[str]:
        return dict(self.metadata).get(key)

    def read(self, name: str, dtype: Optional[str] = None) -> np.ndarray:
        """A copy of the tensor (BF16 as uint16 bits); with dtype, the tensor must have that dtype."""
        e = self.entry(name)
        if dtype is not None and dtype != e.dtype:
            raise TypeError(f"{name} is {e.dtype}, not {dtype}")
        p = C.c_void_p()
        check(lib().lrm_st_data(self._h, self._index[name], C.byref(p)))
        raw = C.string_at(p.value, e.nbytes) if e.nbytes else b""
        return np.frombuffer(raw, dtype=DTYPES[e.dtype][1]).reshape(e.shape).copy()

    def header_bytes(self) -> bytes:
        """The file's own first 8 + N bytes."""
        p = C.c_void_p()
        check(lib().lrm_st_data(self._h, -1, C.byref(p)))
        return C.string_at(p.value, self.data_offset)

    def rebuild_header(self) -> bytes:
        """The header the deterministic writer builds from this file's metadata and entries."""
        return header(self.metadata, [(e.name, e.dtype, e.shape, e.nbytes) for e in self.entries])

    def close(self) -> None:
        if getattr(self, "_h", None):
            check(lib().lrm_st_close(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def load(path: str) -> Dict[str, np.ndarray]:
    """Every tensor of a validated file as numpy arrays (BF16 as uint16 bits)."""
    with SafetensorsFile.open(path) as f:
        return {e.name: f.read(e.name) for e in f.entries}


# ---------------------------------------------------------------- the deterministic writer

def json_string(s: str) -> str:
    """A JSON string escaped as json.dumps(ensure_ascii=True): \\" \\\\ \\n \\r \\t \\b \\f, \\u00xx for the other
    control characters and DEL, \\uxxxx (lowercase) for every UTF-16 unit above U+007E (Safetensors.jsonString,
    Safetensors.fs:98-118). A lone surrogate is refused."""
    _utf8("name", s)
    return json.dumps(s, ensure_ascii=True)


def _utf8(what: str, s: str) -> bytes:
    try:
        return s.encode("utf-8")
    except UnicodeEncodeError:
        raise ValueError(f"{what} {s!r} is not valid Unicode (lone surrogate)") from None


def _code_point_key(s: str) -> bytes:
    return _utf8("name", s)


def header(metadata: Iterable[Tuple[str, str]], entries: Iterable[Tuple[str, str, Sequence[int], int]]) -> bytes:
    """The 8-byte length and the padded header for (name, dtype, shape, byte count) entries (Safetensors.header,
    Safetensors.fs:120-205). Raises ValueError for duplicate or reserved names, lone surrogates and byte counts that
    do not match the shape."""
    metadata, entries = list(metadata), list(entries)
    for what, names in (("metadata keys", [k for k, _ in metadata]), ("tensor names", [e[0] for e in entries])):
        dup = sorted({n for n in names if names.count(n) > 1})
        if dup:
            raise ValueError(f"duplicate {what} {dup}")
    for k, v in metadata:
        _utf8("metadata", k)
        _utf8("metadata", v)
    for name, dtype, shape, nbytes in entries:
        _utf8("entries", name)
        if not name:
            raise ValueError("empty tensor name")
        if name == "__metadata__":
            raise ValueError("the tensor name __metadata__ is reserved")
        if dtype not in DTYPES:
            raise ValueError(f"{name}: unsupported dtype {dtype}")
        expected = math.prod(int(d) for d in shape) * np.dtype(DTYPES[dtype][1]).itemsize
        if nbytes != expected:
            raise ValueError(f"{name}: {nbytes} bytes for {dtype}{list(shape)} (expected {expected})")
    parts = []
    if metadata:
        body = ",".join(json_string(k) + ":" + json_string(v) for k, v in sorted(metadata, key=lambda m: _code_point_key(m[0])))
        parts.append(json_string("__metadata__") + ":{" + body + "}")
    offset = 0
    for name, dtype, shape, nbytes in sorted(entries, key=lambda e: _code_point_key(e[0])):
        dims = ",".join(str(int(d)) for d in shape)
        parts.append(json_string(name) + f':{{"dtype":"{dtype}","shape":[{dims}],"data_offsets":[{offset},{offset + nbytes}]}}')
        offset += nbytes
    text = "{" + ",".join(parts) + "}"
    text += " " * ((8 - len(text) % 8) % 8)
    return struct.pack("<Q", len(text)) + text.encode("ascii")


def _tensor_list(tensors) -> List[Tuple[str, str, np.ndarray]]:
    """{name: (dtype, array)} or [(name, dtype, array)] -> [(name, dtype, contiguous array)]."""
    items = tensors.items() if isinstance(tensors, dict) else [(n, (d, a)) for n, d, a in tensors]
    out = []
    for name, (dtype, arr) in items:
        a = np.asarray(arr)
        if not a.flags.c_contiguous:  # (np.ascontiguousarray would turn a scalar into shape [1])
            a = a.copy(order="C")
        if dtype not in DTYPES:
            raise ValueError(f"{name}: unsupported dtype {dtype}")
        if a.dtype.itemsize != np.dtype(DTYPES[dtype][1]).itemsize:
            raise ValueError(f"{name}: a {a.dtype} array cannot hold {dtype} elements")
        out.append((name, dtype, a))
    return out


def to_bytes(tensors, metadata: Iterable[Tuple[str, str]] = ()) -> bytes:
    """The bytes of a deterministic file (Safetensors.toBytes, Safetensors.fs:221-226)."""
    ts = _tensor_list(tensors)
    head = header(metadata, [(n, d, a.shape, a.nbytes) for n, d, a in ts])
    return head + b"".join(a.tobytes() for _, _, a in sorted(ts, key=lambda t: _code_point_key(t[0])))


def save(path: str, tensors, metadata: Iterable[Tuple[str, str]] = ()) -> None:
    """Writes a deterministic file through a temporary file in the same folder that replaces `path` only when
    complete (Safetensors.writeFile, Safetensors.fs:228-243). tensors: {name: (dtype, array)} or a list of
    (name, dtype, array); the data streams out tensor by tensor."""
    ts = _tensor_list(tensors)
    head = header(metadata, [(n, d, a.shape, a.nbytes) for n, d, a in ts])
    full = os.path.abspath(path)
    temp = f"{full}.tmp-{uuid.uuid4().hex}"
    try:
        with open(temp, "wb") as f:
            f.write(head)
            for _, _, a in sorted(ts, key=lambda t: _code_point_key(t[0])):
                f.write(a.reshape(-1).view(np.uint8))
        os.replace(temp, full)
    finally:
        if os.path.exists(temp):
            os.remove(temp)
