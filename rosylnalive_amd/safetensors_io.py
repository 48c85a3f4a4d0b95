"""A small validating safetensors reader/writer that keeps bf16 as raw uint16 bits.

The reference reads checkpoints and goldens through its own validating reader (src/Lrm.Tensor/Safetensors.fs:504-727):
an 8-byte little-endian header length, a JSON header of {name: {dtype, shape, data_offsets}} plus an optional
"__metadata__" entry, then the raw little-endian data. bf16 tensors stay as their bits (HostTensor<uint16>), which is
what the kernels consume. numpy has no bfloat16, so BF16 maps to uint16 here.
"""
from __future__ import annotations

import json
import struct
from typing import Dict, Tuple

import numpy as np

_DTYPES = {
    "F64": np.float64,
    "F32": np.float32,
    "F16": np.float16,
    "BF16": np.uint16,  # raw bits
    "I64": np.int64,
    "I32": np.int32,
    "U32": np.uint32,
    "I16": np.int16,
    "U16": np.uint16,
    "I8": np.int8,
    "U8": np.uint8,
    "BOOL": np.bool_,
}


def read_header(path: str) -> Tuple[dict, int]:
    """Returns (header, data_start). Raises ValueError on a malformed file."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: shorter than the 8-byte header length")
        (n,) = struct.unpack("<Q", raw)
        if n > 100 * 1024 * 1024:
            raise ValueError(f"{path}: header of {n} bytes")
        header = json.loads(f.read(n).decode("utf-8"))
    return header, 8 + n


def load(path: str) -> Dict[str, np.ndarray]:
    """Every tensor of a file as numpy arrays (BF16 as uint16 bits), checking offsets against the data size."""
    header, start = read_header(path)
    with open(path, "rb") as f:
        f.seek(start)
        data = f.read()
    out: Dict[str, np.ndarray] = {}
    for name, e in header.items():
        if name == "__metadata__":
            continue
        dt = _DTYPES.get(e["dtype"])
        if dt is None:
            raise ValueError(f"{path}: {name} has unsupported dtype {e['dtype']}")
        lo, hi = e["data_offsets"]
        shape = tuple(int(s) for s in e["shape"])
        count = int(np.prod(shape)) if shape else 1
        if not (0 <= lo <= hi <= len(data)) or hi - lo != count * np.dtype(dt).itemsize:
            raise ValueError(f"{path}: {name} offsets {lo}..{hi} do not hold {shape} {e['dtype']}")
        out[name] = np.frombuffer(data[lo:hi], dtype=dt).reshape(shape).copy()
    return out


def save(path: str, tensors: Dict[str, Tuple[str, np.ndarray]]) -> None:
    """Writes {name: (dtype_code, array)} in name order, data 8-byte aligned as the format expects."""
    header = {}
    blobs = []
    offset = 0
    for name in sorted(tensors):
        code, arr = tensors[name]
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": code, "shape": list(arr.shape), "data_offsets": [offset, offset + len(b)]}
        blobs.append(b)
        offset += len(b)
    hj = json.dumps(header, separators=(",", ":")).encode("utf-8")
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)
