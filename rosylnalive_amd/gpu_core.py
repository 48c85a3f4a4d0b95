"""The reference's device abstraction (src/Lrm.Gpu.Core/Backend.fs:104-161) over liblrm_hip.so.

Names follow the reference: IGpuBackendProvider.Enumerate/Create -> HipBackendProvider.enumerate/create,
IGpuBackend -> HipBackend (create_heap, load_kernels, begin, submit, wait), IGpuHeap -> HipHeap (write_table, upload,
download), ICommandList -> HipCommandList (dispatch, barrier, copy, begin_timer, end_timer). Contract violations
raise GpuContractException from the same host-side checks the device runs (src/Lrm.Gpu.Core/Dispatch.fs:149-173).
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import _native as N
from ._native import Fp16RangeError, GpuContractException, HipDeviceError, LrmError, check, lib, u32s, u64s

__all__ = [
    "Fp16RangeError", "GpuContractException", "HipDeviceError", "LrmError", "Heap", "DType", "Arena", "TensorFlags", "Catalog",
    "KernelSpec", "ArgBlock", "HeapLayout", "HeapPlanner", "TensorTable", "SealedTable", "HipBackendProvider",
    "HipBackend", "HipHeap", "HipCommandList", "Submission", "Completion", "TimerResult", "prepare", "grid_physical",
]


class Heap:
    """HeapLayout.fs:149-175."""

    SLOT_COUNT = 64
    TABLE_SLOT = 0
    TABLE_ROWS = 16384
    ROW_BYTES = 64
    TABLE_BYTES = TABLE_ROWS * ROW_BYTES
    MAX_PAGE_BYTES = 1 << 30
    PAGE_GRANULARITY = 64 << 10
    ALLOCATION_ALIGNMENT = 256


class DType:
    """LrmCore DType codes (heap-and-tensor-table.md, TensorRow word 2)."""

    F32, BF16, F16, I32, U32, U8, F64, I64 = 1, 2, 3, 4, 5, 6, 7, 8
    SIZE = {1: 4, 2: 2, 3: 2, 4: 4, 5: 4, 6: 1, 7: 8, 8: 8}
    NAME = {1: "f32", 2: "bf16", 3: "f16", 4: "i32", 5: "u32", 6: "u8", 7: "f64", 8: "i64"}


class Arena:
    """Arena kinds with frozen codes (HeapLayout.fs:6-36)."""

    WEIGHTS, ROPE, KV_CACHE, ACTIVATIONS, SCRATCH, LOGITS, TAPS = 1, 2, 3, 4, 5, 6, 7
    MASTER, GRAD, ADAM_M, ADAM_V, ROSLYN_IN, ROSLYN_OUT = 8, 9, 10, 11, 12, 13


class TensorFlags:
    CONTIGUOUS, READ_ONLY, VIEW = 1, 2, 4


# ---------------------------------------------------------------- catalog and argument blocks

@dataclass
class FieldSpec:
    name: str
    kind: int  # 1 token, 2 u32, 3 i32, 4 f32
    access: int  # 0 none, 1 read, 2 write, 3 readwrite, 4 meta
    dtype_mask: int


@dataclass
class KernelSpec:
    id: int
    name: str
    threads: Tuple[int, int, int]
    linear: bool
    fields: List[FieldSpec]

    def field_index(self, name: str) -> int:
        for i, f in enumerate(self.fields):
            if f.name == name:
                return i
        raise KeyError(f"{self.name} has no field {name}")


class Catalog:
    """Kernels.all (src/Lrm.Gpu.Core/Kernels.g.fs:27-285): KernelId i is Catalog.all()[i]."""

    _all: Optional[List[KernelSpec]] = None

    @classmethod
    def all(cls) -> List[KernelSpec]:
        if cls._all is None:
            L = lib()
            specs = []
            for i in range(L.lrm_catalog_count()):
                name = C.create_string_buffer(64)
                thr = u32s([0, 0, 0])
                lin, nf = C.c_int(), C.c_int()
                check(L.lrm_catalog_kernel(i, name, 64, thr, C.byref(lin), C.byref(nf)))
                fields = []
                for f in range(nf.value):
                    fname = C.create_string_buffer(64)
                    kind, acc, mask = C.c_int(), C.c_int(), C.c_uint32()
                    check(L.lrm_catalog_field(i, f, fname, 64, C.byref(kind), C.byref(acc), C.byref(mask)))
                    fields.append(FieldSpec(fname.value.decode(), kind.value, acc.value, mask.value))
                specs.append(KernelSpec(i, name.value.decode(), (thr[0], thr[1], thr[2]), bool(lin.value), fields))
            cls._all = specs
        return cls._all

    @classmethod
    def find(cls, name: str) -> KernelSpec:
        for k in cls.all():
            if k.name == name:
                return k
        raise KeyError(f"no kernel {name} in the catalog")


def f32_bits(x: float) -> int:
    """ArgBlock.f32Bits (ArgBlock.fs:329-333): the raw IEEE bits, so -0, denormals and NaN payloads pass unchanged."""
    return struct.unpack("<I", struct.pack("<f", x))[0]


class ArgBlock:
    """The 128-byte argument block (ArgBlock.fs:240-325): word 0 = lrm_groups_x (written by Dispatch), field i at
    word i + 1, the rest 0."""

    WORD_COUNT = 32

    def __init__(self, words: Optional[Sequence[int]] = None):
        self.words = [0] * 32 if words is None else [int(w) & 0xFFFFFFFF for w in words]
        if len(self.words) != 32:
            raise ValueError("an argument block is 32 words")

    @classmethod
    def encode(cls, kernel: str, **fields) -> "ArgBlock":
        k = Catalog.find(kernel)
        b = cls()
        for name, v in fields.items():
            i = k.field_index(name)
            f = k.fields[i]
            if f.kind == 4:
                b.words[i + 1] = f32_bits(float(v))
            elif f.kind == 3:
                b.words[i + 1] = int(v) & 0xFFFFFFFF
            else:
                b.words[i + 1] = int(v)
        return b

    def as_c(self):
        return u32s(self.words)

    def __getitem__(self, i):
        return self.words[i]


ATTN_PREFILL_RECORD_WORDS = 64 + 2 * 8448


def attention_prefill_workspace_words(rows: int, kv_heads: int) -> int:
    """u32 words of attention_prefill_f16's workspace (rosylnalive_amd/csrc/attn_prefill.hpp): one record per
    (KV head, pair of 32-row tiles) = a counter padded to 64 words, then two partials of 8448 words, so launches of
    any length share one buffer. The counters (word 0 of each record) must be zero before the first launch; every
    launch leaves them zero."""
    return max(1, kv_heads * (((rows + 31) // 32) // 2)) * ATTN_PREFILL_RECORD_WORDS


def grid_physical(linear: bool, x: int, y: int, z: int) -> Tuple[int, int, int]:
    out = u32s([0, 0, 0])
    check(lib().lrm_grid_physical(int(linear), x, y, z, out))
    return out[0], out[1], out[2]


# ---------------------------------------------------------------- heap layout, planner, table

@dataclass
class Page:
    slot: int
    arena: int
    index: int
    bytes: int


@dataclass
class HeapLayout:
    """HeapLayout.ofPages (HeapLayout.fs:302-420): pages in slots 1..N in contract order."""

    pages: List[Page] = field(default_factory=list)

    @classmethod
    def of_pages(cls, kinds_and_bytes: Sequence[Tuple[int, int]]) -> "HeapLayout":
        # validated by the library on use (create_heap / table creation); the indices are assigned here
        per: Dict[int, int] = {}
        pages = []
        for i, (k, b) in enumerate(kinds_and_bytes):
            pages.append(Page(i + 1, k, per.get(k, 0), b))
            per[k] = per.get(k, 0) + 1
        return cls(pages)

    def arrays(self):
        return u32s([p.arena for p in self.pages]), u64s([p.bytes for p in self.pages]), len(self.pages)

    def slot_of(self, arena: int, index: int) -> int:
        for p in self.pages:
            if p.arena == arena and p.index == index:
                return p.slot
        raise GpuContractException(N.LRM_E_CONTRACT, f"arena {arena} has no page {index}")


class HeapPlanner:
    """Pass one of a static plan (HeapLayout.fs:433-525)."""

    def __init__(self, page_bytes: int = Heap.MAX_PAGE_BYTES):
        self._h = C.c_void_p()
        check(lib().lrm_planner_create(page_bytes, C.byref(self._h)))

    def allocate(self, arena: int, nbytes: int) -> Tuple[int, int, int, int]:
        page, off = C.c_int32(), C.c_uint64()
        check(lib().lrm_planner_allocate(self._h, arena, nbytes, C.byref(page), C.byref(off)))
        return (arena, page.value, off.value, nbytes)

    def build(self) -> HeapLayout:
        arenas, sizes, n = u32s([0] * 63), u64s([0] * 63), C.c_int()
        check(lib().lrm_planner_build(self._h, arenas, sizes, 63, C.byref(n)))
        return HeapLayout.of_pages([(arenas[i], sizes[i]) for i in range(n.value)])

    def __del__(self):
        if getattr(self, "_h", None):
            lib().lrm_planner_destroy(self._h)
            self._h = None


class SealedTable:
    """The 1 MiB table image (TensorTable.fs:321-376)."""

    def __init__(self, layout: HeapLayout, image: bytes, names: Dict[str, int]):
        self.layout = layout
        self.image = image
        self.names = names

    def row(self, token: int) -> List[int]:
        if token >= Heap.TABLE_ROWS:
            raise GpuContractException(N.LRM_E_CONTRACT, f"token {token} is not below 16,384")
        return list(struct.unpack_from("<16I", self.image, token * Heap.ROW_BYTES))


class TensorTable:
    """Pass two of a static plan (TensorTable.fs:378-474): tokens 1, 2, ... then Seal once."""

    def __init__(self, layout: HeapLayout):
        self.layout = layout
        self._h = C.c_void_p()
        a, b, n = layout.arrays()
        check(lib().lrm_table_create(a, b, n, C.byref(self._h)))
        self.names: Dict[str, int] = {}

    def add(self, name: str, slot: int, byte_offset: int, dtype: int, dims: Sequence[int], flags: int = 0) -> int:
        tok = C.c_uint32()
        check(lib().lrm_table_add(self._h, name.encode(), slot, byte_offset, dtype, u32s(dims), len(dims), flags,
                                  C.byref(tok)))
        self.names[name] = tok.value
        return tok.value

    def add_placed(self, name: str, placement, dtype: int, dims: Sequence[int], flags: int = 0) -> int:
        arena, page, off, _ = placement
        return self.add(name, self.layout.slot_of(arena, page), off, dtype, dims, flags)

    def add_view(self, name: str, source: int, dims: Sequence[int], element_offset: int) -> int:
        tok = C.c_uint32()
        check(lib().lrm_table_add_view(self._h, name.encode(), source, u32s(dims), len(dims), element_offset,
                                       C.byref(tok)))
        self.names[name] = tok.value
        return tok.value

    def seal(self) -> SealedTable:
        buf = C.create_string_buffer(Heap.TABLE_BYTES)
        check(lib().lrm_table_seal(self._h, buf))
        return SealedTable(self.layout, buf.raw, dict(self.names))

    def __del__(self):
        if getattr(self, "_h", None):
            lib().lrm_table_destroy(self._h)
            self._h = None


def prepare(table: SealedTable, kernel: int, args: ArgBlock):
    """Dispatch.prepare: returns (words as dispatched, logical grid, physical grid)."""
    out = u32s([0] * 32)
    grid = (C.c_int64 * 3)()
    phys = u32s([0, 0, 0])
    a, b, n = table.layout.arrays()
    buf = C.create_string_buffer(table.image, Heap.TABLE_BYTES)
    check(lib().lrm_prepare(buf, a, b, n, kernel, args.as_c(), out, grid, phys))
    return list(out), (grid[0], grid[1], grid[2]), (phys[0], phys[1], phys[2])


# ---------------------------------------------------------------- the device

@dataclass
class HipDeviceInfo:
    index: int
    name: str
    arch: str
    vendor_id: int
    pci_device_id: int
    pci_bus: str
    driver: str
    memory_bytes: int
    compute_units: int

    @property
    def device_id(self) -> str:
        """GpuClass DeviceId form (gpu-backend.md 'The GPU fill rule'): pci:<vendor>:<device>."""
        return "pci:%04x:%04x" % (self.vendor_id, self.pci_device_id)


def _info(s: N.DeviceInfo) -> HipDeviceInfo:
    return HipDeviceInfo(s.index, s.name.decode(), s.arch.decode(), s.vendor_id, s.pci_device_id, s.pci_bus.decode(),
                         s.driver.decode(), s.memory_bytes, s.compute_units)


@dataclass
class DeviceCandidate:
    info: HipDeviceInfo
    rejections: List[str]

    @property
    def accepted(self) -> bool:
        return not self.rejections


class HipBackendProvider:
    """IGpuBackendProvider for the new "hip" ExecutionBackend (Backend.fs:156-161)."""

    backend = "hip"

    @staticmethod
    def enumerate() -> List[DeviceCandidate]:
        n = C.c_int()
        check(lib().lrm_hip_enumerate(None, 0, C.byref(n)))
        arr = (N.DeviceInfo * max(1, n.value))()
        check(lib().lrm_hip_enumerate(arr, n.value, C.byref(n)))
        out = []
        for i in range(n.value):
            info = _info(arr[i])
            rej = [] if info.arch.split(":")[0] == "gfx950" else [f"requires gfx950 (found {info.arch})"]
            out.append(DeviceCandidate(info, rej))
        return out

    @staticmethod
    def create(index: int = 0, time_dispatches: bool = False) -> "HipBackend":
        return HipBackend(index, time_dispatches)


@dataclass
class TimerResult:
    name: str
    gpu_start_ns: int
    duration_ns: int


@dataclass
class Completion:
    submission: int
    dispatches: int
    timers: List[TimerResult]


class Submission(int):
    pass


class HipBackend:
    """IGpuBackend on one gfx950 device (Backend.fs:139-153)."""

    def __init__(self, index: int = 0, time_dispatches: bool = False):
        self._h = C.c_void_p()
        check(lib().lrm_hip_create(index, 1 if time_dispatches else 0, C.byref(self._h)))
        s = N.DeviceInfo()
        check(lib().lrm_hip_info(self._h, C.byref(s)))
        self.info = _info(s)
        self.heap: Optional[HipHeap] = None
        self.shader_set_hash: Optional[bytes] = None

    @classmethod
    def _wrap(cls, handle) -> "HipBackend":
        b = cls.__new__(cls)
        b._h = C.c_void_p(handle)
        s = N.DeviceInfo()
        check(lib().lrm_hip_info(b._h, C.byref(s)))
        b.info = _info(s)
        b.heap = None
        b.shader_set_hash = None
        b._borrowed = True
        return b

    @property
    def handle(self):
        return self._h

    def create_heap(self, layout: HeapLayout) -> "HipHeap":
        a, b, n = layout.arrays()
        check(lib().lrm_hip_create_heap(self._h, a, b, n))
        self.heap = HipHeap(self, layout)
        return self.heap

    KERNEL_SETS = {"reference": 0, "fast": 1}

    def load_kernels(self, kernel_set: str = "reference") -> bytes:
        """LoadKernels, once per backend: "reference" (catalog ids 0-13, the BatchInvariance contract) or "fast"
        (every id, its own ExecutionClass: same work, same inputs, same bits, and no more). Returns the set's
        shader-set hash."""
        h = C.create_string_buffer(32)
        check(lib().lrm_hip_load_kernel_set(self._h, self.KERNEL_SETS[kernel_set], h))
        self.shader_set_hash = h.raw
        return h.raw

    def contains(self, kernel: int) -> bool:
        return bool(lib().lrm_hip_contains(self._h, kernel))

    def denormal_probe(self) -> Tuple[str, List[int]]:
        mode = C.c_int()
        res = u32s([0] * 7)
        check(lib().lrm_hip_denormal_probe(self._h, C.byref(mode), res))
        return {1: "preserve", 2: "flush", 3: "mixed"}.get(mode.value, "unknown"), list(res)

    def begin(self, reusable: bool = False) -> "HipCommandList":
        l = C.c_void_p()
        check(lib().lrm_hip_begin(self._h, 1 if reusable else 0, C.byref(l)))
        return HipCommandList(self, l, reusable)

    def submit(self, commands: "HipCommandList", repeat: int = 1) -> Submission:
        f = C.c_uint64()
        check(lib().lrm_hip_submit(self._h, commands._h, repeat, C.byref(f)))
        return Submission(f.value)

    def wait(self, submission: int) -> Completion:
        nd, nt = C.c_int(), C.c_int()
        check(lib().lrm_hip_wait(self._h, int(submission), C.byref(nd), C.byref(nt)))
        timers = []
        for i in range(nt.value):
            name = C.create_string_buffer(128)
            st, du = C.c_int64(), C.c_int64()
            check(lib().lrm_hip_timer(self._h, int(submission), i, name, 128, C.byref(st), C.byref(du)))
            timers.append(TimerResult(name.value.decode(), st.value, du.value))
        return Completion(int(submission), nd.value, timers)

    def close(self):
        if getattr(self, "_h", None) and not getattr(self, "_borrowed", False):
            check(lib().lrm_hip_destroy(self._h))
        self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


class HipHeap:
    """IGpuHeap (Backend.fs:111-122)."""

    def __init__(self, backend: HipBackend, layout: HeapLayout):
        self.backend = backend
        self.layout = layout
        self.table: Optional[SealedTable] = None

    def write_table(self, table: SealedTable) -> None:
        buf = C.create_string_buffer(table.image, Heap.TABLE_BYTES)
        check(lib().lrm_hip_write_table(self.backend._h, buf, Heap.TABLE_BYTES))
        self.table = table

    def upload(self, slot: int, offset: int, data) -> None:
        arr = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data)
        check(lib().lrm_hip_upload(self.backend._h, slot, offset, arr.ctypes.data, arr.nbytes))

    def download(self, slot: int, offset: int, nbytes: int) -> bytes:
        buf = C.create_string_buffer(nbytes)
        check(lib().lrm_hip_download(self.backend._h, slot, offset, buf, nbytes))
        return buf.raw


class HipCommandList:
    """ICommandList (Backend.fs:125-136)."""

    def __init__(self, backend: HipBackend, handle, reusable: bool):
        self.backend = backend
        self._h = handle
        self.reusable = reusable

    def dispatch(self, kernel, args: ArgBlock) -> None:
        kid = Catalog.find(kernel).id if isinstance(kernel, str) else int(kernel)
        check(lib().lrm_hip_dispatch(self._h, kid, args.as_c()))

    def dispatch_overlapped(self, kernel, args: ArgBlock) -> None:
        """A dispatch that may run concurrently with the following ones up to the next barrier (side stream)."""
        kid = Catalog.find(kernel).id if isinstance(kernel, str) else int(kernel)
        check(lib().lrm_hip_dispatch_overlapped(self._h, kid, args.as_c()))

    def dispatch_decode_attention_static(self, args: ArgBlock, y: int) -> None:
        """attention_decode_f16 (args, partials token 0) then attention_combine into the f32 tensor y, the split
        partials in the library's static scratch: nothing is allocated (no counterpart in the reference)."""
        check(lib().lrm_hip_dispatch_decode_attention_static(self._h, args.as_c(), int(y)))

    def barrier(self) -> None:
        check(lib().lrm_hip_barrier(self._h))

    def copy(self, source: Tuple[int, int, int], destination: Tuple[int, int, int]) -> None:
        (ss, so, sb), (ds, do, db) = source, destination
        if sb != db:
            raise GpuContractException(N.LRM_E_CONTRACT, "copy ranges must have equal sizes")
        check(lib().lrm_hip_copy(self._h, ss, so, ds, do, sb))

    def begin_timer(self, name: str) -> int:
        t = C.c_int()
        check(lib().lrm_hip_begin_timer(self._h, name.encode(), C.byref(t)))
        return t.value

    def end_timer(self, timer: int) -> None:
        check(lib().lrm_hip_end_timer(self._h, timer))

    def release(self) -> None:
        if self._h:
            check(lib().lrm_hip_release(self.backend._h, self._h))
            self._h = None
