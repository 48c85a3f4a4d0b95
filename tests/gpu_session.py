"""A small conformance session for GPU tests, after the reference's harness (tests/Lrm.Kernels.Conformance/Harness/
Session.fs:144-956, Poison.fs:11-56): every tensor of a case gets its own planner placement, outputs are poisoned
with a NaN pattern no arithmetic produces, each case runs twice, and results must be bit-identical between runs.
"""
from __future__ import annotations

import numpy as np

from rosylnalive_amd.gpu_core import Arena, ArgBlock, Catalog, DType, HeapPlanner, HipBackend, TensorFlags, TensorTable

POISON_F32 = 0x7FA5A5A5  # a signalling NaN: arithmetic never produces it
POISON_16 = 0x7FA5
NP = {DType.F32: np.float32, DType.BF16: np.uint16, DType.F16: np.uint16, DType.U32: np.uint32, DType.I32: np.int32}


class Session:
    def __init__(self, tensors: dict, backend: HipBackend = None):
        """tensors: name -> (dtype, shape, flags, initial ndarray or None)."""
        self.backend = backend or HipBackend(0)
        self.backend.load_kernels("fast")  # every id: the cases dispatch catalog and fast kernels alike
        planner = HeapPlanner()
        self.spec = tensors
        places = {}
        for name, (dt, shape, flags, _) in tensors.items():
            n = int(np.prod(shape))
            places[name] = planner.allocate(Arena.ACTIVATIONS, max(4, (n * DType.SIZE[dt] + 3) // 4 * 4))
        layout = planner.build()
        self.heap = self.backend.create_heap(layout)
        table = TensorTable(layout)
        self.tok = {}
        for name, (dt, shape, flags, _) in tensors.items():
            self.tok[name] = table.add_placed(name, places[name], dt, list(shape), flags)
        self.table = table.seal()
        self.heap.write_table(self.table)
        self.rows = {n: self.table.row(t) for n, t in self.tok.items()}
        for name, (dt, shape, flags, init) in tensors.items():
            self.write(name, init if init is not None else self.poison(name))

    def poison(self, name):
        dt, shape, _, _ = self.spec[name]
        if DType.SIZE[dt] == 4:
            return np.full(shape, POISON_F32, np.uint32)
        return np.full(shape, POISON_16, np.uint16)

    def write(self, name, arr):
        """Uploads whole u32 words: an odd-length bf16 tensor owns its last word (the extent is rounded up to 4)."""
        r = self.rows[name]
        b = np.ascontiguousarray(arr).view(np.uint8).ravel()
        if b.size % 4:
            b = np.concatenate([b, np.zeros(4 - b.size % 4, np.uint8)])
        self.heap.upload(r[0], r[1], b)

    def read(self, name):
        dt, shape, _, _ = self.spec[name]
        r = self.rows[name]
        n = int(np.prod(shape)) * DType.SIZE[dt]
        return np.frombuffer(self.heap.download(r[0], r[1], (n + 3) // 4 * 4)[:n], NP[dt]).reshape(shape).copy()

    def fields(self, kernel: str, **fields):
        """The ArgBlock of one dispatch, tensor names resolved to their tokens."""
        return ArgBlock.encode(kernel, **{k: (self.tok[v] if isinstance(v, str) else v) for k, v in fields.items()})

    def run_list(self, dispatches, outputs, reset=None):
        """Dispatches [(kernel, fields), ...] in one command list, twice, with the outputs re-poisoned and the tensors
        of `reset` (name -> array) rewritten; returns the outputs of the second run after checking both runs gave the
        same bits."""
        results = []
        for _ in range(2):
            for name, arr in (reset or {}).items():
                self.write(name, arr)
            for o in outputs:
                self.write(o, self.poison(o))
            cl = self.backend.begin()
            for kernel, f in dispatches:
                cl.dispatch(kernel, self.fields(kernel, **f))
            c = self.backend.wait(self.backend.submit(cl))
            cl.release()
            assert c.dispatches == len(dispatches)
            results.append({o: self.read(o) for o in outputs})
        for o in outputs:
            assert results[0][o].tobytes() == results[1][o].tobytes(), f"{o} differs between two runs"
        return results[1]

    def run(self, kernel: str, outputs, **fields):
        """Dispatches once per run, twice, with the outputs re-poisoned; returns the outputs of the second run after
        checking both runs gave the same bits."""
        args = {k: (self.tok[v] if isinstance(v, str) else v) for k, v in fields.items()}
        results = []
        for _ in range(2):
            for o in outputs:
                self.write(o, self.poison(o))
            cl = self.backend.begin()
            cl.dispatch(kernel, ArgBlock.encode(kernel, **args))
            c = self.backend.wait(self.backend.submit(cl))
            cl.release()
            assert c.dispatches == 1
            results.append({o: self.read(o) for o in outputs})
        for o in outputs:
            assert results[0][o].tobytes() == results[1][o].tobytes(), f"{kernel}: {o} differs between two runs"
        return results[1]

    def close(self):
        self.backend.close()


def written_everywhere(a: np.ndarray) -> bool:
    """No element still holds the poison pattern."""
    u = a.view(np.uint32) if a.dtype.itemsize == 4 else a.view(np.uint16)
    return not np.any(u == (POISON_F32 if a.dtype.itemsize == 4 else POISON_16))
