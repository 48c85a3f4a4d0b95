"""Per-stage timing of the persistent decode step (decode_step_persistent) on a Qwen3-0.6B-shaped model.

    python -m rosylnalive_amd.build --stamps        # the timing variant, rosylnalive_amd/stamps/liblrm_hip.so
    python -m rosylnalive_amd.persist_stages [contexts]   # e.g. 392,4000 (the default)

The timing variant records constant-clock (100 MHz) stamps at the stage boundaries of one middle layer (and of the
next layer's stage A) in every workgroup, after the exchange entries. For each context: a prefill of that many tokens,
8 decode steps, then one measured step; printed per stage over the 256 workgroups: the median, max and min duration,
the time the last workgroup finished it (from the layer's first stamp), and the hand-off from the last producer of a
stage's input to the last consumer.
"""
from __future__ import annotations

import ctypes as C
import os
import struct
import sys

import numpy as np

from . import _native
from .build import STAMPS_LIB

STAGES = [  # name, first stamp, last stamp, attention workgroups only
    ("A gather (x, global)", 0, 1, False), ("A compute", 1, 2, False), ("B gather (q|k|v, local)", 2, 3, True),
    ("B attention", 3, 4, True), ("C gather (partials, local)", 5, 6, False), ("C combine + o_proj", 6, 8, False),
    ("D gather (p1, global)", 8, 9, False), ("D compute", 9, 10, False), ("E gather (a, local)", 10, 11, False),
    ("E compute", 11, 12, False)]
SUBSTAGES = [  # name, first point, last point (L k: stage boundary k; s k: point k inside a stage), attention only
    ("A norm", "L1", "s0", False), ("A rows", "s0", "s1", False), ("A barrier", "s1", "L2", False),
    ("B q/k norm", "L3", "s2", True), ("B rotate+append", "s2", "s3", True), ("B q to registers", "s3", "s4", True),
    ("B chunks", "s4", "s5", True), ("B partial rows", "s5", "L4", True),
    ("C gather 1", "L5", "s12", False), ("C gather 2", "s12", "s13", False), ("C split weights", "s13", "L6", False),
    ("C combine", "L6", "s6", False), ("C rows", "s6", "s7", False), ("C barrier", "s7", "L8", False),
    ("D issue W_down", "L9", "s8", False), ("D norm", "s8", "s9", False), ("D rows", "s9", "s10", False),
    ("D barrier", "s10", "L10", False), ("E rows", "L11", "s11", False), ("E barrier", "s11", "L12", False)]


def main(argv):
    contexts = [int(c) for c in (argv[0] if argv else "392,4000").split(",")]
    if not os.path.exists(STAMPS_LIB):
        raise SystemExit(f"{STAMPS_LIB} is missing: python -m rosylnalive_amd.build --stamps")
    _native.LIB_PATH = STAMPS_LIB  # before the first library call
    from .gpu_core import HipBackend
    from .qwen import QwenConfig, QwenModel, synthetic_ids, synthetic_weights

    cfg = QwenConfig.qwen3_0_6b(max_pos=(max(contexts) + 256 + 63) // 64 * 64)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fast", max_tokens=2048)
    m.load_weights(synthetic_weights(cfg, seed=1))
    if not m.persistent_decode():
        raise SystemExit("the persistent decode step is not in use on this device")
    for ctx in contexts:
        ids = synthetic_ids(1, "stamps", ctx, cfg.vocab)
        _, nxt = m.forward(ids, 0, logits_rows=1)
        m.decode_set(int(nxt), ctx)
        m.decode_run(8)
        tok = m.token("dec.exchange")
        table = C.create_string_buffer(1 << 20)
        _native.check(_native.lib().lrm_hip_download(b.handle, 0, 0, table, 1 << 20))
        row = struct.unpack_from("<16I", table.raw, tok * 64)
        slot, off, count = row[0], row[1], row[12]
        m.decode_run(1)
        nbytes = 256 * 64 * 8
        raw = C.create_string_buffer(nbytes)
        _native.check(_native.lib().lrm_hip_download(b.handle, slot, off + count * 4 - nbytes, raw, nbytes))
        st = np.frombuffer(raw.raw, np.uint64).reshape(256, 64).astype(np.int64)
        t0 = st[:, 40].min()
        L, L2 = st[:, 0:13], st[:, 16:29]
        attn = L[:, 3] > 0
        us = lambda v: v / 100.0
        print(f"context {ctx + 9}: step {us(st[0, 44] - t0):.1f} us; layers end {us(st[:, 41].max() - t0):.1f}; "
              f"lm_head x gathered {us(st[:, 42].max() - t0):.1f}; lm_head done {us(st[:, 43].max() - t0):.1f}; "
              f"attention workgroups {int(attn.sum())}")
        print(f"  hand-off, last producer to last consumer: B (q|k|v, local) {us(L[:, 3].max() - L[:, 2].max()):.2f} us;"
              f" C (partials, local) {us(L[:, 6].max() - L[attn, 4].max()):.2f}; D (p1, global) "
              f"{us(L[:, 9].max() - L[:, 8].max()):.2f}; E (a, local) {us(L[:, 11].max() - L[:, 10].max()):.2f}; "
              f"next A (p2, global) {us(L2[:, 1].max() - L[:, 12].max()):.2f}")
        lay0 = L[:, 0].min()
        print(f"  {'stage':28s} {'median':>7s} {'max':>7s} {'min':>7s} {'all done at':>12s}  (us)")
        for name, k0, k1, only_attn in STAGES:
            sel = attn if only_attn else slice(None)
            d = us(L[sel, k1] - L[sel, k0])
            print(f"  {name:28s} {np.median(d):7.2f} {d.max():7.2f} {d.min():7.2f} {us(L[sel, k1].max() - lay0):12.2f}")
        print(f"  layer (first start to last end) {us(L[:, 12].max() - lay0):.2f} us")
        P = st[:, 32:38]
        passes = [("A", P[:, 0]), ("B", P[attn, 1]), ("C", P[:, 2])]
        s_used = int(attn.sum()) // 8  # splits holding keys: the attention workgroups of one XCD
        if 2 * s_used * 33 > 3 * 512:  # the partial rows took a second gather
            passes.append(("C, second part", P[:, 3]))
        passes += [("D", P[:, 4]), ("E", P[:, 5])]
        print("  poll passes of thread 0 (median / max): " +
              "; ".join(f"{n} {np.median(v):.0f} / {v.max()}" for n, v in passes))
        Q = st[:, 48:62]
        pts = {f"s{k}": Q[:, k] for k in range(14)}
        pts.update({f"L{k}": L[:, k] for k in range(13)})
        parts = []
        for name, p0, p1, only_attn in SUBSTAGES:
            sel = attn if only_attn else slice(None)
            parts.append(f"{name} {np.median(us(pts[p1][sel] - pts[p0][sel])):.2f}")
        print("  inside the stages, thread 0, median us: " + "; ".join(parts), flush=True)
    m.close()
    b.close()


if __name__ == "__main__":
    main(sys.argv[1:])
