"""Per-workgroup timing of the prefill GEMMs (the direct-to-LDS loop), from the stage-timing build.

    python -m rosylnalive_amd.build --stamps           # on the build host: rosylnalive_amd/stamps/liblrm_hip.so
    python -m rosylnalive_amd.gemm_stages [T]          # GPU box, repository root (T: prompt tokens, default 2048)

Runs the Qwen3-0.6B-shaped fast forward of T synthetic tokens (random N(0, 0.02) weights) three times and reads the
stamps of the last launch of each GEMM kind (layer 27's: the q|k|v GEMM with its norm / RoPE / cache epilogue, gate/up
with SwiGLU, and down_proj's k-split partials). Thread 0 of every workgroup stamps its start, the moment each k tile
has landed in LDS (after the step's wait and barrier), the main loop's end and the epilogue's end (100 MHz constant
clock), and in the q|k|v epilogue of the q and k head tiles four points between (past the barrier that ends the main
loop; the cos / sin and norm weight loads issued; the tile staged in LDS; the rows read back and their squares
summed). Printed per kernel: the launch's span, and over its workgroups the start offset, the time to the first tile,
the k steps, the epilogue and the end offset, plus the median time of every k step.
"""
import ctypes as C
import os
import sys

import numpy as np

from . import _native
from .build import STAMPS_LIB

KINDS = {3: "q|k|v GEMM + q/k norm, RoPE, cache epilogue", 2: "gate/up GEMM + SwiGLU",
         4: "down_proj k-split partials"}
WORDS = 32


def read(backend, kind, blocks):
    buf = np.zeros(blocks * WORDS, np.uint64)
    _native.check(_native.lib().lrm_hip_debug_gemm_stamps(backend.handle, kind, buf.ctypes.data_as(C.c_void_p),
                                                          buf.size))
    return buf.reshape(blocks, WORDS).astype(np.int64)


def summarize(name, st):
    used = st[:, 1] > 0
    st = st[used]
    t0 = st[:, 1].min()
    us = lambda v: v / 100.0
    # k steps recorded: words 2 .. 2 + n - 1 (the same n for every block of a launch, at most 24)
    nk = int(np.max(np.sum(st[:, 2:26] > 0, axis=1)))
    landed = st[:, 2:2 + nk]
    start, first, loop_end, end = st[:, 1], landed[:, 0], st[:, 30], st[:, 31]
    steps = np.diff(landed, axis=1)  # tile kt landed -> tile kt + 1 landed: one step of MFMAs plus the wait
    last = loop_end - landed[:, -1]  # the last tile's MFMAs
    cu = (st[:, 0] >> 32) * 1000 + (st[:, 0] & 0xFFFFFFFF)
    _, per_cu = np.unique(cu, return_counts=True)
    rows = [("start offset", start - t0), ("start -> first tile landed", first - start),
            ("k step (mean per block)", steps.mean(axis=1) if steps.size else np.zeros(len(st))),
            ("last tile's MFMAs", last), ("epilogue", end - loop_end), ("block total", end - start),
            ("end offset", end - t0)]
    inner = (st[:, 26] > 0) & (st[:, 27] > 0)  # the q|k|v epilogue's points (q and k head tiles)
    if inner.any():
        e = st[inner]
        rows[5:5] = [("  epilogue: end-of-loop barrier", e[:, 28] - e[:, 30]),
                     ("  epilogue: issue table loads", e[:, 29] - e[:, 28]),
                     ("  epilogue: tile to LDS", e[:, 26] - e[:, 29]), ("  epilogue: rows back, sums", e[:, 27] - e[:, 26]),
                     ("  epilogue: norm, RoPE, stores", e[:, 31] - e[:, 27])]
    print(f"{name}: {len(st)} workgroups, {nk} k steps each, {len(per_cu)} distinct CUs "
          f"(workgroups per CU: {np.bincount(per_cu).nonzero()[0].tolist()}), launch span {us(end.max() - t0):.2f} us")
    print(f"  {'':28s} {'median':>8s} {'p10':>8s} {'p90':>8s} {'max':>8s}  (us)")
    for label, v in rows:
        v = us(v.astype(np.float64))
        print(f"  {label:28s} {np.median(v):8.2f} {np.percentile(v, 10):8.2f} {np.percentile(v, 90):8.2f} "
              f"{v.max():8.2f}")
    if steps.size:
        med = np.median(us(steps.astype(np.float64)), axis=0)
        print("  median k step by index (us): " + " ".join(f"{x:.2f}" for x in med), flush=True)


def main(argv):
    T = int(argv[0]) if argv else 2048
    if not os.path.exists(STAMPS_LIB):
        raise SystemExit(f"{STAMPS_LIB} is missing: python -m rosylnalive_amd.build --stamps")
    _native.LIB_PATH = STAMPS_LIB  # before the first library call
    from .gpu_core import HipBackend
    from .qwen import QwenConfig, QwenModel, synthetic_ids, synthetic_weights

    cfg = QwenConfig.qwen3_0_6b(max_pos=(T + 63) // 64 * 64)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fast", max_tokens=T)
    m.load_weights(synthetic_weights(cfg, seed=1))
    ids = synthetic_ids(1, "gemm-stamps", T, cfg.vocab)
    for _ in range(3):
        m.forward(ids, 0, logits_rows=1)
    print(f"Qwen3-0.6B shape, {T}-token forward: {m.last_ms():.3f} ms (stage-timing build)", flush=True)
    for kind, name in KINDS.items():
        summarize(name, read(b, kind, 4096))
    m.close()
    b.close()


if __name__ == "__main__":
    main(sys.argv[1:])
