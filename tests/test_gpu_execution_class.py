"""The two kernel sets and the bit-identity claims of each (docs/contracts/batch-invariance.md:7-12 in the reference;
bit-identity is scoped to one ExecutionClass, src/Lrm.Core/ExecutionClass.fs:58).

- The reference set (catalog ids 0-13, what LoadKernels loads, the executor's fp32 mode) keeps the BatchInvariance
  contract: a row computed alone equals the same row inside any batch (matmul rows at M = 1 equal the rows at M = 37,
  512 and 4000, tests/Lrm.Kernels.Conformance/Cases/matmul/MatmulCases.fs:1-20,173-198), and prefill equals decode
  equals chunked prefill, here on the full Qwen3-0.6B shape across a 64-key block boundary.
- The fast set (every id, the executor's fast mode) has its own shader-set hash, so no bit-identity claim crosses the
  two sets; it claims only that the same work on the same inputs gives the same bits: a repeated prefill and a
  repeated persistent decode step give identical logits.
"""
import numpy as np
import pytest

from gpu_session import Session, written_everywhere
from oracle import cpuref, metrics
from rosylnalive_amd.gpu_core import DType, HipBackend, TensorFlags
from rosylnalive_amd._native import LrmError
from rosylnalive_amd.qwen import QwenConfig, QwenModel, synthetic_ids, synthetic_weights

pytestmark = pytest.mark.gpu

F32, BF16, F16 = DType.F32, DType.BF16, DType.F16
RO = TensorFlags.READ_ONLY


def test_each_kernel_set_is_its_own_execution_class():
    """LoadKernels gives the reference set (ids 0-13) under one shader-set hash, the fast set (ids 0-40) under
    another; the fast executor mode refuses a device holding the reference set."""
    ref, fast = HipBackend(0), HipBackend(0)
    try:
        h_ref, h_fast = ref.load_kernels(), fast.load_kernels("fast")
        assert len(h_ref) == 32 and len(h_fast) == 32 and h_ref != h_fast
        assert all(ref.contains(k) for k in range(14)) and not any(ref.contains(k) for k in range(14, 41))
        assert all(fast.contains(k) for k in range(41))
        with pytest.raises(LrmError, match="fast kernel set"):
            QwenModel(ref, QwenConfig(1, 1024, 16, 8, 128, 3072, 4096, 128), mode="fast", max_tokens=64)
    finally:
        ref.close()
        fast.close()
    # a second device of the same library reports the same hashes
    again = HipBackend(0)
    try:
        assert again.load_kernels("fast") == h_fast
    finally:
        again.close()


def test_reference_matmul_rows_equal_alone_and_in_batches_of_37_512_4000():
    """matmul_bf16w at M = 4000 (n 1024, k 1024): the first 37 and 512 rows equal the M = 37 and M = 512 results bit
    for bit, rows 0, 36, 511, 2048 and 3999 computed alone (M = 1) equal their rows in the batch, and those rows equal
    CpuRef F32 (the oracle's sequential fused chain) bit for bit."""
    m, n, k = 4000, 1024, 1024
    r = np.random.default_rng(4000)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = cpuref.bf16_narrow(r.standard_normal((n, k)) * 0.05)
    s = Session({"x": (F32, x.shape, 0, x), "w": (BF16, w.shape, RO, w), "y": (F32, (m, n), 0, None),
                 "x1": (F32, (1, k), 0, None), "y1": (F32, (1, n), 0, None)})
    try:
        y = s.run("matmul_bf16w", ["y"], x="x", w="w", y="y", m=m, n=n, k=k)["y"]
        assert written_everywhere(y)
        for mm in (37, 512):
            ym = s.run("matmul_bf16w", ["y"], x="x", w="w", y="y", m=mm, n=n, k=k)["y"][:mm]
            assert ym.tobytes() == y[:mm].tobytes(), mm
        rows = [0, 36, 511, 2048, 3999]
        for i in rows:
            s.write("x1", x[i:i + 1])
            y1 = s.run("matmul_bf16w", ["y1"], x="x1", w="w", y="y1", m=1, n=n, k=k)["y1"]
            assert y1.tobytes() == y[i:i + 1].tobytes(), i
        assert cpuref.matmul_bf16w(x[rows], w).tobytes() == y[rows].tobytes()
    finally:
        s.close()


def test_fp32_mode_prefill_equals_decode_equals_chunked_on_the_0_6b_shape():
    """The executor's fp32 mode (the reference set) on the full Qwen3-0.6B shape (28 layers, 16/8 heads of 128,
    SwiGLU 3072, vocab 151,936), 80 tokens: one 80-row prefill, a 37 + 43 chunked prefill, and a 60-row prefill then
    20 single-token decode steps (positions 60..79, across the 64-key block boundary): every logits row is the same
    bits in all three schedules (batch-invariance.md:10-12, the M2 and X1 obligations at the real shape)."""
    cfg = QwenConfig.qwen3_0_6b(max_pos=128)
    w = synthetic_weights(cfg, seed=51)
    ids = synthetic_ids(51, "class/fp32", 80, cfg.vocab)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fp32", max_tokens=80)
    try:
        m.load_weights(w)
        whole, _ = m.forward(ids, 0, logits_rows=80)
        assert np.isfinite(whole).all()
        c1, _ = m.forward(ids[:37], 0, logits_rows=37)
        c2, _ = m.forward(ids[37:], 37, logits_rows=43)
        chunked = np.concatenate([c1, c2])
        p, _ = m.forward(ids[:60], 0, logits_rows=60)
        steps = [m.forward(ids[t:t + 1], t, logits_rows=1)[0] for t in range(60, 80)]
        decoded = np.concatenate([p] + steps)
    finally:
        m.close()
        b.close()
    diff_c = int(np.sum(np.any(chunked.view(np.uint32) != whole.view(np.uint32), axis=1)))
    diff_d = int(np.sum(np.any(decoded.view(np.uint32) != whole.view(np.uint32), axis=1)))
    print(f"fp32 mode, 0.6B shape, 80 tokens: rows differing from the whole prefill: chunked {diff_c}, prefill + "
          f"decode {diff_d}", flush=True)
    assert chunked.tobytes() == whole.tobytes()
    assert decoded.tobytes() == whole.tobytes()


def test_fast_mode_repeats_its_bits():
    """The fast set's one claim, on the full Qwen3-0.6B shape: the same 600-token prefill twice gives the same logits
    bits (its last 8 rows), and the same 6 persistent decode steps from the same state twice give the same ids and
    the same logits bits."""
    cfg = QwenConfig.qwen3_0_6b(max_pos=1024)
    w = synthetic_weights(cfg, seed=52)
    ids = synthetic_ids(52, "class/fast", 600, cfg.vocab)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fast", max_tokens=1024)
    try:
        m.load_weights(w)
        runs = []
        for _ in range(2):
            lg, nxt = m.forward(ids, 0, logits_rows=8)
            m.decode_set(int(nxt), 600)
            rows = []
            for _s in range(6):
                m.decode_run(1)
                rows.append(m.read_logits(1)[0])
            runs.append((lg, nxt, np.stack(rows), m.decode_ids(6)))
    finally:
        m.close()
        b.close()
    (l0, n0, d0, i0), (l1, n1, d1, i1) = runs
    assert np.isfinite(l0).all() and np.isfinite(d0).all()
    assert l0.tobytes() == l1.tobytes() and n0 == n1
    assert d0.tobytes() == d1.tobytes() and i0.tolist() == i1.tolist()
    assert metrics.max_abs(d0, d1) == 0.0
