"""GPU tests of the HIP device through the C ABI: provider, heap, table, command lists, the selftest kernels and every
reference catalog kernel (ids 0..13) against the oracle with the reference's KernelBounds
(src/Lrm.Tensor/KernelBounds.fs: bit-exact kernels compare bits; relative kernels relL2(gpu, CpuRef64) <=
max(1e-6, 2 relL2(CpuRef32, CpuRef64))). Every case runs twice with poisoned outputs and must repeat its bits.
"""
import struct

import numpy as np
import pytest

from gpu_session import Session, written_everywhere
from oracle import cpuref, metrics
from rosylnalive_amd.gpu_core import (ArgBlock, DType, GpuContractException, HeapLayout, HipBackend,
                                      HipBackendProvider, TensorFlags, TensorTable)
from rosylnalive_amd.qwen import QWEN3_INV_FREQ_HD128

pytestmark = pytest.mark.gpu

F32, BF16, U32 = DType.F32, DType.BF16, DType.U32
RO = TensorFlags.READ_ONLY


def rng(seed):
    return np.random.default_rng(seed)


def bf16(a):
    return cpuref.bf16_narrow(np.asarray(a, np.float32))


def check_relative(gpu, ref32, ref64, what):
    r = metrics.check_relative(gpu, ref32, ref64)
    assert r["passed"], (what, r)
    return r


# ---------------------------------------------------------------- provider, heap, selftests


def test_provider_enumerates_gfx950():
    cands = HipBackendProvider.enumerate()
    print("devices:", [(c.info.name, c.info.arch, c.info.device_id, c.info.compute_units) for c in cands], flush=True)
    assert cands and cands[0].accepted, cands
    assert cands[0].info.vendor_id == 0x1002 and cands[0].info.memory_bytes > 100 << 30


def test_once_only_rules_and_denormal_probe():
    b = HipBackend(0)
    try:
        h = b.load_kernels()
        assert len(h) == 32 and any(h)
        with pytest.raises(GpuContractException):
            b.load_kernels()
        mode, res = b.denormal_probe()
        print("fp32 denormals:", mode, ["%08x" % r for r in res], flush=True)
        assert mode in ("preserve", "flush", "mixed")
        layout = HeapLayout.of_pages([(4, 64 << 10)])
        heap = b.create_heap(layout)
        with pytest.raises(GpuContractException):
            b.create_heap(layout)
        t = TensorTable(layout)
        t.add("x", 1, 0, F32, [16])
        sealed = t.seal()
        cl = b.begin()
        with pytest.raises(GpuContractException, match="table"):
            cl.dispatch("scale_f32", ArgBlock.encode("scale_f32", x=1, y=1, n=16, a=2.0))
        heap.write_table(sealed)
        with pytest.raises(GpuContractException):
            heap.write_table(sealed)
        heap.upload(1, 0, np.arange(16, dtype=np.float32))
        cl = b.begin()
        tm = cl.begin_timer("gpu.test")
        cl.dispatch("scale_f32", ArgBlock.encode("scale_f32", x=1, y=1, n=16, a=2.0))
        cl.barrier()
        cl.end_timer(tm)
        s1 = b.submit(cl)
        comp = b.wait(s1)
        assert comp.dispatches == 1 and comp.timers[0].name == "gpu.test" and comp.timers[0].duration_ns >= 0
        assert b.wait(s1) == comp  # idempotent
        with pytest.raises(GpuContractException):
            b.submit(cl)  # a list is used once
        got = np.frombuffer(heap.download(1, 0, 64), np.float32)
        assert (got == 2 * np.arange(16, dtype=np.float32)).all()
        with pytest.raises(GpuContractException):
            heap.upload(0, 0, np.zeros(4, np.uint8))  # slot 0 is the table
        # a loop that submits and waits once per step holds bounded host memory: the last 1024 completions stay
        # waitable, older ones are dropped with a clear error
        fences = []
        for _ in range(1030):
            cl = b.begin()
            cl.dispatch("scale_f32", ArgBlock.encode("scale_f32", x=1, y=1, n=16, a=1.0))
            fences.append(b.submit(cl))
            assert b.wait(fences[-1]).dispatches == 1
        assert b.wait(fences[-1]).dispatches == 1 and b.wait(fences[-1024]).dispatches == 1
        with pytest.raises(GpuContractException, match="dropped"):
            b.wait(s1)
        with pytest.raises(GpuContractException, match="never made"):
            b.wait(fences[-1] + 1)
    finally:
        b.close()


def test_selftest_kernels():
    n = 70000 * 1  # groups_echo with more than 65,535 groups exercises folding
    s = Session({
        "x": (F32, (1000,), 0, None), "y": (F32, (1000,), 0, None), "echo": (U32, (32,), 0, None),
        "groups": (U32, (n + 64,), 0, None), "bx": (BF16, (999,), 0, None), "by": (F32, (999,), 0, None),
    })
    try:
        x = np.frombuffer(np.array([0x3F800000, 0x01000000, 0x00800000, 0x80800000, 0x00000002, 0x807FFFFE, 0x00400000]
                                   * 150, np.uint32)[:1000].tobytes(), np.float32).copy()
        x[-1] = -0.0
        s.write("x", x)
        y = s.run("scale_f32", ["y"], x="x", y="y", n=1000, a=0.5)["y"]
        ref = (np.float32(0.5) * x).astype(np.float32)
        mode, _ = s.backend.denormal_probe()
        if mode == "preserve":
            assert y.view(np.uint32).tolist() == ref.view(np.uint32).tolist()
        # table_echo: the row of token 1, and the null row
        e = s.run("table_echo", ["echo"], src="x", y="echo")["echo"]
        assert e[:16].tolist() == s.table.row(s.tok["x"]) and written_everywhere(e[:16])
        e = s.run("table_echo", ["echo"], src=0, y="echo")["echo"]
        assert e[:16].tolist() == [0] * 16
        # args_echo: all 32 words as dispatched, word 0 = physical groups x = 1
        words = {f"v{i}": 1000 + i for i in range(2, 32)}
        e = s.run("args_echo", ["echo"], y="echo", **words)["echo"]
        assert e[0] == 1 and e[1] == s.tok["echo"] and e[2:].tolist() == [1000 + i for i in range(2, 32)]
        # groups_echo above 65,535 groups: folded, the extra groups write nothing
        g = s.run("groups_echo", ["groups"], y="groups", groups=n)["groups"]
        assert g[:n].tolist() == list(range(n)) and (g[n:] == 0x7FA5A5A5).all()
        # bf16_unpack: exact widening, NaN payloads included
        bx = np.arange(999, dtype=np.uint32).astype(np.uint16) * 65 + 0x7F81
        s.write("bx", bx)
        by = s.run("bf16_unpack", ["by"], x="bx", y="by", n=999)["by"]
        assert by.view(np.uint32).tolist() == (bx.astype(np.uint32) << 16).tolist()
    finally:
        s.close()


# ---------------------------------------------------------------- the K1 kernels


def test_embed_gather_bit_exact_with_nan_rows():
    r = rng(1)
    table = bf16(r.standard_normal((300, 96)))
    table[5, :4] = [0x7F81, 0xFF80, 0x0001, 0x8000]
    ids = np.array([5, 0, 299, 300, 7000, 12], np.uint32)
    s = Session({"ids": (U32, (6,), 0, ids), "t": (BF16, (300, 96), RO, table), "y": (F32, (6, 96), 0, None)})
    try:
        y = s.run("embed_gather_bf16", ["y"], ids="ids", table="t", y="y", rows=6, cols=96, vocab=300)["y"]
        ref = cpuref.embed_gather(table, ids)
        assert y.tobytes() == ref.tobytes()
    finally:
        s.close()


@pytest.mark.parametrize("rows,cols", [(1, 1024), (13, 64), (7 * 16, 128), (3, 3000)])
def test_rmsnorm_rows(rows, cols):
    r = rng(rows * cols)
    x = (r.standard_normal((rows, cols)) * 3).astype(np.float32)
    w = bf16(r.standard_normal(cols))
    s = Session({"x": (F32, (rows, cols), 0, x), "w": (BF16, (cols,), RO, w), "y": (F32, (rows, cols), 0, None)})
    try:
        y = s.run("rmsnorm_rows", ["y"], x="x", w="w", y="y", rows=rows, cols=cols, eps=1e-6)["y"]
        check_relative(y, cpuref.rmsnorm(x, w, 1e-6), cpuref.rmsnorm(x.astype(np.float64), w, 1e-6), "rmsnorm")
    finally:
        s.close()


@pytest.mark.parametrize("heads,hd,pos0", [(4, 16, 0), (16, 128, 37), (8, 128, 4000)])
def test_rope_apply_equals_cpuref(heads, hd, pos0):
    from rosylnalive_amd.qwen import inv_freq_bits
    t = 5
    cos, sin = cpuref.rope_table(inv_freq_bits(hd), pos0 + t)
    x = rng(hd).standard_normal((t, heads * hd)).astype(np.float32)
    s = Session({"x": (F32, x.shape, 0, x), "c": (F32, cos.shape, RO, cos), "s": (F32, sin.shape, RO, sin),
                 "y": (F32, x.shape, 0, None)})
    try:
        y = s.run("rope_apply", ["y"], x="x", cos_table="c", sin_table="s", y="y", rows=t * heads, heads=heads,
                  head_dim=hd, pos0=pos0)["y"]
        # products rounded before the add on both sides: bit-equal to CpuRef F32
        assert y.tobytes() == cpuref.rope_apply(cos, sin, x, heads, pos0).tobytes()
    finally:
        s.close()


def test_silu_mul_add_copy_rows():
    r = rng(3)
    n = 70000  # folded grid
    g = (r.standard_normal(n) * 6).astype(np.float32)
    g[:6] = [0.0, -0.0, 90.0, -90.0, 1e-40, -200.0]
    u = r.standard_normal(n).astype(np.float32)
    s = Session({"g": (F32, (n,), 0, g), "u": (F32, (n,), 0, u), "y": (F32, (n,), 0, None),
                 "src": (F32, (40, 64), 0, r.standard_normal((40, 64)).astype(np.float32)),
                 "dst": (F32, (100, 80), 0, np.zeros((100, 80), np.float32))})
    try:
        y = s.run("silu_mul", ["y"], gate="g", up="u", y="y", n=n)["y"]
        check_relative(y, cpuref.silu_mul(g, u), cpuref.silu_mul(g.astype(np.float64), u), "silu_mul")
        y = s.run("add", ["y"], a="g", b="u", y="y", n=n)["y"]
        assert y.tobytes() == cpuref.add(g, u).tobytes()
        s.write("dst", np.zeros((100, 80), np.float32))
        cl = s.backend.begin()
        cl.dispatch("copy_rows", ArgBlock.encode("copy_rows", src=s.tok["src"], dst=s.tok["dst"], rows=10, cols=64,
                                                 src_row0=3, dst_row0=50, src_stride=64, dst_stride=80))
        s.backend.wait(s.backend.submit(cl))
        d = s.read("dst")
        assert d[50:60, :64].tobytes() == s.read("src")[3:13].tobytes() and (d[:50] == 0).all() and (d[50:60, 64:] == 0).all()
    finally:
        s.close()


def test_argmax_rows_ties_nan_and_wide_rows():
    r = rng(4)
    x = r.standard_normal((6, 151936)).astype(np.float32)
    x[1, :] = 0.0
    x[1, 77] = -0.0
    x[2, 100000] = 50.0
    x[2, 150000] = 50.0
    x[3, 12345] = np.nan
    x[4, :] = -np.inf
    s = Session({"x": (F32, x.shape, 0, x), "y": (U32, (6,), 0, None)})
    try:
        y = s.run("argmax_rows", ["y"], x="x", y="y", rows=6, cols=151936)["y"]
        assert y.tolist() == cpuref.argmax_rows(x).tolist()
        assert y[1] == 0 and y[2] == 100000 and y[3] == 0xFFFFFFFF and y[4] == 0
    finally:
        s.close()


# ---------------------------------------------------------------- K2 / K3


@pytest.mark.parametrize("m,n,k", [(1, 2048, 1024), (37, 1024, 1024), (16, 192, 64), (5, 96, 256), (130, 70, 50)])
def test_matmul_bf16w_is_cpuref_f32(m, n, k):
    r = rng(m * n + k)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = bf16(r.standard_normal((n, k)) * 0.1)
    s = Session({"x": (F32, x.shape, 0, x), "w": (BF16, w.shape, RO, w), "y": (F32, (m, n), 0, None)})
    try:
        y = s.run("matmul_bf16w", ["y"], x="x", w="w", y="y", m=m, n=n, k=k)["y"]
        ref = cpuref.matmul_bf16w(x, w)
        # the same sequential fused chain: equal to CpuRef F32 bit for bit, so also inside KernelBounds
        assert y.tobytes() == ref.tobytes()
    finally:
        s.close()


@pytest.mark.parametrize("rows,past,qh,kvh,hd", [(1, 0, 4, 2, 16), (16, 0, 4, 2, 16), (1, 383, 16, 8, 128),
                                                 (70, 0, 4, 2, 32), (7, 120, 16, 8, 128), (3, 4095, 16, 8, 128)])
def test_attention_gqa_causal(rows, past, qh, kvh, hd):
    r = rng(rows + past)
    tk = past + rows
    q = r.standard_normal((rows, qh * hd)).astype(np.float32)
    k = r.standard_normal((tk, kvh * hd)).astype(np.float32)
    v = r.standard_normal((tk, kvh * hd)).astype(np.float32)
    scale = cpuref.attention_scale(hd, np.float32)
    s = Session({"q": (F32, q.shape, 0, q), "k": (F32, k.shape, 0, k), "v": (F32, v.shape, 0, v),
                 "y": (F32, q.shape, 0, None)})
    try:
        y = s.run("attention_gqa_causal", ["y"], q="q", k="k", v="v", y="y", rows=rows, q_row0=0, past=past,
                  q_heads=qh, kv_heads=kvh, head_dim=hd, scale=float(scale))["y"]
        assert written_everywhere(y)
        r32 = cpuref.attention(q, k, v, qh, kvh, hd, past, scale)
        r64 = cpuref.attention(q.astype(np.float64), k, v, qh, kvh, hd, past, float(scale))
        check_relative(y, r32, r64, "attention")
    finally:
        s.close()


def test_attention_gqa_causal_isolated_op_2048_fp32():
    """The isolated GQA causal prefill attention at full size, fp32 leg: batch 1, seq 2048, 16 Q heads, 8 KV heads,
    head_dim 128; Q, K, V ~ N(0, 1) from a seed, per-head RMSNorm (weights 1) and RoPE (theta 1e6, positions 0..2047)
    applied to Q and K first; scale 1/sqrt(128), causal mask. Within KernelBounds of CpuRef F32 against F64."""
    T, qh, kvh, hd = 2048, 16, 8, 128
    r = rng(2048)
    q = r.standard_normal((T, qh * hd)).astype(np.float32)
    k = r.standard_normal((T, kvh * hd)).astype(np.float32)
    v = r.standard_normal((T, kvh * hd)).astype(np.float32)
    ones = np.full(hd, 0x3F80, np.uint16)
    cos, sin = cpuref.rope_table(np.array(QWEN3_INV_FREQ_HD128, np.uint32), T)
    q = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(q.reshape(-1, hd), ones, 1e-6).reshape(T, -1), qh, 0)
    k = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(k.reshape(-1, hd), ones, 1e-6).reshape(T, -1), kvh, 0)
    scale = cpuref.attention_scale(hd, np.float32)
    s = Session({"q": (F32, q.shape, 0, q), "k": (F32, k.shape, 0, k), "v": (F32, v.shape, 0, v),
                 "y": (F32, q.shape, 0, None)})
    try:
        y = s.run("attention_gqa_causal", ["y"], q="q", k="k", v="v", y="y", rows=T, q_row0=0, past=0,
                  q_heads=qh, kv_heads=kvh, head_dim=hd, scale=float(scale))["y"]
        assert written_everywhere(y)
        r32 = cpuref.attention(q, k, v, qh, kvh, hd, 0, scale)
        r64 = cpuref.attention(q.astype(np.float64), k, v, qh, kvh, hd, 0, float(scale))
        chk = check_relative(y, r32, r64, "attention 2048")
        print(f"attention_gqa_causal T 2048 fp32: relL2 vs F64 {chk['measured']:.3g} (bound {chk['bound']:.3g})",
              flush=True)
    finally:
        s.close()
