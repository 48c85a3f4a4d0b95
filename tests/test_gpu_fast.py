"""GPU tests of the fast kernels in isolation, through catalog dispatches: the fp16 MFMA GEMM epilogues, the MFMA
flash-attention prefill kernel (the isolated-attention workload: T 2048, 16/8 heads, head_dim 128, Q/K RMS-normed
and RoPE'd first), the decode GEMVs, the split-KV decode attention with its cache append, and the on-device argmax,
each against the oracle or an float64 restatement on the same rounded inputs.
"""
import numpy as np
import pytest

from gpu_session import POISON_16, Session, written_everywhere
from kv_layout import v_block, v_unblock
from oracle import cpuref, metrics
from rosylnalive_amd.gpu_core import (ATTN_PREFILL_RECORD_WORDS, DType, TensorFlags,
                                      attention_prefill_workspace_words)
from rosylnalive_amd.qwen import inv_freq_bits, synthetic_normal_f32

pytestmark = pytest.mark.gpu

F32, BF16, F16, U32 = DType.F32, DType.BF16, DType.F16, DType.U32
RO = TensorFlags.READ_ONLY


def bf16(a):
    return cpuref.bf16_narrow(np.asarray(a, np.float32))


def widen(b):
    return cpuref.bf16_widen(b)


def f16(a):
    """float -> fp16 bits (round to nearest even)."""
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def hwiden(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------- prefill kernels

@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (512, 1024, 1024), (37, 300, 192), (2048, 2048, 1024),
                                   (300, 200, 128), (2048, 1024, 3072), (4000, 1024, 1024)])
def test_gemm_f32_and_residual(m, n, k):
    """f32 and residual epilogues over whole and partial tiles; the residual GEMMs with few tiles and an even number
    of 64-wide k steps (1024, 128, 3072) run with K split between two wave groups of the block."""
    r = np.random.default_rng(m + n + k)
    a = f16(r.standard_normal((m, k)))
    w = f16(r.standard_normal((n, k)) * 0.05)
    x0 = r.standard_normal((m, n)).astype(np.float32)
    s = Session({"a": (F16, (m, k), 0, a), "w": (F16, (n, k), RO, w), "y": (F32, (m, n), 0, None),
                 "x": (F32, (m, n), 0, x0)})
    try:
        ref = hwiden(a).astype(np.float64) @ hwiden(w).astype(np.float64).T
        y = s.run("gemm_f32", ["y"], a="a", w="w", y="y", m=m, n=n, k=k)["y"]
        assert written_everywhere(y)
        assert metrics.rel_l2(y, ref) < 1e-6, metrics.rel_l2(y, ref)
        cl = s.backend.begin()
        cl.dispatch("gemm_residual", s.fields("gemm_residual", a="a", w="w", x="x", m=m, n=n, k=k))
        s.backend.wait(s.backend.submit(cl))
        cl.release()
        assert metrics.rel_l2(s.read("x"), x0 + ref) < 1e-6
    finally:
        s.close()


@pytest.mark.parametrize("m,n,k,splits", [(2048, 1024, 3072, 2), (512, 1024, 2048, 8), (300, 256, 512, 4),
                                          (128, 512, 1024, 1), (77, 1024, 1024, 2), (16, 2048, 6144, 2),
                                          (5, 2048, 2048, 2), (16, 1024, 4096, 4), (4000, 1024, 3072, 2)])
def test_gemm_residual_split_and_add_norm(m, n, k, splits):
    """The k-split residual GEMM: each split's partial product against float64 (whole and partial tiles, the
    direct-to-LDS loop at 512 blocks and the register loop otherwise, the skinny form for m <= 16); residual_add_norm: x + p0 + p1 + ... in split
    order, bit for bit with float32 arithmetic on the same partials, and its f16 norm output bit for bit with
    rmsnorm_rows_f16 on the resulting x."""
    r = np.random.default_rng(m + n + k + splits)
    a = f16(r.standard_normal((m, k)))
    w = f16(r.standard_normal((n, k)) * 0.05)
    x0 = r.standard_normal((m, n)).astype(np.float32)
    nw = bf16(1 + 0.1 * r.standard_normal(n))
    s = Session({"a": (F16, (m, k), 0, a), "w": (F16, (n, k), RO, w), "p": (F32, (splits, m, n), 0, None),
                 "x": (F32, (m, n), 0, x0), "nw": (BF16, (n,), RO, nw), "h": (F16, (m, n), 0, None),
                 "h2": (F16, (m, n), 0, None)})
    try:
        part = s.run("gemm_residual_split", ["p"], a="a", w="w", partials="p", m=m, n=n, k=k, splits=splits)["p"]
        part = part.reshape(splits, m, n)
        ks = k // splits
        for z in range(splits):
            ref = hwiden(a[:, z * ks:(z + 1) * ks]).astype(np.float64) @ hwiden(w[:, z * ks:(z + 1) * ks]).astype(np.float64).T
            assert metrics.rel_l2(part[z], ref) < 1e-6, (z, metrics.rel_l2(part[z], ref))
        cl = s.backend.begin()
        cl.dispatch("residual_add_norm", s.fields("residual_add_norm", x="x", partials="p", w="nw", y="h", rows=m,
                                                  cols=n, splits=splits, eps=1e-6))
        cl.barrier()
        cl.dispatch("rmsnorm_rows_f16", s.fields("rmsnorm_rows_f16", x="x", w="nw", y="h2", rows=m, cols=n, eps=1e-6,
                                                 x_row0=0))
        s.backend.wait(s.backend.submit(cl))
        cl.release()
        xe = x0.copy()
        for z in range(splits):
            xe = xe + part[z]  # float32, split order
        assert np.array_equal(s.read("x").view(np.uint32), xe.view(np.uint32))
        assert np.array_equal(s.read("h"), s.read("h2"))
    finally:
        s.close()


@pytest.mark.parametrize("m,n,k", [(2048, 4096, 256), (300, 131100, 128)])
def test_gemm_f32_large_grids(m, n, k):
    """gemm_f32 over grids of whole rounds of blocks (2048 x 4096: 512 tiles, the direct-to-LDS loop) and of tiles
    partial in both m and n (131,100 columns: 1025 column tiles, the lm_head's shape class), against float64."""
    r = np.random.default_rng(m + n + k)
    a = f16(r.standard_normal((m, k)))
    w = f16(r.standard_normal((n, k)) * 0.05)
    s = Session({"a": (F16, (m, k), 0, a), "w": (F16, (n, k), RO, w), "y": (F32, (m, n), 0, None)})
    try:
        y = s.run("gemm_f32", ["y"], a="a", w="w", y="y", m=m, n=n, k=k)["y"]
        assert written_everywhere(y)
        ref = hwiden(a).astype(np.float64) @ hwiden(w).astype(np.float64).T
        assert metrics.rel_l2(y, ref) < 1e-6, metrics.rel_l2(y, ref)
    finally:
        s.close()


@pytest.mark.parametrize("m,inter,k", [(200, 192, 128), (512, 3072, 1024), (2048, 4096, 128), (2048, 3072, 1024),
                                       (2000, 3072, 256)])
def test_gemm_swiglu(m, inter, k):
    """SwiGLU epilogue on 64-pair tiles (200 rows: partial tiles; 512 rows: 48 x 4 tiles on the register loop; 2048
    rows, 4096 pairs: 1024 tiles on the direct-to-LDS loop), and on the 96-pair tiles (3072 pairs: 32 x 16 = 512 tiles)
    of the 2048-token prefill, also with a partial last row tile."""
    r = np.random.default_rng(3)
    a = f16(r.standard_normal((m, k)))
    w = f16(r.standard_normal((2 * inter, k)) * 0.1)
    s = Session({"a": (F16, (m, k), 0, a), "w": (F16, (2 * inter, k), RO, w), "y": (F16, (m, inter), 0, None)})
    try:
        y = hwiden(s.run("gemm_swiglu", ["y"], a="a", w="w", y="y", m=m, inter=inter, k=k)["y"])
        assert np.isfinite(y).all()
        h = hwiden(a).astype(np.float64) @ hwiden(w).astype(np.float64).T
        g, u = h[:, :inter], h[:, inter:]
        ref = g / (1 + np.exp(-g)) * u
        assert metrics.rel_l2(y, ref) < 2e-3
    finally:
        s.close()


@pytest.mark.parametrize("kernel,m,inter,k", [("gemm_swiglu", 2048, 3072, 1024), ("gemm_swiglu", 200, 192, 128),
                                              ("gemm_skinny_swiglu", 16, 3072, 1024)])
def test_swiglu_a_shift(kernel, m, inter, k):
    """a_shift s makes the SwiGLU producers store a 2^-s. Where a 2^-s is still a normal fp16 number (here: where
    |a| >= 2^-5) the stored value times 2^s is the unshifted store bit for bit; below that the two differ by at most
    two half-ulps of the subnormal grid (2^-17 each after rescaling)."""
    r = np.random.default_rng(11)
    a = f16(r.standard_normal((m, k)))
    w = f16(r.standard_normal((2 * inter, k)) * 0.1)
    s = Session({"a": (F16, (m, k), 0, a), "w": (F16, (2 * inter, k), RO, w), "y": (F16, (m, inter), 0, None)})
    try:
        y0 = hwiden(s.run(kernel, ["y"], a="a", w="w", y="y", m=m, inter=inter, k=k, a_shift=0)["y"])
        y8 = hwiden(s.run(kernel, ["y"], a="a", w="w", y="y", m=m, inter=inter, k=k, a_shift=8)["y"])
        big = np.abs(y0) >= 2.0 ** -5
        assert big.mean() > 0.5
        assert np.array_equal(y8[big] * 256, y0[big])
        assert np.abs(y8[~big] * 256 - y0[~big]).max() <= 2.0 ** -16
    finally:
        s.close()


@pytest.mark.parametrize("kernel,m,n,k,splits", [("gemm_residual", 512, 1024, 1024, 0),
                                                 ("gemm_residual", 2048, 2048, 1024, 0),
                                                 ("gemm_skinny_residual", 16, 1024, 3072, 0),
                                                 ("gemm_residual_split", 2048, 1024, 3072, 2),
                                                 ("gemm_residual_split", 300, 256, 512, 4),
                                                 ("gemm_residual_split", 77, 1024, 1024, 2),
                                                 ("gemm_residual_split", 16, 1024, 4096, 4)])
def test_residual_a_shift_is_exact(kernel, m, n, k, splits):
    """The SwiGLU output's consumers multiply their sums by 2^a_shift: a 2^-8 in with a_shift 8 gives the bits of a in
    with a_shift 0 (a power-of-two scale commutes with every float32 rounding of the sums), on every loop the kernels
    choose (narrow and wide residual tiles, the skinny form, the split GEMM's direct-to-LDS, register, 64-row and
    skinny forms)."""
    r = np.random.default_rng(m + n + k + splits)
    a_lo = f16(r.standard_normal((m, k)) * 0.01)
    a_hi = f16(hwiden(a_lo) * 256)
    assert np.array_equal(hwiden(a_hi), hwiden(a_lo) * 256)  # exact: no fp16 overflow
    w = f16(r.standard_normal((n, k)) * 0.05)
    x0 = r.standard_normal((m, n)).astype(np.float32)
    out = (F32, (max(splits, 1), m, n), 0, None)
    s = Session({"lo": (F16, (m, k), 0, a_lo), "hi": (F16, (m, k), 0, a_hi), "w": (F16, (n, k), RO, w),
                 "x": (F32, (m, n), 0, x0), "p": out})
    try:
        def run(a, shift):
            if kernel == "gemm_residual_split":
                return s.run(kernel, ["p"], a=a, w="w", partials="p", m=m, n=n, k=k, splits=splits,
                             a_shift=shift)["p"]
            s.write("x", x0)
            cl = s.backend.begin()
            cl.dispatch(kernel, s.fields(kernel, a=a, w="w", x="x", m=m, n=n, k=k, a_shift=shift))
            s.backend.wait(s.backend.submit(cl))
            cl.release()
            return s.read("x")
        y0, y8 = run("hi", 0), run("lo", 8)
        assert np.isfinite(y0).all()
        assert np.array_equal(y0.view(np.uint32), y8.view(np.uint32))
    finally:
        s.close()


@pytest.mark.parametrize("T,pos0,max_pos", [(100, 37, 256), (300, 64, 512), (512, 64, 640), (1100, 37, 1152),
                                           (2048, 37, 2112), (2048, 64, 2112)])
def test_gemm_qkv_rope_epilogue(T, pos0, max_pos):
    """q|k|v projection with the per-head RMSNorm + RoPE epilogue and the K / V^T cache writes, against CpuRef F64
    on the same fp16 operands. Under 256 tiles of 128 rows the tiles are 64 rows: 100 and 300 rows at an unaligned
    position (element-wise V^T stores) and an aligned one (16-byte rows for the whole row tiles, element-wise for the
    partial last), 512 rows (the 512-token prefill: 32 x 8 tiles); 1100 rows: 128-row tiles on the register loop;
    2048 rows (512 tiles: the direct-to-LDS loop of the 2048-token prefill) at both kinds of first position."""
    H = 256
    r = np.random.default_rng(11)
    h = f16(r.standard_normal((T, H)))
    w = f16(r.standard_normal((32 * 128, H)) * 0.06)
    qn = bf16(1 + 0.1 * r.standard_normal(128))
    kn = bf16(1 + 0.1 * r.standard_normal(128))
    cos, sin = cpuref.rope_table(inv_freq_bits(128), max_pos)
    s = Session({"h": (F16, h.shape, 0, h), "w": (F16, w.shape, RO, w), "qn": (BF16, (128,), RO, qn),
                 "kn": (BF16, (128,), RO, kn), "cos": (F32, cos.shape, RO, cos), "sin": (F32, sin.shape, RO, sin),
                 "q": (F16, (T, 2048), 0, None), "kc": (F16, (8, max_pos, 128), 0, None),
                 "vc": (F16, (8, 128, max_pos), 0, None)})
    try:
        out = s.run("gemm_qkv_rope", ["q", "kc", "vc"], h="h", w="w", q_norm="qn", k_norm="kn", cos_table="cos",
                    sin_table="sin", q="q", k_cache="kc", v_cache="vc", m=T, hidden=H, q_heads=16, kv_heads=8,
                    pos0=pos0, max_pos=max_pos, eps=1e-6)
        proj = hwiden(h).astype(np.float64) @ hwiden(w).astype(np.float64).T
        qr = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(proj[:, :2048].copy(), qn, 1e-6), 16, pos0)
        kr = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(proj[:, 2048:3072].copy(), kn, 1e-6), 8, pos0)
        v = proj[:, 3072:]
        vt = v_unblock(out["vc"], 8, max_pos)  # the cache's 64-position blocks -> [head, dim, position]
        kc = hwiden(out["kc"][:, pos0:pos0 + T, :]).transpose(1, 0, 2).reshape(T, 1024)
        vc = hwiden(vt[:, :, pos0:pos0 + T]).transpose(2, 0, 1).reshape(T, 1024)
        for got, ref in [(hwiden(out["q"]), qr), (kc, kr), (vc, v)]:
            assert metrics.max_abs(got, ref) <= 2e-3 * max(1.0, np.abs(ref).max()), metrics.max_abs(got, ref)
        # rows outside [pos0, pos0 + T) are untouched
        for c in (out["kc"][:, :pos0, :], out["kc"][:, pos0 + T:, :], vt[:, :, :pos0], vt[:, :, pos0 + T:]):
            assert np.all(c == POISON_16)
    finally:
        s.close()


def _qkv_inputs(T, pos0, max_pos, seed):
    """Q, K, V ~ N(0, 1) for 16 q heads / 8 kv heads, head_dim 128, with per-head RMSNorm (weight 1) and RoPE
    (theta 1e6) applied to Q and K at positions pos0.., rounded to fp16 as the fast path stores them."""
    cos, sin = cpuref.rope_table(inv_freq_bits(128), max_pos)
    q = synthetic_normal_f32(seed, "attn/q", (T, 16 * 128))
    k = synthetic_normal_f32(seed, "attn/k", (pos0 + T, 8 * 128))
    v = synthetic_normal_f32(seed, "attn/v", (pos0 + T, 8 * 128))
    ones = np.full(128, 0x3F80, np.uint16)
    qn = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(q, ones, 1e-6), 16, pos0)
    kn = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(k, ones, 1e-6), 8, 0)
    return f16(qn), f16(kn), f16(v)


def _caches(kb, vb, max_pos, fill=0):
    """Token-major [pos, kvh * 128] fp16 rows -> the fast path's head-major K cache and its V cache (64-position blocks
    of [dim][position] tiles); positions past the rows hold `fill`."""
    P = kb.shape[0]
    kc = np.full((8, max_pos, 128), fill, np.uint16)
    vt = np.full((8, 128, max_pos), fill, np.uint16)
    kc[:, :P, :] = kb.reshape(P, 8, 128).transpose(1, 0, 2)
    vt[:, :, :P] = vb.reshape(P, 8, 128).transpose(1, 2, 0)
    return kc, v_block(vt)


def test_attention_prefill_f16_split_across_xcds():
    """8 query / 4 KV heads at T 4160: 130 tiles x 4 KV heads = 520 workgroups, so the long tiles split, and the two
    parts of a pair are 65 x 4 = 260 workgroups apart: on the 8 XCDs of an MI355X (workgroup L on XCD L % 8) they run
    on different XCDs, so their partials meet only through device-scope memory. Against the oracle's attention, with
    the counters back at zero."""
    T, qh, kvh, max_pos = 4160, 8, 4, 4224
    r = np.random.default_rng(4160)
    qb = f16(r.standard_normal((T, qh * 128)))
    kb = f16(r.standard_normal((T, kvh * 128)))
    vb = f16(r.standard_normal((T, kvh * 128)))
    kc = np.full((kvh, max_pos, 128), 0x7E00, np.uint16)
    vt = np.full((kvh, 128, max_pos), 0x7E00, np.uint16)
    kc[:, :T, :] = kb.reshape(T, kvh, 128).transpose(1, 0, 2)
    vt[:, :, :T] = vb.reshape(T, kvh, 128).transpose(1, 2, 0)
    vc = v_block(vt)
    nws = attention_prefill_workspace_words(T, kvh)
    s = Session({"q": (F16, qb.shape, 0, qb), "k": (F16, kc.shape, 0, kc), "v": (F16, vc.shape, 0, vc),
                 "y": (F16, qb.shape, 0, None), "ws": (U32, (nws,), 0, np.zeros(nws, np.uint32))})
    try:
        scale = float(cpuref.attention_scale(128, np.float32))
        y = hwiden(s.run("attention_prefill_f16", ["y"], q="q", k_cache="k", v_cache="v", y="y", workspace="ws",
                         rows=T, past=0, q_heads=qh, kv_heads=kvh, max_pos=max_pos, scale=scale)["y"])
        assert not s.read("ws")[::ATTN_PREFILL_RECORD_WORDS].any()
        ref = cpuref.attention(hwiden(qb).astype(np.float64), hwiden(kb), hwiden(vb), qh, kvh, 128, 0, scale)
        err, rel = metrics.max_abs(y, ref), metrics.rel_l2(y, ref)
        print(f"attention prefill 8/4 heads T={T}: max-abs {err:.3g}, relL2 {rel:.3g}", flush=True)
        assert err <= 1e-2 and rel <= 5e-3
    finally:
        s.close()


def test_attention_prefill_f16_shared_workspace():
    """Launches of different lengths on one workspace (a record per tile pair): 2048 rows (512 workgroups: the long
    tiles split in two parts), then 512 (no split), then 2048 again, each against the oracle's attention, with the
    counters back at zero after each."""
    max_pos = 2112
    qb, kb, vb = _qkv_inputs(2048, 0, max_pos, seed=77)
    kc, vc = _caches(kb, vb, max_pos, fill=0x7E00)
    nws = attention_prefill_workspace_words(2048, 8)
    s = Session({"q": (F16, qb.shape, 0, qb), "k": (F16, kc.shape, 0, kc), "v": (F16, vc.shape, 0, vc),
                 "y": (F16, qb.shape, 0, None), "ws": (U32, (nws,), 0, np.zeros(nws, np.uint32))})
    try:
        scale = float(cpuref.attention_scale(128, np.float32))
        qf, kf, vf = hwiden(qb), hwiden(kb), hwiden(vb)
        for T in (2048, 512, 2048):
            cl = s.backend.begin()
            cl.dispatch("attention_prefill_f16", s.fields("attention_prefill_f16", q="q", k_cache="k", v_cache="v",
                                                          y="y", workspace="ws", rows=T, past=0, q_heads=16,
                                                          kv_heads=8, max_pos=max_pos, scale=scale))
            s.backend.wait(s.backend.submit(cl))
            cl.release()
            y = hwiden(s.read("y")[:T])
            ref = cpuref.attention(qf[:T].astype(np.float64), kf[:T], vf[:T], 16, 8, 128, 0, float(scale))
            assert metrics.max_abs(y, ref) <= 1e-2 and metrics.rel_l2(y, ref) <= 5e-3, T
            assert not s.read("ws")[::ATTN_PREFILL_RECORD_WORDS].any()
    finally:
        s.close()


@pytest.mark.parametrize("T,past", [(64, 0), (100, 0), (2048, 0), (77, 300), (1, 0), (33, 31), (512, 2048)])
def test_attention_prefill_f16(T, past):
    max_pos = ((past + T + 63) // 64) * 64 + 64
    qb, kb, vb = _qkv_inputs(T, past, max_pos, seed=T + past)
    kc, vc = _caches(kb, vb, max_pos, fill=0x7E00)  # NaN past the context: the kernel must never use it
    nws = attention_prefill_workspace_words(T, 8)
    s = Session({"q": (F16, qb.shape, 0, qb), "k": (F16, kc.shape, 0, kc), "v": (F16, vc.shape, 0, vc),
                 "y": (F16, qb.shape, 0, None), "ws": (U32, (nws,), 0, np.zeros(nws, np.uint32))})
    try:
        scale = float(cpuref.attention_scale(128, np.float32))
        y = hwiden(s.run("attention_prefill_f16", ["y"], q="q", k_cache="k", v_cache="v", y="y", workspace="ws",
                         rows=T, past=past, q_heads=16, kv_heads=8, max_pos=max_pos, scale=scale)["y"])
        # every split tile was merged once per launch: the counters (word 0 of each record) are back at zero
        assert not s.read("ws")[::ATTN_PREFILL_RECORD_WORDS].any()
        qf, kf, vf = hwiden(qb), hwiden(kb), hwiden(vb)
        ref = cpuref.attention(qf.astype(np.float64), kf, vf, 16, 8, 128, past, float(scale))
        err, rel = metrics.max_abs(y, ref), metrics.rel_l2(y, ref)
        print(f"attention prefill T={T} past={past}: max-abs {err:.3g}, relL2 {rel:.3g}", flush=True)
        assert err <= 1e-2 and rel <= 5e-3
    finally:
        s.close()


# ---------------------------------------------------------------- decode kernels

def test_convert_bf16_f16_bit_exact():
    n = 1_000_003
    r = np.random.default_rng(1)
    x = bf16(r.standard_normal(n) * np.exp2(r.integers(-30, 17, n)))  # subnormal and overflow ranges included
    x[:4] = [0x7F80, 0xFF80, 0x7FC0, 0x8000]
    s = Session({"x": (BF16, (n,), RO, x), "y": (F16, (n,), 0, None)})
    try:
        y = s.run("convert_bf16_f16", ["y"], x="x", y="y", n=n)["y"]
        ref = widen(x).astype(np.float16).view(np.uint16)
        nan = np.isnan(widen(x))
        assert np.array_equal(y[~nan], ref[~nan]) and np.isnan(hwiden(y[nan])).all()
    finally:
        s.close()


@pytest.mark.parametrize("reusable", [False, True])
def test_prefetch_overlapped(reusable):
    """An overlapped prefetch (side stream, joined by the barrier and by the end of the list) beside ordinary
    dispatches: the ordinary results are exact, in a one-shot list and in a reusable (graph) list replayed 3 times."""
    n = 1 << 20
    r = np.random.default_rng(5)
    x = bf16(r.standard_normal(n))
    big = bf16(r.standard_normal(3 * n))
    s = Session({"x": (BF16, (n,), RO, x), "big": (BF16, (3 * n,), RO, big), "y": (F16, (n,), 0, None),
                 "z": (F16, (n,), 0, None)})
    try:
        cl = s.backend.begin(reusable)
        cl.dispatch_overlapped("prefetch", s.fields("prefetch", x0="big", x1="x", x2="big", x3="x"))
        cl.dispatch("convert_bf16_f16", s.fields("convert_bf16_f16", x="x", y="y", n=n))
        cl.barrier()
        cl.dispatch_overlapped("prefetch", s.fields("prefetch", x0="x", x1="x", x2="x", x3="big"))
        cl.dispatch("convert_bf16_f16", s.fields("convert_bf16_f16", x="x", y="z", n=n))
        c = s.backend.wait(s.backend.submit(cl, repeat=3 if reusable else 1))
        assert c.dispatches == 4 * (3 if reusable else 1)
        cl.release()
        ref = widen(x).astype(np.float16).view(np.uint16)
        assert np.array_equal(s.read("y"), ref) and np.array_equal(s.read("z"), ref)
    finally:
        s.close()


@pytest.mark.parametrize("rows,cols,row0", [(37, 1024, 5), (16, 2048, 0), (9, 256, 1), (5, 300, 2), (3, 64, 0)])
def test_rmsnorm_rows_f16(rows, cols, row0):
    """Widths that are multiples of 256 take the wave-per-row form, the others the block-per-row one."""
    r = np.random.default_rng(2 + cols)
    x = (r.standard_normal((rows + row0, cols)) * 3).astype(np.float32)
    w = bf16(1 + 0.1 * r.standard_normal(cols))
    s = Session({"x": (F32, x.shape, RO, x), "w": (BF16, (cols,), RO, w), "y": (F16, (rows, cols), 0, None)})
    try:
        y = hwiden(s.run("rmsnorm_rows_f16", ["y"], x="x", w="w", y="y", rows=rows, cols=cols, eps=1e-6,
                         x_row0=row0)["y"])
        ref = cpuref.rmsnorm(x[row0:].astype(np.float64), w, 1e-6)
        assert np.all(np.abs(y - ref) <= np.abs(ref) * 2.0 ** -10 + 2.0 ** -24)  # within one fp16 rounding
    finally:
        s.close()


def _gemv_ref(w, x):
    return widen(w).astype(np.float64) @ np.asarray(x, np.float64)


@pytest.mark.parametrize("n,k", [(4096, 1024), (1000, 2048), (3, 8)])
def test_gemv_norm_dec(n, k):
    r = np.random.default_rng(n + k)
    x = (r.standard_normal(k) * 2).astype(np.float32)
    nw = bf16(1 + 0.1 * r.standard_normal(k))
    w = bf16(r.standard_normal((n, k)) * 0.05)
    s = Session({"x": (F32, (k,), RO, x), "nw": (BF16, (k,), RO, nw), "w": (BF16, (n, k), RO, w),
                 "y": (F32, (n,), 0, None)})
    try:
        y = s.run("gemv_norm_dec", ["y"], x="x", norm="nw", w="w", y="y", n=n, k=k, eps=1e-6)["y"]
        ref = _gemv_ref(w, cpuref.rmsnorm(x[None].astype(np.float64), nw, 1e-6)[0])
        assert metrics.rel_l2(y, ref) < 1e-5
    finally:
        s.close()


@pytest.mark.parametrize("n,k", [(1024, 2048), (1024, 3072), (4096, 1024), (77, 64)])
def test_gemv_residual_dec(n, k):
    r = np.random.default_rng(n * 7 + k)
    a = r.standard_normal(k).astype(np.float32)
    w = bf16(r.standard_normal((n, k)) * 0.05)
    x0 = r.standard_normal(n).astype(np.float32)
    s = Session({"a": (F32, (k,), RO, a), "w": (BF16, (n, k), RO, w), "x": (F32, (n,), 0, x0)})
    try:
        s.run_list([("gemv_residual_dec", dict(a="a", w="w", x="x", n=n, k=k))], [], reset={"x": x0})
        assert metrics.rel_l2(s.read("x"), x0 + _gemv_ref(w, a)) < 1e-5
    finally:
        s.close()


def test_gemv_swiglu_dec():
    inter, hidden = 3072, 1024
    r = np.random.default_rng(9)
    x = r.standard_normal(hidden).astype(np.float32)
    nw = bf16(1 + 0.1 * r.standard_normal(hidden))
    w = bf16(r.standard_normal((2 * inter, hidden)) * 0.05)
    s = Session({"x": (F32, (hidden,), RO, x), "nw": (BF16, (hidden,), RO, nw), "w": (BF16, w.shape, RO, w),
                 "y": (F32, (inter,), 0, None)})
    try:
        y = s.run("gemv_swiglu_dec", ["y"], x="x", norm="nw", w="w", y="y", inter=inter, hidden=hidden, eps=1e-6)["y"]
        h = _gemv_ref(w, cpuref.rmsnorm(x[None].astype(np.float64), nw, 1e-6)[0])
        g, u = h[:inter], h[inter:]
        assert metrics.rel_l2(y, g / (1 + np.exp(-g)) * u) < 1e-5
    finally:
        s.close()


def _lm_session(vocab, hidden, e):
    r = np.random.default_rng(vocab)
    x = r.standard_normal(hidden).astype(np.float32)
    nw = bf16(1 + 0.1 * r.standard_normal(hidden))
    return x, nw, Session({
        "x": (F32, (hidden,), RO, x), "nw": (BF16, (hidden,), RO, nw), "e": (BF16, e.shape, RO, e),
        "logits": (F32, (vocab,), 0, None), "part": (F32, (2048,), 0, None), "state": (U32, (4,), 0, None),
        "ids": (U32, (8,), 0, np.zeros(8, np.uint32))})


def _lm_run(s, vocab, hidden, state):
    return s.run_list([("lmhead_dec", dict(x="x", norm="nw", embed="e", logits="logits", partials="part", vocab=vocab,
                                          hidden=hidden, eps=1e-6, write_logits=1)),
                       ("argmax_dec", dict(partials="part", state="state", out_ids="ids", max_steps=8))],
                      ["logits"], reset={"state": state})


def test_lmhead_and_argmax_dec():
    vocab, hidden = 50021, 1024
    r = np.random.default_rng(4)
    e = bf16(r.standard_normal((vocab, hidden)) * 0.05)
    x, nw, s = _lm_session(vocab, hidden, e)
    try:
        out = _lm_run(s, vocab, hidden, np.array([17, 5, 3, 0], np.uint32))
        ref = _gemv_ref(e, cpuref.rmsnorm(x[None].astype(np.float64), nw, 1e-6)[0])
        assert metrics.rel_l2(out["logits"], ref) < 1e-5
        am = int(np.argmax(out["logits"]))
        assert list(s.read("state")[:3]) == [18, am, 4] and int(s.read("ids")[3]) == am
        # a tie between two rows resolves to the lower index, across blocks
        twin = 30001 if am != 30001 else 30002
        e2 = e.copy()
        e2[twin] = e2[am]  # the same dot product, the same bits, in another block
        s.write("e", e2)
        out2 = _lm_run(s, vocab, hidden, np.array([0, 0, 0, 0], np.uint32))
        top = np.flatnonzero(out2["logits"] == out2["logits"].max())
        assert top.size >= 2 and int(s.read("state")[1]) == int(top[0]) == min(am, twin)
        # a NaN logit gives id 0xFFFFFFFF
        e3 = e.copy()
        e3[12345, 7] = 0x7FC0
        s.write("e", e3)
        _lm_run(s, vocab, hidden, np.array([0, 0, 0, 0], np.uint32))
        assert int(s.read("state")[1]) == 0xFFFFFFFF and int(s.read("ids")[0]) == 0xFFFFFFFF
    finally:
        s.close()


def test_embed_dec():
    vocab, hidden = 300, 1024
    e = bf16(np.random.default_rng(5).standard_normal((vocab, hidden)))
    s = Session({"e": (BF16, e.shape, RO, e), "state": (U32, (4,), 0, np.array([9, 123, 0, 0], np.uint32)),
                 "x": (F32, (hidden,), 0, None)})
    try:
        x = s.run("embed_dec", ["x"], embed="e", state="state", x="x", hidden=hidden, vocab=vocab, batch=1)["x"]
        assert x.tobytes() == widen(e[123]).tobytes()
        s.write("state", np.array([9, vocab, 0, 0], np.uint32))
        x = s.run("embed_dec", ["x"], embed="e", state="state", x="x", hidden=hidden, vocab=vocab, batch=1)["x"]
        assert np.isnan(x).all()
    finally:
        s.close()


@pytest.mark.parametrize("pos,chunks", [(0, 1), (63, 1), (64, 1), (383, 1), (1000, 1), (4095, 1), (0, 4), (383, 4),
                                        (1000, 8), (4095, 16), (4095, 3), (130, 2)])
def test_attention_decode_f16(pos, chunks):
    """One decode step's attention: raw q|k|v projection in, q/k RMSNorm + RoPE at `pos`, the new key and value
    appended to the caches, split-KV attention over positions 0..pos (`chunks` 64-key chunks per split block, so
    blocks of one chunk, of several, and a last split cut short by max_pos), then the split combine."""
    max_pos = 4096
    S = max_pos // 64
    r = np.random.default_rng(pos)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), max_pos)
    _, kb, vb = _qkv_inputs(1, pos, max_pos, seed=pos + 1)  # fp16 cache rows for positions 0 .. pos
    kc, vc = _caches(kb[:pos], vb[:pos], max_pos, fill=0x7E00)  # position pos onwards: NaN until written
    qkv = (r.standard_normal(4096) * 1.5).astype(np.float32)
    qn = bf16(1 + 0.1 * r.standard_normal(128))
    kn = bf16(1 + 0.1 * r.standard_normal(128))
    state = np.array([pos, 0, 0, 0], np.uint32)
    s = Session({"qkv": (F32, (4096,), RO, qkv), "qn": (BF16, (128,), RO, qn), "kn": (BF16, (128,), RO, kn),
                 "cos": (F32, cos.shape, RO, cos), "sin": (F32, sin.shape, RO, sin),
                 "kc": (F16, kc.shape, 0, kc), "vc": (F16, vc.shape, 0, vc),
                 "part": (F32, (16 * S * 130,), 0, None), "y": (F32, (2048,), 0, None),
                 "state": (U32, (4,), RO, state)})
    try:
        scale = float(cpuref.attention_scale(128, np.float32))
        y = s.run_list([("attention_decode_f16", dict(qkv="qkv", q_norm="qn", k_norm="kn", cos_table="cos",
                                                      sin_table="sin", k_cache="kc", v_cache="vc", partials="part",
                                                      state="state", q_heads=16, kv_heads=8, max_pos=max_pos,
                                                      eps=1e-6, scale=scale, batch=1, chunks=chunks)),
                        ("attention_combine", dict(partials="part", y="y", state="state", q_heads=16,
                                                   max_pos=max_pos, batch=1, chunks=chunks))], ["y"])["y"]
        q64 = qkv[None].astype(np.float64)
        qr = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(q64[:, :2048].copy(), qn, 1e-6), 16, pos)
        kr = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(q64[:, 2048:3072].copy(), kn, 1e-6), 8, pos)
        kc2, vc2 = s.read("kc"), v_unblock(s.read("vc"), 8, max_pos)
        k_new = hwiden(kc2[:, pos, :]).reshape(1, 1024)
        v_new = vc2[:, :, pos].reshape(1, 1024)
        assert np.all(np.abs(k_new - kr) <= np.abs(kr) * 2.0 ** -10 + 2.0 ** -24), "appended key"
        assert v_new.tobytes() == f16(qkv[3072:]).reshape(1, 1024).tobytes(), "appended value"
        # other positions are untouched
        assert np.array_equal(np.delete(kc2, pos, axis=1), np.delete(kc, pos, axis=1))
        assert np.array_equal(np.delete(vc2, pos, axis=2), np.delete(v_unblock(vc, 8, max_pos), pos, axis=2))
        kf = np.concatenate([hwiden(kb[:pos]), k_new]).astype(np.float64)
        vf = np.concatenate([hwiden(vb[:pos]), hwiden(v_new)]).astype(np.float64)
        ref = cpuref.attention(qr, kf, vf, 16, 8, 128, pos, scale)
        err, rel = metrics.max_abs(y, ref), metrics.rel_l2(y, ref)
        print(f"attention decode pos={pos} chunks={chunks}: max-abs {err:.3g}, relL2 {rel:.3g}", flush=True)
        assert err <= 1e-3 and rel <= 1e-4
    finally:
        s.close()


def test_fill_normal_f16_statistics():
    n = 1 << 20
    s = Session({"y": (F16, (n,), 0, None)})
    try:
        y = hwiden(s.run("fill_normal_f16", ["y"], y="y", n=n, seed_lo=7, seed_hi=0, stream_lo=3, stream_hi=1,
                         std=1.0)["y"])
        assert np.isfinite(y).all() and abs(y.mean()) < 0.01 and abs(y.std() - 1) < 0.01
        assert np.array_equal(widen(bf16(y)), y), "every value is a bf16 value"
    finally:
        s.close()


def test_argmax_rows_split_matches_cpuref():
    """argmax_rows_partial + argmax_rows_final == CpuRef.argmaxRows: lowest index of the maximum, 0xFFFFFFFF for a row
    holding a NaN, ties across the 64 column slices, -0/+0, all -inf."""
    rows, cols = 9, 151936
    r = np.random.default_rng(12)
    x = r.standard_normal((rows, cols)).astype(np.float32)
    x[1, [5, 100000]] = 50.0          # tie across slices: 5 wins
    x[2, 7] = np.nan                  # NaN row
    x[3, :] = -np.inf                 # all -inf: index 0
    x[4, :] = 0.0
    x[4, 0] = -0.0                    # -0 then +0: index 0
    x[5, cols - 1] = 99.0             # last column
    x[6, [70000, 70001]] = 30.0       # tie inside one slice
    s = Session({"x": (F32, x.shape, RO, x), "part": (F32, (rows * 64 * 2,), 0, None), "out": (U32, (rows,), 0, None)})
    try:
        out = s.run_list([("argmax_rows_partial", dict(x="x", partials="part", rows=rows, cols=cols)),
                          ("argmax_rows_final", dict(partials="part", out="out", rows=rows))], ["out"])["out"]
        ref = cpuref.argmax_rows(x)
        assert out.tolist() == ref.tolist(), (out, ref)
        assert out[1] == 5 and out[2] == 0xFFFFFFFF and out[3] == 0 and out[4] == 0 and out[5] == cols - 1
        # row0: rows row0 .. row0 + n - 1 alone (the forward reduces only its last row)
        for row0, n in ((rows - 1, 1), (5, 2), (0, 1)):
            sub = s.run_list([("argmax_rows_partial", dict(x="x", partials="part", rows=n, cols=cols, row0=row0)),
                              ("argmax_rows_final", dict(partials="part", out="out", rows=n))], ["out"])["out"][:n]
            assert sub.tolist() == ref[row0:row0 + n].tolist(), (row0, n, sub)
    finally:
        s.close()


# ---------------------------------------------------------------- batched decode kernels

@pytest.mark.parametrize("m,n,k", [(1, 96, 1024), (5, 4096, 1024), (16, 2048, 2048), (16, 1000, 3072), (3, 9000, 1024)])
def test_gemm_skinny(m, n, k):
    r = np.random.default_rng(m * 31 + n + k)
    a = f16(r.standard_normal((m, k)))
    w = f16(r.standard_normal((n, k)) * 0.05)
    x0 = r.standard_normal((m, n)).astype(np.float32)
    s = Session({"a": (F16, (m, k), RO, a), "w": (F16, (n, k), RO, w), "y": (F32, (m, n), 0, None),
                 "x": (F32, (m, n), 0, x0)})
    try:
        ref = hwiden(a).astype(np.float64) @ hwiden(w).astype(np.float64).T
        y = s.run("gemm_skinny_f32", ["y"], a="a", w="w", y="y", m=m, n=n, k=k)["y"]
        assert written_everywhere(y) and metrics.rel_l2(y, ref) < 1e-6
        s.run_list([("gemm_skinny_residual", dict(a="a", w="w", x="x", m=m, n=n, k=k))], [], reset={"x": x0})
        assert metrics.rel_l2(s.read("x"), x0 + ref) < 1e-6
    finally:
        s.close()


@pytest.mark.parametrize("m,inter,k", [(11, 3072, 1024), (16, 6144, 2048), (3, 100, 1024), (7, 6010, 1024)])
def test_gemm_skinny_swiglu(m, inter, k):
    """Each block pairs 16 gate columns with the matching 16 up columns, or 24 with 24 where that makes one round of
    256 blocks (6144 and 6010 pairs: 256 and 251 blocks); inter 100 and 6010 end in a partial block. The 24-pair
    blocks give the bits of the 16-pair ones: the first 4096 pairs again as a 4096-pair GEMM (256 blocks of 16)."""
    r = np.random.default_rng(21)
    a = f16(r.standard_normal((m, k)))
    w = f16(r.standard_normal((2 * inter, k)) * 0.05)
    n16 = min(inter, 4096)
    w16 = np.concatenate([w[:n16], w[inter:inter + n16]])
    s = Session({"a": (F16, (m, k), RO, a), "w": (F16, w.shape, RO, w), "y": (F16, (m, inter), 0, None),
                 "w16": (F16, w16.shape, RO, w16), "y16": (F16, (m, n16), 0, None)})
    try:
        yb = s.run("gemm_skinny_swiglu", ["y"], a="a", w="w", y="y", m=m, inter=inter, k=k)["y"]
        y = hwiden(yb)
        h = hwiden(a).astype(np.float64) @ hwiden(w).astype(np.float64).T
        g, u = h[:, :inter], h[:, inter:]
        assert metrics.rel_l2(y, g / (1 + np.exp(-g)) * u) < 2e-3
        y16 = s.run("gemm_skinny_swiglu", ["y16"], a="a", w="w16", y="y16", m=m, inter=n16, k=k)["y16"]
        assert np.array_equal(y16, yb[:, :n16])
    finally:
        s.close()


@pytest.mark.parametrize("chunks,splits", [(1, 0), (4, 0), (8, 0), (0, 1), (0, 2), (0, 3), (0, 16)])
def test_attention_decode_batched_f16_combine(chunks, splits):
    """Three sequences at positions 5, 64 and 700 in one dispatch (batch on the grid), then the fp16 combine; each
    sequence against CpuRef F64 on its own cache. splits > 0: each sequence's keys spread evenly over that many
    splits (3: 64, 64 and 256 keys per split; 16: one chunk each, 1, 2 and 11 splits holding keys). The streaming
    form holds four chunks in flight: position 700 runs 8 + 3 chunks per split at chunks = 8, 11 in one split, and
    6 + 5 in two, so its loop of four-chunk groups runs once or twice and every length of the last group (1 .. 4)
    occurs."""
    max_pos, S = 1024, 16
    positions = [5, 64, 700]
    B = len(positions)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), max_pos)
    r = np.random.default_rng(33)
    qkv = (r.standard_normal((B, 4096)) * 1.5).astype(np.float32)
    qn = bf16(1 + 0.1 * r.standard_normal(128))
    kn = bf16(1 + 0.1 * r.standard_normal(128))
    kcs, vcs, rows = [], [], []
    for b, pos in enumerate(positions):
        _, kb, vb = _qkv_inputs(1, pos, max_pos, seed=100 + b)
        kc, vc = _caches(kb[:pos], vb[:pos], max_pos, fill=0x7E00)
        kcs.append(kc); vcs.append(vc); rows.append((kb[:pos], vb[:pos]))
    state = np.array(positions + [0] * B + [0, 0], np.uint32)
    s = Session({"qkv": (F32, qkv.shape, RO, qkv), "qn": (BF16, (128,), RO, qn), "kn": (BF16, (128,), RO, kn),
                 "cos": (F32, cos.shape, RO, cos), "sin": (F32, sin.shape, RO, sin),
                 "kc": (F16, (B * 8, max_pos, 128), 0, np.concatenate(kcs)),
                 "vc": (F16, (B * 8 * max_pos // 64, 128, 64), 0, np.concatenate(vcs).reshape(-1, 128, 64)),
                 "part": (F32, (B * 16 * S * 130,), 0, None), "y": (F16, (B, 2048), 0, None),
                 "state": (U32, state.shape, RO, state)})
    try:
        scale = float(cpuref.attention_scale(128, np.float32))
        y = hwiden(s.run_list([("attention_decode_f16", dict(qkv="qkv", q_norm="qn", k_norm="kn", cos_table="cos",
                                                             sin_table="sin", k_cache="kc", v_cache="vc",
                                                             partials="part", state="state", q_heads=16, kv_heads=8,
                                                             max_pos=max_pos, eps=1e-6, scale=scale, batch=B,
                                                             chunks=chunks, splits=splits)),
                               ("attention_combine_f16", dict(partials="part", y="y", state="state", q_heads=16,
                                                              max_pos=max_pos, batch=B, chunks=chunks,
                                                              splits=splits))],
                              ["y"])["y"])
        kc2 = s.read("kc").reshape(B, 8, max_pos, 128)
        vc2 = v_unblock(s.read("vc"), B * 8, max_pos).reshape(B, 8, 128, max_pos)
        for b, pos in enumerate(positions):
            q64 = qkv[b][None].astype(np.float64)
            qr = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(q64[:, :2048].copy(), qn, 1e-6), 16, pos)
            k_new = hwiden(kc2[b, :, pos, :]).reshape(1, 1024)
            v_new = hwiden(vc2[b, :, :, pos]).reshape(1, 1024)
            kf = np.concatenate([hwiden(rows[b][0]), k_new]).astype(np.float64)
            vf = np.concatenate([hwiden(rows[b][1]), v_new]).astype(np.float64)
            ref = cpuref.attention(qr, kf, vf, 16, 8, 128, pos, scale)
            err = metrics.max_abs(y[b], ref[0])
            print(f"batched decode attention seq {b} pos {pos}: max-abs {err:.3g}", flush=True)
            assert err <= 2e-3, (b, err)  # fp16 output rounding included
    finally:
        s.close()


def test_decode_advance():
    B = 5
    state = np.array([10, 11, 12, 13, 14, 1, 2, 3, 4, 5, 7, 0], np.uint32)
    am = np.array([100, 200, 300, 400, 500], np.uint32)
    s = Session({"am": (U32, (B,), RO, am), "state": (U32, state.shape, 0, state), "out": (U32, (16 * B,), 0, None)})
    try:
        out = s.run_list([("decode_advance", dict(argmax="am", state="state", out_ids="out", batch=B, max_steps=16))],
                         ["out"], reset={"state": state})["out"]
        assert s.read("state")[:2 * B + 1].tolist() == [11, 12, 13, 14, 15, 100, 200, 300, 400, 500, 8]
        assert out[7 * B:8 * B].tolist() == am.tolist()
    finally:
        s.close()
