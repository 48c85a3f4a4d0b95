"""The reference's attention conformance matrix (tests/Lrm.Kernels.Conformance/Cases/attention/AttentionCases.fs:100-357)
through this device, and the same adversarial magnitudes for the fast path's fp16 attention kernels.

- attention_gqa_causal (catalog id 13, fp32): the layout cases (tiny 4:2 head_dim 32, MHA 4:4, MQA 8:1, 6:3, 3:1,
  head_dim 1, 3, 64, 96, 130, 200, 256, one query of one head, 8,192 queries of one head) and the adversarial ones
  (scores in the thousands and near 1e24, scores of about -113, a maximum that rises in every block, a dominant first
  or last key, q = 0 over 2,001 keys, tied keys, values near 1e30, 1e-30 and denormal, denormal values on every other
  key). As the reference's harness runs them: every cache row past the last key (64 of them) and every q row the
  dispatch does not own holds the quiet NaN, y's spare rows must stay untouched, each case runs twice with the same
  bits, the result is within KernelBounds of CpuRef F64 against CpuRef F32, and the batch-invariance splits (the first
  query alone as a decode step at `past`, the last query alone, the middle third as a chunk) give the same bits as the
  whole dispatch. The input generators follow the reference's (same distributions; this session's seeds).
- attention_prefill_f16 and attention_decode_f16 (fast path, head_dim 128, 16/8 heads, fp16 q/K/V): the adversarial
  scores that stay inside the fp16 range (large, negative, rising, dominant first and last, q = 0, tied keys), against
  float64 attention on the same fp16-rounded inputs. These exercise the lazy rescale of the prefill kernel (it moves its
  reference maximum only when a block's maximum exceeds it by more than 8 in log2) and the decode kernel's online
  softmax far from the RMS-normed inputs of a model.
"""
import zlib

import numpy as np
import pytest

from gpu_session import POISON_F32, Session
from kv_layout import v_block, v_unblock
from oracle import cpuref, metrics
from rosylnalive_amd.gpu_core import DType, TensorFlags, attention_prefill_workspace_words
from rosylnalive_amd.qwen import inv_freq_bits

pytestmark = pytest.mark.gpu

F32, BF16, F16, U32 = DType.F32, DType.BF16, DType.F16, DType.U32
RO = TensorFlags.READ_ONLY
UNREAD = np.uint32(0x7FC00000)  # the quiet NaN of every row a dispatch must not read
SPARE_ROWS, UNREAD_KEYS = 2, 64


def rng(name):
    return np.random.default_rng(zlib.crc32(name.encode()))


def uni(r, n, lo, hi):
    return r.uniform(lo, hi, n).astype(np.float32)


# ---- input generators (AttentionCases.fs:96-189): (r, qh, kvh, hd, rows, keys) -> q, k, v flat float32

def uniform(qr, kr, vr):
    return lambda r, qc, kc, rows, keys: (uni(r, rows * qc, -qr, qr), uni(r, keys * kc, -kr, kr),
                                          uni(r, keys * kc, -vr, vr))


def dominant_at(which):
    def gen(r, qc, kc, rows, keys):
        q, k, v = uni(r, rows * qc, 0.5, 1.5), uni(r, keys * kc, -1, 1), uni(r, keys * kc, -1, 1)
        for j in which(keys):
            k[j * kc:(j + 1) * kc] = 8.4
        return q, k, v
    return gen


def rising(r, qc, kc, rows, keys):
    q = np.full(rows * qc, 0.5, np.float32)
    k = (0.03 * (np.arange(keys * kc) // kc) + uni(r, keys * kc, -0.05, 0.05)).astype(np.float32)
    return q, k, uni(r, keys * kc, -1, 1)


def negative(r, qc, kc, rows, keys):
    return uni(r, rows * qc, 0.5, 1.5), uni(r, keys * kc, -11, -9), uni(r, keys * kc, -1, 1)


def zero_queries(r, qc, kc, rows, keys):
    return np.zeros(rows * qc, np.float32), uni(r, keys * kc, -1, 1), uni(r, keys * kc, -1, 1)


def tied_keys(r, qc, kc, rows, keys):
    first = uni(r, kc, -1, 1)
    return uni(r, rows * qc, -1, 1), np.tile(first, keys), uni(r, keys * kc, -1, 1)


def denormal_values(r, qc, kc, rows, keys):
    w = r.integers(0, 1 << 32, keys * kc, dtype=np.uint64).astype(np.uint32)
    v = ((w & 0x80000000) | 0x00002000 | (w & 0x007FFFFF)).astype(np.uint32).view(np.float32)
    return uni(r, rows * qc, -1, 1), uni(r, keys * kc, -1, 1), v


def mixed_denormal_values(r, qc, kc, rows, keys):
    q, k, d = denormal_values(r, qc, kc, rows, keys)
    normal = uni(r, keys * kc, -1, 1)
    odd = (np.arange(keys * kc) // kc) % 2 == 1
    return q, k, np.where(odd, d, normal).astype(np.float32)


QWEN, TINY = (16, 8, 128), (4, 2, 32)
SMALL = uniform(1.0, 1.0, 1.0)
# name, (q_heads, kv_heads, head_dim), rows, q_row0, past, generator  (AttentionCases.fs:220-357)
CATALOG_CASES = [
    ("qwen_decode_p0", QWEN, 1, 0, 0, uniform(2, 2, 1)),
    ("qwen_decode_p63", QWEN, 1, 0, 63, uniform(2, 2, 1)),
    ("qwen_decode_p64", QWEN, 1, 0, 64, uniform(2, 2, 1)),
    ("qwen_decode_p127_q5", QWEN, 1, 5, 127, uniform(2, 2, 1)),
    ("qwen_prefill_t7", QWEN, 7, 0, 0, uniform(2, 2, 1)),
    ("qwen_prefill_t130", QWEN, 130, 0, 0, uniform(2, 2, 1)),
    ("qwen_chunk_t64_past64", QWEN, 64, 0, 64, uniform(2, 2, 1)),
    ("qwen_chunk_t37_past100_q3", QWEN, 37, 3, 100, uniform(2, 2, 1)),
    ("qwen_decode_p4000", QWEN, 1, 0, 4000, uniform(2, 2, 1)),
    ("qwen_decode_p4095", QWEN, 1, 0, 4095, uniform(2, 2, 1)),
    ("qwen_chunk_t128_past3968", QWEN, 128, 0, 3968, uniform(2, 2, 1)),
    ("tiny_prefill_t9", TINY, 9, 0, 0, SMALL),
    ("tiny_chunk_t6_past70_q2", TINY, 6, 2, 70, SMALL),
    ("mha_4x4_hd64_t20_past50", (4, 4, 64), 20, 0, 50, SMALL),
    ("mqa_8x1_hd96_t5_past200", (8, 1, 96), 5, 0, 200, SMALL),
    ("gqa_6x3_hd130_t3_past66", (6, 3, 130), 3, 1, 66, SMALL),
    ("gqa_3x1_hd3_t11_past129", (3, 1, 3), 11, 0, 129, SMALL),
    ("hd1_t70", (1, 1, 1), 70, 0, 0, SMALL),
    ("hd200_t4_past61", (2, 1, 200), 4, 0, 61, SMALL),
    ("hd256_t3_past140", (4, 2, 256), 3, 0, 140, SMALL),
    ("one_query_one_head", (1, 1, 128), 1, 0, 0, SMALL),
    ("grid_rows8192", (1, 1, 1), 8192, 0, 0, SMALL),
    ("adv_large_scores", QWEN, 4, 0, 300, uniform(40, 40, 1)),
    ("adv_huge_scores", QWEN, 3, 0, 150, uniform(1e12, 1e12, 1)),
    ("adv_negative_scores", QWEN, 3, 0, 120, negative),
    ("adv_rising_scores", QWEN, 3, 0, 400, rising),
    ("adv_dominant_first", QWEN, 3, 0, 200, dominant_at(lambda keys: [0])),
    ("adv_dominant_last", QWEN, 4, 0, 146, dominant_at(lambda keys: [keys - 1])),
    ("adv_zero_queries", QWEN, 3, 0, 2000, zero_queries),
    ("adv_tied_keys", QWEN, 2, 0, 300, tied_keys),
    ("adv_large_values", QWEN, 3, 0, 100, uniform(1, 1, 1e30)),
    ("adv_small_values", QWEN, 3, 0, 100, uniform(1, 1, 1e-30)),
    ("adv_denormal_values", QWEN, 2, 0, 70, denormal_values),
    ("adv_mixed_denormal_values", QWEN, 3, 0, 70, mixed_denormal_values),
]


def _place(cap, cols, at, values):
    words = np.full(cap * cols, UNREAD, np.uint32)
    bits = np.ascontiguousarray(values, np.float32).view(np.uint32)
    words[at * cols:at * cols + bits.size] = bits
    return words.view(np.float32).reshape(cap, cols)


@pytest.mark.parametrize("name,heads,rows,q0,past,gen", CATALOG_CASES, ids=[c[0] for c in CATALOG_CASES])
def test_attention_gqa_causal_reference_cases(name, heads, rows, q0, past, gen):
    qh, kvh, hd = heads
    qc, kc = qh * hd, kvh * hd
    keys = past + rows
    q, k, v = gen(rng("attention." + name), qc, kc, rows, keys)
    q_cap, kv_cap = q0 + rows + SPARE_ROWS, keys + UNREAD_KEYS
    qa, ka, va = _place(q_cap, qc, q0, q), _place(kv_cap, kc, 0, k), _place(kv_cap, kc, 0, v)
    scale = cpuref.attention_scale(hd, np.float32)
    s = Session({"q": (F32, qa.shape, RO, qa), "k": (F32, ka.shape, RO, ka), "v": (F32, va.shape, RO, va),
                 "y": (F32, (q_cap, qc), 0, None)})
    try:
        def run(r0, n, p):
            return s.run("attention_gqa_causal", ["y"], q="q", k="k", v="v", y="y", rows=n, q_row0=r0, past=p,
                         q_heads=qh, kv_heads=kvh, head_dim=hd, scale=float(scale))["y"]
        y = run(q0, rows, past)
        spare = np.ones(q_cap, bool)
        spare[q0:q0 + rows] = False
        assert np.all(y[spare].view(np.uint32) == POISON_F32), "rows outside the dispatch were written"
        got = y[q0:q0 + rows]
        assert not np.isnan(got).any(), "NaN: a key past the bound or a foreign q row was read"
        qq = q.reshape(rows, qc)
        r32 = cpuref.attention(qq, ka[:keys], va[:keys], qh, kvh, hd, past, scale)
        r64 = cpuref.attention(qq.astype(np.float64), ka[:keys], va[:keys], qh, kvh, hd, past, float(scale))
        chk = metrics.check_relative(got, r32, r64)
        print(f"{name}: relL2 vs F64 {chk['measured']:.3g}, bound {chk['bound']:.3g}", flush=True)
        assert chk["passed"], chk
        # batch invariance: the first query alone (decode at past), the last alone, the middle third as a chunk
        splits = [(0, 1), (rows - 1, 1)]
        if rows >= 3:
            splits.append((rows // 3, rows // 3))
        for off, n in splits:
            part = run(q0 + off, n, past + off)
            assert part[q0 + off:q0 + off + n].tobytes() == got[off:off + n].tobytes(), (name, off, n)
    finally:
        s.close()


# ---------------------------------------------------------------- the fast path's fp16 kernels

def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def _hw(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


FAST_CASES = [
    ("large_scores", uniform(40, 40, 1)),
    ("negative_scores", negative),
    ("rising_scores", rising),
    ("dominant_first", dominant_at(lambda keys: [0])),
    ("dominant_last", dominant_at(lambda keys: [keys - 1])),
    ("zero_queries", zero_queries),
    ("tied_keys", tied_keys),
    ("large_values", uniform(1, 1, 1000)),
]


@pytest.mark.parametrize("T,past", [(96, 300), (1, 2000), (200, 0), (2048, 0)])
@pytest.mark.parametrize("name,gen", FAST_CASES, ids=[c[0] for c in FAST_CASES])
def test_attention_prefill_f16_adversarial(name, gen, T, past):
    """attention_prefill_f16 on fp16 q, K, V^T with the adversarial scores (head_dim 128, 16/8 heads); positions past
    the context hold NaN. At T 2048 (512 workgroups) the long tiles run in two parts merged through the workspace."""
    keys, mp = past + T, ((past + T + 63) // 64 + 1) * 64
    q, k, v = gen(rng(f"fast.{name}.{T}.{past}"), 2048, 1024, T, keys)
    qb = _f16(q.reshape(T, 2048))
    kb, vb = _f16(k.reshape(keys, 1024)), _f16(v.reshape(keys, 1024))
    kc = np.full((8, mp, 128), 0x7E00, np.uint16)
    vt = np.full((8, 128, mp), 0x7E00, np.uint16)
    kc[:, :keys] = kb.reshape(keys, 8, 128).transpose(1, 0, 2)
    vt[:, :, :keys] = vb.reshape(keys, 8, 128).transpose(1, 2, 0)
    vc = v_block(vt)  # the cache's 64-position blocks
    nws = attention_prefill_workspace_words(T, 8)
    s = Session({"q": (F16, qb.shape, 0, qb), "k": (F16, kc.shape, 0, kc), "v": (F16, vc.shape, 0, vc),
                 "y": (F16, qb.shape, 0, None), "ws": (U32, (nws,), 0, np.zeros(nws, np.uint32))})
    try:
        scale = float(cpuref.attention_scale(128, np.float32))
        y = _hw(s.run("attention_prefill_f16", ["y"], q="q", k_cache="k", v_cache="v", y="y", workspace="ws",
                      rows=T, past=past, q_heads=16, kv_heads=8, max_pos=mp, scale=scale)["y"])
        ref = cpuref.attention(_hw(qb).astype(np.float64), _hw(kb), _hw(vb), 16, 8, 128, past, scale)
        assert np.isfinite(y).all()
        err, rel = metrics.max_abs(y, ref), metrics.rel_l2(y, ref)
        top = max(1.0, float(np.abs(ref).max()))
        print(f"prefill f16 {name} T={T} past={past}: max-abs {err:.3g} (|ref| <= {top:.3g}), relL2 {rel:.3g}",
              flush=True)
        assert err <= 1e-2 * top and rel <= 5e-3
    finally:
        s.close()


@pytest.mark.parametrize("pos,chunks", [(150, 1), (1000, 1), (1000, 4)])
@pytest.mark.parametrize("name,gen", FAST_CASES, ids=[c[0] for c in FAST_CASES])
def test_attention_decode_f16_adversarial(name, gen, pos, chunks):
    """attention_decode_f16 + attention_combine at position pos over a cache holding the adversarial keys and values
    of positions 0 .. pos - 1; the raw projection holds the generator's query and its key and value for pos. The kernel
    RMS-normalises q and the new key, so their norm weights are the RMS of the generated rows (rounded to bf16), which
    gives the normed rows the generator's magnitudes (and q = 0 stays 0)."""
    mp = ((pos + 64) // 64 + 1) * 64
    r = rng(f"dec.{name}.{pos}")
    q, k, v = gen(r, 2048, 1024, 1, pos + 1)
    kr, vr = k.reshape(pos + 1, 1024), v.reshape(pos + 1, 1024)
    kb, vb = _f16(kr[:pos]), _f16(vr[:pos])
    kc = np.full((8, mp, 128), 0x7E00, np.uint16)
    vt = np.full((8, 128, mp), 0x7E00, np.uint16)
    kc[:, :pos] = kb.reshape(pos, 8, 128).transpose(1, 0, 2)
    vt[:, :, :pos] = vb.reshape(pos, 8, 128).transpose(1, 2, 0)
    vc = v_block(vt)  # the cache's 64-position blocks
    rms = lambda x: float(np.sqrt(np.mean(np.asarray(x, np.float64) ** 2)))
    qn = cpuref.bf16_narrow(np.full(128, rms(q), np.float32))
    kn = cpuref.bf16_narrow(np.full(128, rms(kr[pos]), np.float32))
    qkv = np.concatenate([q, kr[pos], vr[pos]]).astype(np.float32)
    state = np.array([pos, 0, 0, 0], np.uint32)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), mp)
    S = mp // 64
    s = Session({"qkv": (F32, (4096,), RO, qkv), "qn": (BF16, (128,), RO, qn), "kn": (BF16, (128,), RO, kn),
                 "cos": (F32, cos.shape, RO, cos), "sin": (F32, sin.shape, RO, sin),
                 "kc": (F16, kc.shape, 0, kc), "vc": (F16, vc.shape, 0, vc),
                 "part": (F32, (16 * S * 130,), 0, None), "y": (F32, (2048,), 0, None),
                 "state": (U32, (4,), RO, state)})
    try:
        scale = float(cpuref.attention_scale(128, np.float32))
        y = s.run_list([("attention_decode_f16", dict(qkv="qkv", q_norm="qn", k_norm="kn", cos_table="cos",
                                                      sin_table="sin", k_cache="kc", v_cache="vc", partials="part",
                                                      state="state", q_heads=16, kv_heads=8, max_pos=mp, eps=1e-6,
                                                      scale=scale, batch=1, chunks=chunks)),
                        ("attention_combine", dict(partials="part", y="y", state="state", q_heads=16, max_pos=mp,
                                                   batch=1, chunks=chunks))], ["y"], reset={"kc": kc, "vc": vc})["y"]
        q64 = qkv[None].astype(np.float64)
        qr = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(q64[:, :2048].copy(), qn, 1e-6), 16, pos)
        kc2, vc2 = s.read("kc"), v_unblock(s.read("vc"), 8, mp)
        k_new = _hw(kc2[:, pos, :]).reshape(1, 1024)
        v_new = _hw(vc2[:, :, pos]).reshape(1, 1024)
        kf = np.concatenate([_hw(kb), k_new]).astype(np.float64)
        vf = np.concatenate([_hw(vb), v_new]).astype(np.float64)
        ref = cpuref.attention(qr, kf, vf, 16, 8, 128, pos, scale)
        assert np.isfinite(y).all()
        err, rel = metrics.max_abs(y, ref), metrics.rel_l2(y, ref)
        top = max(1.0, float(np.abs(ref).max()))
        print(f"decode f16 {name} pos={pos} chunks={chunks}: max-abs {err:.3g} (|ref| <= {top:.3g}), relL2 {rel:.3g}",
              flush=True)
        assert err <= 2e-3 * top and rel <= 1e-3
    finally:
        s.close()
