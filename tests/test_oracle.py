"""Pins the oracle (oracle/cpuref.c) before anything is checked against it.

Every check here comes from outside the oracle's own formulas: the reference's contract vectors
(docs/contracts/cpu-reference.md:101-113, tests/Lrm.Tensor.Tests/CpuRefTests.fs:138-352), its committed tiny-model
goldens (goldens/tiny/g1: torch32 and torch64p taps, greedy ids, the T_spec table), its RoPE digests and entries
(tests/Lrm.Tensor.Tests/RopeTests.fs:116-190), closed forms (float64 brute force on tiny inputs) and invariants
(thread-count invariance, prefill == decode, batch invariance) chosen so a dropped term, a wrong sign, a transposed
operand or a wrong index fails at least one test.
"""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

from conftest import GOLDEN, golden
from oracle import cpuref, metrics

VEC = json.load(open(os.path.join(GOLDEN, "reference_vectors.json")))


def bits32(x):
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


def hexbits(a):
    return ["%08x" % v for v in np.asarray(a, np.float32).view(np.uint32).ravel()]


def u32(h):
    return int(h, 16)


# ---------------------------------------------------------------- contract vectors (cpu-reference.md:101-113)


def test_fused_dot_vector():
    """cpu-reference.md:107: x = (1, 1 + 2^-12), y = (-1, 1 + 2^-12) gives 2^-11 + 2^-24 (3a000400) fused, 3a000000
    unfused. Neither operand is a bf16, so the oracle's dot is probed through an attention score: key 0 is y, key 1
    scores exactly 2^-11, and with scale 2^20 the two scores are 512.0625 (fused) against 512, so the weight of key 0
    is 1 / (1 + exp(-0.0625)) = 0.5156..., where an unfused dot would give exactly 0.5."""
    e = 2.0**-12
    q = np.array([[1.0, 1.0 + e]], np.float32)
    k = np.array([[-1.0, 1.0 + e], [2.0**-11, 0.0]], np.float32)
    v = np.array([[1.0, 0.0], [0.0, 0.0]], np.float32)
    y = cpuref.attention(q, k, v, 1, 1, 2, 1, np.float32(2.0**20))
    fused = np.float32(np.float64(1.0 + e) * np.float64(1.0 + e) - 1.0)
    assert "%08x" % bits32(fused) == VEC["fused_dot"]["bits"]
    assert abs(float(y[0, 0]) - 1.0 / (1.0 + np.exp(-0.0625))) < 1e-6


def test_reduction_order_vector():
    # x = (1, 1e8, -1e8), y = (1, 1, 1): increasing index order gives 0 (summed from the end it would be 1).
    x = np.array([[1.0, 1e8, -1e8]], np.float32)
    w = cpuref.bf16_narrow(np.array([[1.0, 1.0, 1.0]], np.float32))
    assert cpuref.matmul_bf16w(x, w)[0, 0] == 0.0


def test_rmsnorm_vector():
    vec = VEC["rmsnorm"]
    w = cpuref.bf16_narrow(np.array(vec["w"], np.float32))
    y = cpuref.rmsnorm(np.array([vec["x"]], np.float32), w, 0.0)
    assert hexbits(y) == vec["y_bits"]
    r = np.float32(1.0) / np.sqrt(np.float32(12.5))
    assert "%08x" % bits32(r) == vec["r_bits"]
    y0 = cpuref.rmsnorm(np.array([vec["x"]], np.float32), np.zeros(2, np.uint16), 0.0)
    assert (y0 == 0).all(), "the weight is used as w, never 1 + w"


def test_attention_vectors():
    # cpu-reference.md:110: one head, hd 2, past 1, scale 1; q = (1, 0); k = ((0, 5), (ln 3, 7)); v = ((4, 8), (0, 4))
    q = np.array([[1.0, 0.0]])
    k = np.array([[0.0, 5.0], [np.log(3.0), 7.0]])
    v = np.array([[4.0, 8.0], [0.0, 4.0]])
    y = cpuref.attention(q, k, v, 1, 1, 2, 1, 1.0)
    np.testing.assert_allclose(y[0], [1.0, 5.0], rtol=1e-14)
    # CpuRefTests.fs:287-300: one key returns V; GQA maps head h to KV head h / group; a future NaN row is never read.
    q = np.array([[1.0, 0.0, 0.0, 1.0, 2.0, 2.0, -1.0, 0.5]])
    k = np.array([[0.5, 0.5, 1.0, -1.0], [np.nan] * 4])
    v = np.array([[10.0, 20.0, 30.0, 40.0], [np.nan] * 4])
    y = cpuref.attention(q, k, v, 4, 2, 2, 0, 1.0)
    assert y[0].tolist() == [10.0, 20.0, 10.0, 20.0, 30.0, 40.0, 30.0, 40.0]


def test_attention_scale_vectors():
    assert "%08x" % bits32(cpuref.attention_scale(128, np.float32)) == VEC["attention_scale_hd128_f32"]
    assert cpuref.attention_scale(32, np.float64) == VEC["attention_scale_hd32_f64"]


def test_embed_vectors():
    table = np.array([[0x3F80, 0x0001], [0xFF80, 0x7F81]], np.uint16)
    y = cpuref.embed(table, [1, 0])
    assert hexbits(y) == ["ff800000", "7f810000", "3f800000", "00010000"]
    with pytest.raises(cpuref.OracleError):
        cpuref.embed(table, [2])
    g = cpuref.embed_gather(table, [5])
    assert hexbits(g) == ["7fc00000", "7fc00000"]
    g64 = cpuref.embed_gather(table, [2], np.float64)
    assert ["%016x" % b for b in g64.view(np.uint64).ravel()] == ["7ff8000000000000"] * 2


def test_argmax_vectors():
    assert cpuref.argmax_rows(np.array([[1.0, 3.0, 3.0]], np.float32))[0] == 1
    assert cpuref.argmax_rows(np.array([[-0.0, 0.0]], np.float32))[0] == 0
    assert cpuref.argmax_rows(np.array([[-np.inf, -np.inf]], np.float32))[0] == 0
    r = cpuref.argmax_rows(np.array([[1.0, np.nan], [2.0, 2.0]], np.float32))
    assert r.tolist() == [0xFFFFFFFF, 0]


def test_one_hot_matmul_returns_the_widened_column():
    rng = np.random.default_rng(11)
    w = cpuref.bf16_narrow(rng.standard_normal((5, 3)).astype(np.float32) * 3)
    y = cpuref.matmul_bf16w(np.array([[0.0, 1.0, 0.0]], np.float32), w)
    assert (y[0].view(np.uint32) == (w[:, 1].astype(np.uint32) << 16)).all()
    yd = cpuref.matmul_bf16w(np.array([[0.0, 1.0, 0.0]]), w)
    assert (yd[0] == cpuref.bf16_widen(w[:, 1]).astype(np.float64)).all()


def test_bf16_narrow_vectors():
    cases = {1.0: 0x3F80, -2.0: 0xC000, 1.00390625: 0x3F80, 1.01171875: 0x3F82, np.inf: 0x7F80, 3.4e38: 0x7F80}
    for x, b in cases.items():
        assert int(cpuref.bf16_narrow(np.array([x], np.float32))[0]) == b, x
        assert cpuref.lib().orc_bf16_narrow_rne(x) == b
    assert int(cpuref.bf16_narrow(np.array([np.float32(-np.nan)]))[0]) in (0xFFC0, 0x7FC0)
    # every non-NaN bf16 round-trips through widen (exhaustive)
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    keep = (allb & 0x7FFF) <= 0x7F80
    rt = cpuref.bf16_narrow(cpuref.bf16_widen(allb[keep]))
    assert (rt == allb[keep]).all()


# ---------------------------------------------------------------- brute force on tiny inputs (closed forms)


def test_matmul_is_the_textbook_fused_dot():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((7, 33)).astype(np.float32)
    w = cpuref.bf16_narrow(rng.standard_normal((70, 33)).astype(np.float32))
    y = cpuref.matmul_bf16w(x, w)
    wf = cpuref.bf16_widen(w).astype(np.float64)
    ref = np.zeros((7, 70), np.float32)
    for i in range(7):
        for j in range(70):
            acc = np.float32(0)
            for p in range(33):
                acc = np.float32(np.float64(x[i, p]) * wf[j, p] + np.float64(acc))  # exact product, one rounding
            ref[i, j] = acc
    assert (y.view(np.uint32) == ref.view(np.uint32)).all()
    # the transposed operand would differ
    assert not np.allclose(cpuref.matmul_bf16w(x, w), x @ cpuref.bf16_widen(w)[:, :].T[:, ::-1])


def test_attention_brute_force_float64():
    rng = np.random.default_rng(5)
    qh, kvh, hd, past, rows = 4, 2, 8, 5, 3
    q = rng.standard_normal((rows, qh * hd))
    k = rng.standard_normal((past + rows, kvh * hd))
    v = rng.standard_normal((past + rows, kvh * hd))
    scale = 1 / np.sqrt(hd)
    y = cpuref.attention(q, k, v, qh, kvh, hd, past, scale)
    for i in range(rows):
        for h in range(qh):
            kv = h // (qh // kvh)
            kk = k[: past + i + 1, kv * hd : (kv + 1) * hd]
            vv = v[: past + i + 1, kv * hd : (kv + 1) * hd]
            s = kk @ q[i, h * hd : (h + 1) * hd] * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            np.testing.assert_allclose(y[i, h * hd : (h + 1) * hd], p @ vv, rtol=1e-12, atol=1e-13)


def test_rmsnorm_rope_silu_closed_forms_float64():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((6, 16))
    w = cpuref.bf16_narrow(rng.standard_normal(16).astype(np.float32))
    y = cpuref.rmsnorm(x, w, 1e-6)
    wf = cpuref.bf16_widen(w).astype(np.float64)
    np.testing.assert_allclose(y, wf * x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6), rtol=1e-13)
    g, u = rng.standard_normal(50) * 4, rng.standard_normal(50)
    np.testing.assert_allclose(cpuref.silu_mul(g, u), g / (1 + np.exp(-g)) * u, rtol=1e-14)
    cos, sin = cpuref.rope_table(np.array([0x3F800000, 0x3E800000], np.uint32), 8)
    xr = rng.standard_normal((3, 2 * 4))
    yr = cpuref.rope_apply(cos, sin, xr, 2, 4)
    for t in range(3):
        for h in range(2):
            a = xr[t, h * 4 : h * 4 + 2]
            b = xr[t, h * 4 + 2 : h * 4 + 4]
            c = cos[4 + t].astype(np.float64)
            s = sin[4 + t].astype(np.float64)
            np.testing.assert_allclose(yr[t, h * 4 : h * 4 + 2], a * c - b * s, rtol=1e-14)
            np.testing.assert_allclose(yr[t, h * 4 + 2 : h * 4 + 4], b * c + a * s, rtol=1e-14)


# ---------------------------------------------------------------- RoPE (RopeTests.fs:116-190)


def _qwen_inv():
    return np.array([u32(h) for h in VEC["qwen_inv_freq_hd128"]], np.uint32)


def test_inv_freq_hashes(tiny):
    assert hashlib.sha256(_qwen_inv().tobytes()).hexdigest() == VEC["qwen_inv_freq_sha256"]
    bits = tiny["rope"]["inv_freq.bits"]
    assert hashlib.sha256(bits.tobytes()).hexdigest() == VEC["tiny_inv_freq_sha256"]
    # head_dim 32 word j is head_dim 128 word 4j (theta^(-2j/32) = theta^(-8j/128), the same float32 exponent)
    assert (bits == _qwen_inv()[::4]).all()


def test_tiny_table_equals_golden_and_digest(tiny):
    r = tiny["rope"]
    assert (tiny["cos"].view(np.uint32) == r["t_spec.cos"].view(np.uint32)).all()
    assert (tiny["sin"].view(np.uint32) == r["t_spec.sin"].view(np.uint32)).all()
    d = hashlib.sha256(tiny["cos"].tobytes() + tiny["sin"].tobytes()).hexdigest()
    assert d == VEC["tiny_table_digest_512"]


@pytest.fixture(scope="module")
def qwen_table():
    return cpuref.rope_table(_qwen_inv(), 8192)


def test_qwen_table_digest(qwen_table):
    cos, sin = qwen_table
    assert hashlib.sha256(cos.tobytes() + sin.tobytes()).hexdigest() == VEC["qwen_table_digest_8192"]


def test_table_entries(tiny, qwen_table):
    tables = {"tiny": (tiny["cos"], tiny["sin"]), "qwen": qwen_table}
    for name, pos, j, c, s in VEC["entries"]:
        cos, sin = tables[name]
        assert ("%08x" % cos.view(np.uint32)[pos, j], "%08x" % sin.view(np.uint32)[pos, j]) == (c, s)


def test_exact_cos_sin_special_arguments():
    c, s = cpuref.cos_sin_exact(1.0)
    assert ["%016x" % struct.unpack("<Q", struct.pack("<d", v))[0] for v in (c, s)] == VEC["cos_sin_1_f64"]
    assert cpuref.cos_sin_exact(0.0) == (1.0, 0.0)
    c, s = cpuref.cos_sin_exact(-0.0)
    assert np.signbit(s)
    t = 2.0**-30
    assert cpuref.cos_sin_exact(t) == (1.0, t)
    c, s = cpuref.cos_sin_exact(float("nan"))
    assert np.isnan(c) and np.isnan(s)
    c, s = cpuref.cos_sin_exact(1e30)
    assert abs(c * c + s * s - 1) < 1e-15
    rng = np.random.default_rng(1)
    for x in rng.uniform(-2**14, 2**14, 200).astype(np.float32):
        c, s = cpuref.cos_sin_exact(float(x))
        assert abs(c - np.cos(np.float64(x))) <= np.spacing(abs(c)) and abs(s - np.sin(np.float64(x))) <= np.spacing(abs(s))
        assert cpuref.cos_sin_exact(float(-x)) == (c, -s)


def test_rope_table_rejects_bad_inputs():
    with pytest.raises(cpuref.OracleError):
        cpuref.rope_table(np.array([0x7F800000], np.uint32), 4)
    with pytest.raises(cpuref.OracleError):
        cpuref.rope_table(np.array([0x3F800000], np.uint32), 0)


# ---------------------------------------------------------------- tiny-model goldens (TinyModelTests.fs:17-334)

F64_OP_BOUND, F32_OP_BOUND = 1e-12, 1e-6
CHAIN_REL, LOGIT_MAXABS, LOGIT_KL = 1e-5, 2e-3, 1e-7


@pytest.mark.parametrize("prompt", ["p0", "p1"])
@pytest.mark.parametrize("mode", ["f32", "f64"])
def test_per_op_against_goldens(tiny, prompt, mode):
    """Each op fed the torch oracle's own input taps (TinyModelTests.fs:39-129)."""
    dt, gname, bound = (np.float32, "fwd_f32", F32_OP_BOUND) if mode == "f32" else (np.float64, "fwd_f64p", F64_OP_BOUND)
    g = golden(f"{gname}.{prompt}.safetensors")
    c, W = tiny["cfg"], tiny["weights"]
    eps = c["eps"]
    scale = cpuref.attention_scale(c["head_dim"], dt)
    tap = lambda n: g[n].astype(dt)
    worst = []

    def check(name, got):
        r = metrics.rel_l2(got, g[name])
        worst.append((r, name))
        assert r <= bound, (name, r)

    check("embed.out", cpuref.embed(W["model.embed_tokens.weight"], g["input_ids"], dt))
    for i in range(c["layers"]):
        p = f"L{i}."
        lw = lambda n: W[f"model.layers.{i}.{n}"]
        x = tap("embed.out" if i == 0 else f"L{i - 1}.out")
        check(p + "input_layernorm.out", cpuref.rmsnorm(x, lw("input_layernorm.weight"), eps))
        h = tap(p + "input_layernorm.out")
        check(p + "attn.q_proj.out", cpuref.matmul_bf16w(h, lw("self_attn.q_proj.weight")))
        check(p + "attn.k_proj.out", cpuref.matmul_bf16w(h, lw("self_attn.k_proj.weight")))
        check(p + "attn.v_proj.out", cpuref.matmul_bf16w(h, lw("self_attn.v_proj.weight")))
        check(p + "attn.q_norm.out", cpuref.rmsnorm(tap(p + "attn.q_proj.out"), lw("self_attn.q_norm.weight"), eps))
        check(p + "attn.k_norm.out", cpuref.rmsnorm(tap(p + "attn.k_proj.out"), lw("self_attn.k_norm.weight"), eps))
        check(p + "attn.q_rope", cpuref.rope_apply(tiny["cos"], tiny["sin"], tap(p + "attn.q_norm.out"), c["heads"], 0))
        check(p + "attn.k_rope", cpuref.rope_apply(tiny["cos"], tiny["sin"], tap(p + "attn.k_norm.out"), c["kv_heads"], 0))
        check(p + "attn.v_cache", tap(p + "attn.v_proj.out"))
        check(p + "attn.o_proj.in", cpuref.attention(tap(p + "attn.q_rope"), tap(p + "attn.k_rope"), tap(p + "attn.v_cache"),
                                                     c["heads"], c["kv_heads"], c["head_dim"], 0, scale))
        check(p + "attn.o_proj.out", cpuref.matmul_bf16w(tap(p + "attn.o_proj.in"), lw("self_attn.o_proj.weight")))
        check(p + "resid_mid", cpuref.add(x, tap(p + "attn.o_proj.out")))
        check(p + "post_attention_layernorm.out", cpuref.rmsnorm(tap(p + "resid_mid"), lw("post_attention_layernorm.weight"), eps))
        h2 = tap(p + "post_attention_layernorm.out")
        check(p + "mlp.gate.out", cpuref.matmul_bf16w(h2, lw("mlp.gate_proj.weight")))
        check(p + "mlp.up.out", cpuref.matmul_bf16w(h2, lw("mlp.up_proj.weight")))
        check(p + "mlp.down.in", cpuref.silu_mul(tap(p + "mlp.gate.out"), tap(p + "mlp.up.out")))
        check(p + "mlp.down.out", cpuref.matmul_bf16w(tap(p + "mlp.down.in"), lw("mlp.down_proj.weight")))
        check(p + "out", cpuref.add(tap(p + "resid_mid"), tap(p + "mlp.down.out")))
    check("final_norm.out", cpuref.rmsnorm(tap(f"L{c['layers'] - 1}.out"), W["model.norm.weight"], eps))
    check("logits", cpuref.matmul_bf16w(tap("final_norm.out"), W["model.embed_tokens.weight"]))
    assert len(worst) == 3 + 18 * c["layers"]


@pytest.mark.parametrize("prompt", ["p0", "p1"])
def test_chain_against_goldens(tiny, prompt):
    """The whole forward from the ids (TinyModelTests.fs:243-302)."""
    m = tiny["oracle"]
    g32 = golden(f"fwd_f32.{prompt}.safetensors")
    g64 = golden(f"fwd_f64p.{prompt}.safetensors")
    names = cpuref.tap_names(tiny["cfg"]["layers"])
    lg, taps = m.forward(m.new_cache(np.float64), 0, g32["input_ids"], np.float64, taps=True)
    for n in names:
        assert metrics.rel_l2(taps[n], g64[n]) <= F64_OP_BOUND, n
    lg, taps = m.forward(m.new_cache(np.float32), 0, g32["input_ids"], np.float32, taps=True)
    for n in names:
        assert metrics.rel_l2(taps[n], g32[n]) <= CHAIN_REL, n
        assert metrics.rel_l2(taps[n], g64[n]) <= CHAIN_REL, n
    assert metrics.max_abs(taps["logits"], g32["logits"]) <= LOGIT_MAXABS
    assert metrics.kl_max(taps["logits"], g32["logits"]) <= LOGIT_KL


def test_p2_logits_across_a_64_key_block(tiny):
    m = tiny["oracle"]
    g32, g64 = golden("fwd_f32.p2.safetensors"), golden("fwd_f64p.p2.safetensors")
    ids = g32["input_ids"]
    assert ids.size == 70
    assert metrics.rel_l2(m.forward(m.new_cache(np.float64), 0, ids, np.float64), g64["logits"]) <= F64_OP_BOUND
    assert metrics.rel_l2(m.forward(m.new_cache(np.float32), 0, ids, np.float32), g32["logits"]) <= CHAIN_REL


@pytest.mark.parametrize("prompt", ["p0", "p1"])
def test_greedy_64_steps_equal_both_oracles(tiny, prompt):
    g = golden("greedy.safetensors")
    ids = golden(f"fwd_f32.{prompt}.safetensors")["input_ids"]
    m = tiny["oracle"]
    assert (m.greedy(ids, 64, np.float32) == g[f"{prompt}.ids.torch32"]).all()
    assert (m.greedy(ids, 64, np.float64) == g[f"{prompt}.ids.torch64p"]).all()


# ---------------------------------------------------------------- invariants


def test_thread_count_invariance(tiny):
    m = tiny["oracle"]
    ids = golden("fwd_f32.p2.safetensors")["input_ids"]
    old = cpuref.threads()
    try:
        out = {}
        for n in (1, 7):
            cpuref.set_threads(n)
            for dt in (np.float32, np.float64):
                _, taps = m.forward(m.new_cache(dt), 0, ids, dt, taps=True)
                out[(n, dt)] = taps
        for dt in (np.float32, np.float64):
            for name, a in out[(1, dt)].items():
                assert a.tobytes() == out[(7, dt)][name].tobytes(), name
    finally:
        cpuref.set_threads(old)


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_prefill_equals_token_by_token_decode(tiny, dt):
    m = tiny["oracle"]
    ids = golden("fwd_f32.p2.safetensors")["input_ids"]
    pc = m.new_cache(dt)
    pre = m.forward(pc, 0, ids, dt)
    dc = m.new_cache(dt)
    for t in range(ids.size):
        step = m.forward(dc, t, ids[t : t + 1], dt)
        assert step.tobytes() == pre[t : t + 1].tobytes(), t
    assert pc[0].tobytes() == dc[0].tobytes() and pc[1].tobytes() == dc[1].tobytes()


@pytest.mark.parametrize("t", [1, 7, 33])
def test_rows_do_not_depend_on_the_batch(t):
    rng = np.random.default_rng(t)
    x = rng.standard_normal((t, 48)).astype(np.float32)
    w = cpuref.bf16_narrow(rng.standard_normal((70, 48)).astype(np.float32))
    nw = cpuref.bf16_narrow(rng.standard_normal(48).astype(np.float32))
    y = cpuref.matmul_bf16w(x, w)
    yn = cpuref.rmsnorm(x, nw, 1e-6)
    for r in range(t):
        assert cpuref.matmul_bf16w(x[r : r + 1], w).tobytes() == y[r : r + 1].tobytes()
        assert cpuref.rmsnorm(x[r : r + 1], nw, 1e-6).tobytes() == yn[r : r + 1].tobytes()
    # attention: each row equals a decode step over the same cache, and a chunked prefill equals the whole
    qh, kvh, hd = 4, 2, 16
    q = rng.standard_normal((t, qh * hd)).astype(np.float32)
    k = rng.standard_normal((t, kvh * hd)).astype(np.float32)
    v = rng.standard_normal((t, kvh * hd)).astype(np.float32)
    full = cpuref.attention(q, k, v, qh, kvh, hd, 0, np.float32(0.25))
    for r in range(t):
        one = cpuref.attention(q[r : r + 1], k, v, qh, kvh, hd, r, np.float32(0.25))
        assert one.tobytes() == full[r : r + 1].tobytes()


def test_metrics_kernel_bound_vectors():
    """KernelBounds vectors (kernel-bounds.md 'Vectors')."""
    assert metrics.relative_bound(1e-9) == 1e-6
    assert metrics.relative_bound(3e-6) == 6e-6
    assert np.isnan(metrics.relative_bound(float("nan")))
    r64 = np.array([1e-39, -2e-39])
    chk = metrics.check_relative(np.zeros(2), r64, r64)
    assert chk["passed"] and chk["measured"] == 1.0
    chk = metrics.check_relative(np.array([0.5, 0.0]), np.array([1.0, 1e-39]), np.array([1.0, 1e-39]))
    assert not chk["passed"]


# ---------------------------------------------------------------- softmax, logSumExp and KL (Rows.fs:84-135,275-292)


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_softmax_logsumexp_kl_known_answers(dt):
    """CpuRefTests.fs:168-180: softmax (0, 0) = (1/2, 1/2); logSumExp (0, 0) = log 2; a NaN spreads over the softmax
    row; KL((0, 0) || (0, log 3)) = log(4/3) / 2."""
    y = cpuref.softmax_rows(np.array([[0.0, 0.0]], dt))
    assert y[0].tolist() == [0.5, 0.5]
    assert cpuref.logsumexp_rows(np.array([[0.0, 0.0]], dt))[0] == dt(np.log(2.0))
    assert np.isnan(cpuref.softmax_rows(np.array([[1.0, np.nan]], dt))).all()
    kl = cpuref.kl_rows(np.array([[0.0, 0.0]], dt), np.array([[0.0, np.log(3.0)]], dt))[0]
    tol = (1e-15, 1e-14) if dt == np.float64 else (1e-7, 1e-6)
    assert abs(float(kl) - 0.5 * np.log(4.0 / 3.0)) <= tol[0] + tol[1] * 0.5 * np.log(4.0 / 3.0)


def test_logsumexp_and_kl_with_infinite_logits():
    """CpuRefTests.fs:182-211: an infinite row maximum is the answer; a NaN beats +inf; a logit masked in both rows
    adds nothing to KL; P with mass where Q has none gives +inf; a NaN spreads."""
    lse = lambda r, dt=np.float64: cpuref.logsumexp_rows(np.array([r], dt))[0]
    assert lse([1.0, np.inf]) == np.inf
    assert lse([-np.inf, -np.inf]) == -np.inf
    assert lse([-np.inf, 0.0], np.float32) == 0.0
    assert np.isnan(lse([np.inf, np.nan]))
    assert np.isnan(lse([np.nan, -np.inf]))
    kl = lambda p, q, dt=np.float64: cpuref.kl_rows(np.array([p], dt), np.array([q], dt))[0]
    p, q = [1.0, -np.inf, 0.0], [1.0, -np.inf, 0.5]
    finite = kl(p, q)
    assert np.isfinite(finite) and finite > 0.0
    assert finite == kl([1.0, 0.0], [1.0, 0.5])
    # Metrics.klRow (candidate q, reference p): sum_i P_i (log P_i - log Q_i) over the unmasked entries, in float64
    lp = np.array([1.0, 0.0]) - np.log(np.exp(1.0) + np.exp(0.0))
    lq = np.array([1.0, 0.5]) - np.log(np.exp(1.0) + np.exp(0.5))
    closed = float(np.sum(np.exp(lp) * (lp - lq)))
    assert abs(finite - closed) <= 1e-15 + 1e-13 * closed
    assert np.isfinite(kl(p, q, np.float32))
    assert kl([0.0, 0.0], [0.0, -np.inf]) == np.inf
    assert np.isnan(kl([0.0, np.nan], [0.0, 0.0]))


def test_softmax_logsumexp_kl_against_float64_closed_forms():
    """Random rows with a wide logit spread (a shifted maximum, large and small entries) against the textbook forms
    in float64: softmax rows sum to 1 and equal exp(x - max) / sum; logSumExp equals scipy's; KL equals
    sum p (log p - log q), is 0 for identical rows and changes under a swap of P and Q (the operand order is pinned)."""
    from scipy.special import logsumexp

    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 300)) * 8.0 + 40.0
    q = x + rng.standard_normal((6, 300))
    for dt, tol in ((np.float64, 1e-13), (np.float32, 2e-5)):
        xs, qs = x.astype(dt), q.astype(dt)
        xd = xs.astype(np.float64)
        ref = np.exp(xd - xd.max(axis=1, keepdims=True))
        ref /= ref.sum(axis=1, keepdims=True)
        sm = cpuref.softmax_rows(xs).astype(np.float64)
        assert np.max(np.abs(sm - ref)) <= tol * ref.max()
        assert np.allclose(sm.sum(axis=1), 1.0, atol=10 * tol)
        assert np.allclose(cpuref.logsumexp_rows(xs), logsumexp(xd, axis=1), rtol=tol, atol=0)
        qd = qs.astype(np.float64)
        lp = xd - logsumexp(xd, axis=1, keepdims=True)
        lq = qd - logsumexp(qd, axis=1, keepdims=True)
        klr = np.sum(np.exp(lp) * (lp - lq), axis=1)
        kl = cpuref.kl_rows(xs, qs).astype(np.float64)
        assert np.allclose(kl, klr, rtol=50 * tol, atol=1e-12 if dt == np.float64 else 5e-5)
        assert np.all(cpuref.kl_rows(xs, xs) == 0)
        swapped = cpuref.kl_rows(qs, xs).astype(np.float64)
        assert np.max(np.abs(swapped - kl)) > 1e-3
