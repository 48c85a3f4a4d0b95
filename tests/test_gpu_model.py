"""GPU tests of the Qwen3 executor through the C ABI against the oracle and the reference's committed goldens.

fp32 mode (the reference catalog kernels): the tiny-g1 taps against torch32 within the reference's CPU32 floors
(TinyModelTests.fs:17-23), the 64 greedy ids of both goldens, prefill == token-by-token decode bit for bit, and the
plumbing config (hd 16, vocab 512) greedy ids equal to the oracle's.
fast mode (bf16 weights, fp16 MFMA operands and KV cache): logits within max-abs 2e-2 of CpuRef F32 and top-1
agreement >= 99%, for prefill, chunked prefill and on-device decode.
"""
import numpy as np
import pytest

from conftest import golden
from oracle import cpuref, metrics
from rosylnalive_amd.gpu_core import HipBackend
from rosylnalive_amd.qwen import QwenConfig, QwenModel, inv_freq_bits, synthetic_ids, synthetic_weights

pytestmark = pytest.mark.gpu

CHAIN_REL, LOGIT_MAXABS, LOGIT_KL = 1e-5, 2e-3, 1e-7


def tiny_cfg(tiny):
    c = tiny["cfg"]
    return QwenConfig(c["layers"], c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["intermediate"],
                      c["vocab"], c["max_pos"], c["eps"])


@pytest.fixture(scope="module")
def tiny_fp32(tiny):
    m = QwenModel(HipBackend(0), tiny_cfg(tiny), mode="fp32", max_tokens=80, taps=True,
                  inv_freq=tiny["rope"]["inv_freq.bits"])
    m.load_weights(tiny["weights"])
    yield m
    m.close()
    m.backend.close()


@pytest.mark.parametrize("prompt", ["p0", "p1", "p2"])
def test_tiny_fp32_taps_match_goldens(tiny, tiny_fp32, prompt):
    g32 = golden(f"fwd_f32.{prompt}.safetensors")
    ids = g32["input_ids"].astype(np.int32)
    logits, am = tiny_fp32.forward(ids, 0)
    taps = tiny_fp32.taps(ids.size)
    names = [n for n in cpuref.tap_names(tiny["cfg"]["layers"]) if n in g32]
    worst = 0.0
    for n in names:
        r = metrics.rel_l2(taps[n], g32[n])
        worst = max(worst, r)
        assert r <= CHAIN_REL, (n, r)
    assert metrics.rel_l2(logits, g32["logits"]) <= CHAIN_REL
    assert metrics.max_abs(logits, g32["logits"]) <= LOGIT_MAXABS
    assert metrics.kl_max(logits, g32["logits"]) <= LOGIT_KL
    assert am == int(np.argmax(g32["logits"][-1]))
    print(f"{prompt}: worst tap relL2 vs torch32 {worst:.3g}", flush=True)


@pytest.mark.parametrize("prompt", ["p0", "p1"])
def test_tiny_fp32_greedy_64_equals_goldens(tiny, tiny_fp32, prompt):
    g = golden("greedy.safetensors")
    ids = golden(f"fwd_f32.{prompt}.safetensors")["input_ids"].astype(np.int32)
    out = tiny_fp32.greedy(ids, 64)
    assert out.tolist() == g[f"{prompt}.ids.torch32"].tolist()
    assert out.tolist() == g[f"{prompt}.ids.torch64p"].tolist()


def test_tiny_fp32_prefill_equals_decode_bit_for_bit(tiny, tiny_fp32):
    """Batch invariance of the catalog kernels (docs/contracts/batch-invariance.md): a prefill row equals the same
    position decoded alone, and so do the caches."""
    ids = golden("fwd_f32.p2.safetensors")["input_ids"].astype(np.int32)[:40]
    pre, _ = tiny_fp32.forward(ids, 0)
    kc = [tiny_fp32.read_cache(l, "k", 0, 40) for l in range(2)]
    for t in range(ids.size):
        row, _ = tiny_fp32.forward(ids[t:t + 1], t)
        assert row.tobytes() == pre[t:t + 1].tobytes(), t
    for l in range(2):
        assert tiny_fp32.read_cache(l, "k", 0, 40).tobytes() == kc[l].tobytes()


def test_plumbing_config_greedy_equals_oracle():
    """The plumbing config: 2 layers, hidden 64, 4/2 heads, head_dim 16, SwiGLU 192, vocab 512; N(0, 0.02) weights,
    norms 1; 16 prompt ids then 8 greedy tokens."""
    cfg = QwenConfig.tiny_plumbing(max_pos=64)
    w = synthetic_weights(cfg, seed=11)
    prompt = synthetic_ids(11, "plumbing/prompt", 16, cfg.vocab)
    cos, sin = cpuref.rope_table(inv_freq_bits(16), cfg.max_pos)
    orc = cpuref.QwenOracle(cfg.oracle_dict(), w, cos, sin)
    ref = orc.greedy(prompt, 8)
    b = HipBackend(0)
    try:
        m = QwenModel(b, cfg, mode="fp32", max_tokens=32)
        m.load_weights(w)
        got = m.greedy(prompt, 8)
        assert got.tolist() == ref.tolist()
        lg, _ = m.forward(prompt, 0)
        ol = orc.forward(orc.new_cache(), 0, prompt)
        rng_ = float(ol.max() - ol.min())
        assert metrics.max_abs(lg, ol) <= 1e-3 * rng_
        m.close()
    finally:
        b.close()


# ---------------------------------------------------------------- fast path

def reduced_0_6b(layers=2, max_pos=512):
    c = QwenConfig.qwen3_0_6b(max_pos=max_pos)
    c.layers = layers
    return c


@pytest.fixture(scope="module")
def fast_setup():
    cfg = reduced_0_6b(layers=2, max_pos=512)
    w = synthetic_weights(cfg, seed=5)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), cfg.max_pos)
    orc = cpuref.QwenOracle(cfg.oracle_dict(), w, cos, sin)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fast", max_tokens=256)
    m.load_weights(w)
    yield cfg, w, orc, m
    m.close()
    b.close()


def test_fast_weights_round_trip(fast_setup):
    cfg, w, orc, m = fast_setup
    for name in ["model.layers.1.self_attn.k_proj.weight", "model.layers.0.mlp.up_proj.weight",
                 "model.embed_tokens.weight"]:
        assert m.read_weight(name).tobytes() == w[name].tobytes()


def test_fast_rejects_weights_outside_fp16(fast_setup):
    cfg, w, orc, m = fast_setup
    name = "model.layers.0.self_attn.o_proj.weight"
    bad = w[name].copy()
    bad[3, 5] = 0x4780  # 65536: no fp16 counterpart
    with pytest.raises(Exception, match="fp16 range"):
        m.set_weight(name, bad)
    m.set_weight(name, w[name])


def test_fast_prefill_logits_within_tolerance_of_cpuref(fast_setup):
    """A 200-token fast-mode prefill against CpuRef F32: logits within 2e-2 max-abs, top-1 agreement at least 0.99,
    every top-1 disagreement a near tie (gap at most twice the max-abs error), and the returned id the last row's
    argmax."""
    cfg, w, orc, m = fast_setup
    ids = synthetic_ids(5, "fast/prompt", 200, cfg.vocab)
    lg, am = m.forward(ids, 0)
    ol = orc.forward(orc.new_cache(), 0, ids)
    err = metrics.max_abs(lg, ol)
    top1 = metrics.top1_agreement(lg, ol)
    print(f"fast prefill vs CpuRef F32: max-abs {err:.4g} (logit range {ol.min():.3g}..{ol.max():.3g}), "
          f"top-1 {top1:.4f}", flush=True)
    assert err <= 2e-2 and top1 >= 0.99 and np.all(metrics.top1_flip_gaps(lg, ol) <= 2 * err)
    assert am == int(np.argmax(lg[-1]))


def test_fast_chunked_prefill_equals_whole(fast_setup):
    cfg, w, orc, m = fast_setup
    ids = synthetic_ids(6, "fast/chunk", 300, cfg.vocab)  # 300 > max_tokens 256: two chunks
    lg, am = m.forward(ids, 0, logits_rows=300)
    ol = orc.forward(orc.new_cache(), 0, ids)
    err, top1, gaps = metrics.max_abs(lg, ol), metrics.top1_agreement(lg, ol), metrics.top1_flip_gaps(lg, ol)
    print(f"chunked prefill vs CpuRef F32: max-abs {err:.4g}, top-1 {top1:.4f}, flip gaps {gaps}", flush=True)
    assert err <= 2e-2 and top1 >= 0.99 and np.all(gaps <= 2 * err)
    assert am == int(np.argmax(lg[-1]))
    # a logits window that straddles the chunk boundary lands at the right rows
    lg2, _ = m.forward(ids, 0, logits_rows=60)
    assert np.array_equal(lg2, lg[-60:])


def test_fast_decode_on_device_matches_oracle(fast_setup):
    """Teacher-forced decode: each step's logits (the recorded HIP graph, position and token read from device
    memory) against CpuRef F32 at the same position."""
    cfg, w, orc, m = fast_setup
    prompt = synthetic_ids(7, "fast/decode", 64, cfg.vocab)
    cont = synthetic_ids(7, "fast/decode/cont", 40, cfg.vocab)
    seq = np.concatenate([prompt, cont])
    m.forward(prompt, 0, logits_rows=1)
    ol = orc.forward(orc.new_cache(), 0, seq)
    agree, worst = 0, 0.0
    for i, tok in enumerate(cont):
        pos = prompt.size + i
        m.decode_set(int(tok), pos)
        m.decode_run(1)
        lg = m.read_logits(1)
        worst = max(worst, metrics.max_abs(lg, ol[pos:pos + 1]))
        agree += int(np.argmax(lg[0]) == np.argmax(ol[pos]))
        assert int(m.decode_ids(1)[0]) == int(np.argmax(lg[0]))
    print(f"fast decode vs CpuRef F32: worst max-abs {worst:.4g}, top-1 {agree}/{cont.size}", flush=True)
    assert worst <= 2e-2 and agree >= 0.99 * cont.size - 1e-9


def test_fast_greedy_runs_on_device(fast_setup):
    cfg, w, orc, m = fast_setup
    prompt = synthetic_ids(8, "fast/greedy", 32, cfg.vocab)
    out = m.greedy(prompt, 24)
    # replaying the produced sequence through the prefill path gives the same argmax at every generated step
    seq = np.concatenate([prompt, out[:-1]])
    lg, _ = m.forward(seq, 0)
    agree = np.mean(np.argmax(lg[prompt.size - 1:], axis=1) == out)
    assert agree >= 0.95, agree


def test_fast_batched_decode_matches_oracle_per_sequence():
    """Four sequences of different lengths, each prefilled into its own cache (forward(seq=b)), then teacher-forced
    batched decode steps (skinny MFMA GEMMs over the fp16 weight copies, attention batched on the grid): every row of
    the step's logits against CpuRef F32 of that sequence at that position, and the on-device ids = the row argmax."""
    cfg = reduced_0_6b(layers=2, max_pos=256)
    w = synthetic_weights(cfg, seed=9)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), cfg.max_pos)
    orc = cpuref.QwenOracle(cfg.oracle_dict(), w, cos, sin)
    B = 4
    lens = [20, 33, 47, 64]
    steps = 6
    seqs = [synthetic_ids(50 + b, "batch/seq", lens[b] + steps, cfg.vocab) for b in range(B)]
    ref = [orc.forward(orc.new_cache(), 0, seqs[b]) for b in range(B)]
    b_ = HipBackend(0)
    m = QwenModel(b_, cfg, mode="fast", max_tokens=64, batch=B)
    try:
        m.load_weights(w)
        for b in range(B):
            m.forward(seqs[b][:lens[b]], 0, logits_rows=1, seq=b)
        worst, agree = 0.0, 0
        for s in range(steps):
            pos = [lens[b] + s for b in range(B)]
            toks = [int(seqs[b][pos[b]]) for b in range(B)]
            ids = m.decode_batch(toks, pos, 1)
            lg = m.read_logits(B)
            for b in range(B):
                o = ref[b][pos[b]]
                worst = max(worst, metrics.max_abs(lg[b], o))
                agree += int(np.argmax(lg[b]) == np.argmax(o))
                assert int(ids[0, b]) == int(np.argmax(lg[b]))
        print(f"batched decode vs CpuRef F32: worst max-abs {worst:.4g}, top-1 {agree}/{B * steps}", flush=True)
        assert worst <= 2e-2 and agree >= B * steps - 1
    finally:
        m.close()
        b_.close()


# ---------------------------------------------------------------- the persistent decode step

def _fast_model(cfg, w, kernels: bool, max_tokens: int = 64):
    """A fast-mode model whose one-sequence decode step is the persistent launch (kernels=False) or the recorded
    per-stage kernel list (kernels=True, LRM_HIP_DECODE=kernels at construction)."""
    import os
    old = os.environ.get("LRM_HIP_DECODE")
    if kernels:
        os.environ["LRM_HIP_DECODE"] = "kernels"
    else:
        os.environ.pop("LRM_HIP_DECODE", None)
    try:
        m = QwenModel(HipBackend(0), cfg, mode="fast", max_tokens=max_tokens)
    finally:
        if old is None:
            os.environ.pop("LRM_HIP_DECODE", None)
        else:
            os.environ["LRM_HIP_DECODE"] = old
    m.load_weights(w)
    return m


def test_fast_decode_runs_the_persistent_step(fast_setup):
    """The Qwen3-0.6B layer shape on an MI355X (256 CUs) decodes through decode_step_persistent."""
    cfg, w, orc, m = fast_setup
    assert m.persistent_decode()


def test_persistent_decode_step_matches_kernel_list():
    """decode_step_persistent against the per-stage kernel list on the same weights and caches: teacher-forced steps
    at short context (one split) and over random caches at positions whose splits take 1, 2 and 3 chunks of 64 keys
    (2047 and 3700: one chunk more than 32 splits need, to keep to 28 splits; 3000: 24 splits, gathered in two
    passes), then 20 greedy steps. Layer 0's appended cache rows agree to one fp16 rounding (the same per-lane products, but the
    persistent step multiplies by the fp16 copies of the matrices, which differ from the bf16 weights only for weights
    under 2^-17 in magnitude); after it the residual rows differ by the order of a few partial sums, and so do the
    logits."""
    cfg = reduced_0_6b(layers=2, max_pos=4352)
    w = synthetic_weights(cfg, seed=11)
    mp = _fast_model(cfg, w, kernels=False)
    mk = _fast_model(cfg, w, kernels=True)
    try:
        assert mp.persistent_decode() and not mk.persistent_decode()
        worst = 0.0

        def step(tok, pos):
            nonlocal worst
            lg = []
            for m in (mp, mk):
                m.decode_set(int(tok), pos)
                m.decode_run(1)
                lg.append(m.read_logits(1))
            err = metrics.max_abs(lg[0], lg[1])
            worst = max(worst, err)
            assert err <= 1e-3, (pos, err)
            assert np.all(metrics.top1_flip_gaps(lg[0], lg[1]) <= 2 * err + 1e-6), pos
            assert int(mp.decode_ids(1)[0]) == int(np.argmax(lg[0][0]))
            for layer in range(cfg.layers):
                for which in ("k", "v"):
                    a = mp.read_cache(layer, which, pos, 1)
                    b = mk.read_cache(layer, which, pos, 1)
                    if layer == 0:  # the same input row: within one fp16 rounding
                        assert np.all(np.abs(a - b) <= np.abs(b) * 2.0 ** -10 + 2.0 ** -24), (pos, layer, which)
                    else:  # the residual row entering the layer differs in the last bits
                        assert np.max(np.abs(a - b)) <= 1e-2 * max(1.0, float(np.max(np.abs(b)))), (pos, layer, which)

        prompt = synthetic_ids(11, "persist/prompt", 40, cfg.vocab)
        cont = synthetic_ids(11, "persist/cont", 6, cfg.vocab)
        for m in (mp, mk):
            m.forward(prompt, 0, logits_rows=1)
        for i, tok in enumerate(cont):
            step(tok, prompt.size + i)
        for m in (mp, mk):
            m.fill_cache_random(5, 4320)
        toks = synthetic_ids(11, "persist/long", 6, cfg.vocab)
        for tok, pos in zip(toks, (63, 2047, 2048, 3000, 3700, 4319)):
            step(tok, pos)
        print(f"persistent vs kernel-list decode: worst logits max-abs {worst:.3g}", flush=True)
        g = [m.greedy(prompt, 20) for m in (mp, mk)]
        assert g[0].tolist() == g[1].tolist(), g
    finally:
        for m in (mp, mk):
            m.close()
            m.backend.close()


def test_persistent_decode_aborts_past_its_wait_bound_and_recovers(fast_setup):
    """The failure path, forced from the host: a 1 us bound on every wait of the persistent step's workgroups
    (LRM_HIP_PERSIST_WAIT_US, read by decode_set) makes the step abort; every workgroup still ends, decode_run raises,
    and the position does not advance. decode_set with the default bound clears the abort, and the next step's logits
    match the oracle."""
    import os
    cfg, w, orc, m = fast_setup
    prompt = synthetic_ids(12, "persist/abort", 30, cfg.vocab)
    tok = int(synthetic_ids(12, "persist/abort/tok", 1, cfg.vocab)[0])
    m.forward(prompt, 0, logits_rows=1)
    os.environ["LRM_HIP_PERSIST_WAIT_US"] = "1"
    try:
        m.decode_set(tok, prompt.size)
        with pytest.raises(Exception, match="waited past its bound"):
            m.decode_run(1)
    finally:
        os.environ.pop("LRM_HIP_PERSIST_WAIT_US", None)
    m.decode_set(tok, prompt.size)
    m.decode_run(1)
    lg = m.read_logits(1)
    ol = orc.forward(orc.new_cache(), 0, np.concatenate([prompt, [tok]]).astype(np.int32))[-1:]
    assert metrics.max_abs(lg, ol) <= 2e-2
    assert int(np.argmax(lg[0])) == int(np.argmax(ol[0])) == int(m.decode_ids(1)[0])


def test_fast_hidden_1536_prefill_and_decode_match_oracle():
    """A hidden size outside the add-and-norm pass's row widths (1536): the prefill residual GEMMs run unsplit with
    a separate norm, and decode runs the per-stage list (the persistent step covers hidden 1024). Prefill logits and
    teacher-forced decode steps against CpuRef F32."""
    cfg = QwenConfig(2, 1536, 16, 8, 128, 4096, 4096, 256)
    w = synthetic_weights(cfg, seed=15)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), cfg.max_pos)
    orc = cpuref.QwenOracle(cfg.oracle_dict(), w, cos, sin)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fast", max_tokens=128)
    try:
        m.load_weights(w)
        assert not m.persistent_decode()
        ids = synthetic_ids(15, "h1536/prompt", 100, cfg.vocab)
        cont = synthetic_ids(15, "h1536/cont", 8, cfg.vocab)
        ol = orc.forward(orc.new_cache(), 0, np.concatenate([ids, cont]).astype(np.int32))
        lg, am = m.forward(ids, 0)
        err = metrics.max_abs(lg, ol[:100])
        assert err <= 2e-2 and metrics.top1_agreement(lg, ol[:100]) >= 0.99, err
        assert am == int(np.argmax(lg[-1]))
        worst = 0.0
        for i, tok in enumerate(cont):
            m.decode_set(int(tok), 100 + i)
            m.decode_run(1)
            d = m.read_logits(1)
            worst = max(worst, metrics.max_abs(d, ol[100 + i:101 + i]))
            assert int(m.decode_ids(1)[0]) == int(np.argmax(d[0]))
        print(f"hidden 1536: prefill max-abs {err:.4g}, decode worst max-abs {worst:.4g}", flush=True)
        assert worst <= 2e-2
    finally:
        m.close()
        b.close()
