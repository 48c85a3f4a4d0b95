"""The fast path's fp16 range monitor: a value it narrows to fp16 (normed hidden rows, q, the K/V cache, the attention
and SwiGLU outputs) that overflows makes the forward or decode call fail with Fp16RangeError naming the site, instead
of passing inf on into logits the caller would take as results; a forward whose SwiGLU output overflows first runs
again with that output shifted down (stored as a 2^-s, the down_proj sums scaled by 2^s). The overflows are forced from the host through the
weights (data only: every kernel still runs to its end), and the same model then runs clean again, bit for bit.
"""
import numpy as np
import pytest

from oracle import cpuref, metrics
from rosylnalive_amd.gpu_core import Fp16RangeError, HipBackend
from rosylnalive_amd.qwen import QwenConfig, QwenModel, inv_freq_bits, synthetic_ids, synthetic_weights

pytestmark = pytest.mark.gpu

CFG = QwenConfig(2, 1024, 16, 8, 128, 3072, 4096, 256)


def bf16(x, shape):
    return cpuref.bf16_narrow(np.broadcast_to(np.float32(x), shape).copy())


@pytest.fixture(scope="module")
def model():
    b = HipBackend(0)
    m = QwenModel(b, CFG, mode="fast", max_tokens=64)
    w = synthetic_weights(CFG, seed=23)
    m.load_weights(w)
    yield m, w
    m.close()
    b.close()


def _clean_forward(m, ids):
    lg, am = m.forward(ids, 0)
    assert np.isfinite(lg).all()
    return lg, am


def _swiglu_outlier(w, value):
    """gate and up rows 0 .. 63 all +value and rows 64 .. 127 all -value in layer 1, after a post-attention norm of 30:
    for either sign of a row's sum one half of those columns has gate = up ~ 30 value sum(normed x), so silu(gate) up
    runs far past 65,504 while h (|h| ~ 30) and the float32 reference stay finite."""
    gname, uname = "model.layers.1.mlp.gate_proj.weight", "model.layers.1.mlp.up_proj.weight"
    nname = "model.layers.1.post_attention_layernorm.weight"
    g, u = w[gname].copy(), w[uname].copy()
    for a in (g, u):
        a[:64] = bf16(value, (64, CFG.hidden))
        a[64:128] = bf16(-value, (64, CFG.hidden))
    return {gname: g, uname: u, nname: bf16(30.0, (CFG.hidden,))}


def _swiglu_spikes(w):
    """Layer 1: post-attention norm weights of 500 on hidden columns 0 .. 63 (|h| there up to about 2,000), gate and
    up rows 0 .. 63 the unit rows of those columns, and those columns zeroed in every other gate / up row. SwiGLU
    outputs 0 .. 63 are then silu(h_c) h_c, about h_c^2 (up to ~4e6) for positive h_c: past 65,504 at shift 0 and
    within range at shift 8, with no cancelling sum in front of them (every value keeps fp16's relative precision),
    while the other outputs keep their usual size."""
    gname, uname = "model.layers.1.mlp.gate_proj.weight", "model.layers.1.mlp.up_proj.weight"
    nname = "model.layers.1.post_attention_layernorm.weight"
    one = bf16(1.0, (1,))[0]
    out = {}
    for name in (gname, uname):
        a = w[name].copy()
        a[:, :64] = 0
        a[np.arange(64), np.arange(64)] = one
        out[name] = a
    nw = w[nname].copy()
    nw[:64] = bf16(500.0, (64,))
    out[nname] = nw
    return out


def test_swiglu_outlier_reruns_the_forward_shifted(model):
    """SwiGLU outputs past the fp16 range: the forward runs again with them stored 2^-8 scaled and the down_proj sums
    scaled back, and its logits meet the fast path's bound against the float32 oracle on the same weights (max-abs
    2e-2, top-1 >= 99 %). The shift stays for the next forward (same logits, bit for bit) and goes back to 0 when a
    weight is written: the restored model runs as before, bit for bit."""
    m, w = model
    ids = synthetic_ids(23, "range/prompt", 48, CFG.vocab)
    base, am = _clean_forward(m, ids)
    assert m.swiglu_shift() == 0
    bad = _swiglu_spikes(w)
    w2 = dict(w)
    w2.update(bad)
    try:
        for n, v in bad.items():
            m.set_weight(n, v)
        lg, am2 = m.forward(ids, 0, logits_rows=48)
        shift = m.swiglu_shift()
        lg2, _ = m.forward(ids, 0, logits_rows=48)
        assert m.swiglu_shift() == shift and lg2.tobytes() == lg.tobytes()
    finally:
        for n in bad:
            m.set_weight(n, w[n])
    assert m.swiglu_shift() == 0
    cos, sin = cpuref.rope_table(inv_freq_bits(128), CFG.max_pos)
    orc = cpuref.QwenOracle(CFG.oracle_dict(), w2, cos, sin)
    ol = orc.forward(orc.new_cache(), 0, ids)
    err, top1 = metrics.max_abs(lg, ol), metrics.top1_agreement(lg, ol)
    print(f"SwiGLU outlier: shift {shift}, max-abs {err:.4g} (logit range {ol.min():.3g}..{ol.max():.3g}), "
          f"top-1 {top1:.4f}", flush=True)
    assert shift == 8
    assert err <= 2e-2 and top1 >= 0.99 and am2 == int(np.argmax(lg[-1]))
    lg3, am3 = _clean_forward(m, ids)
    assert lg3.tobytes() == base.tobytes() and am3 == am


def test_swiglu_outlier_past_the_largest_shift_fails_and_names_the_site(model):
    """Gate and up rows of 100 after a norm of 30 take the SwiGLU output to ~9e10, past 65,504 x 2^16: the forward
    fails with Fp16RangeError naming the site after its reruns at shifts 8 and 16; the restored model runs as before,
    bit for bit."""
    m, w = model
    ids = synthetic_ids(23, "range/prompt", 48, CFG.vocab)
    base, am = _clean_forward(m, ids)
    bad = _swiglu_outlier(w, 100.0)
    try:
        for n, v in bad.items():
            m.set_weight(n, v)
        with pytest.raises(Fp16RangeError) as e:
            m.forward(ids, 0)
        print(e.value, flush=True)
        assert "SwiGLU output (a)" in str(e.value)
        assert m.swiglu_shift() == 16
    finally:
        for n in bad:
            m.set_weight(n, w[n])
    lg, am2 = _clean_forward(m, ids)  # the words were cleared: the same call runs clean, bit for bit
    assert lg.tobytes() == base.tobytes() and am2 == am


def test_hidden_overflow_fails_the_forward(model):
    """An input norm weight of 30,000: the normed rows (|x / rms| reaches 3 or more) overflow."""
    m, w = model
    ids = synthetic_ids(23, "range/prompt2", 32, CFG.vocab)
    base, _ = _clean_forward(m, ids)
    name = "model.layers.0.input_layernorm.weight"
    try:
        m.set_weight(name, bf16(30000.0, (CFG.hidden,)))
        with pytest.raises(Fp16RangeError) as e:
            m.forward(ids, 0)
        assert "normed hidden rows (h)" in str(e.value)
    finally:
        m.set_weight(name, w[name])
    lg, _ = _clean_forward(m, ids)
    assert lg.tobytes() == base.tobytes()


def test_cache_overflow_fails_the_decode(model):
    """Prefill clean, then a k_norm weight of 30,000 in layer 0: the key that the decode step appends to the fp16
    cache overflows, and decode_run fails naming the cache. Restored, the next steps run clean."""
    m, w = model
    ids = synthetic_ids(23, "range/prompt3", 40, CFG.vocab)
    _, am = _clean_forward(m, ids)
    name = "model.layers.0.self_attn.k_norm.weight"
    try:
        m.set_weight(name, bf16(30000.0, (CFG.head_dim,)))
        m.decode_set(am, ids.size)
        with pytest.raises(Fp16RangeError) as e:
            m.decode_run(1)
        print(e.value, flush=True)
        assert "K/V cache" in str(e.value)
    finally:
        m.set_weight(name, w[name])
    _clean_forward(m, ids)
    m.decode_set(am, ids.size)
    m.decode_run(4)
    assert np.isfinite(m.read_logits(1)).all()


def test_batched_decode_overflow_raises_the_shift_for_the_steps_after_it():
    """Batched decode (two sequences; its skinny SwiGLU GEMM stores fp16), prefilled on the clean weights, then the
    spike weights set (layer 1's MLP only: the prefilled caches are those of the new weights too). The first step
    fails naming the SwiGLU output and raises the shift to 8; that step again and the ones after it run shifted, each
    sequence's logits against the float32 oracle on the new weights at that position."""
    w = synthetic_weights(CFG, seed=23)
    bad = _swiglu_spikes(w)
    w2 = dict(w)
    w2.update(bad)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), CFG.max_pos)
    orc = cpuref.QwenOracle(CFG.oracle_dict(), w2, cos, sin)
    B, lens, steps = 2, [20, 33], 4
    seqs = [synthetic_ids(60 + b, "range/batch", lens[b] + steps, CFG.vocab) for b in range(B)]
    ref = [orc.forward(orc.new_cache(), 0, seqs[b]) for b in range(B)]
    b_ = HipBackend(0)
    m = QwenModel(b_, CFG, mode="fast", max_tokens=64, batch=B)
    try:
        m.load_weights(w)
        for b in range(B):
            m.forward(seqs[b][:lens[b]], 0, logits_rows=1, seq=b)
        for n, v in bad.items():
            m.set_weight(n, v)
        with pytest.raises(Fp16RangeError) as e:
            m.decode_batch([int(seqs[b][lens[b]]) for b in range(B)], lens, 1)
        print(e.value, flush=True)
        assert "SwiGLU output (a)" in str(e.value) and m.swiglu_shift() == 8
        worst, agree = 0.0, 0
        for s in range(steps):
            pos = [lens[b] + s for b in range(B)]
            ids = m.decode_batch([int(seqs[b][pos[b]]) for b in range(B)], pos, 1)
            lg = m.read_logits(B)
            for b in range(B):
                o = ref[b][pos[b]]
                worst = max(worst, metrics.max_abs(lg[b], o))
                agree += int(np.argmax(lg[b]) == np.argmax(o))
                assert int(ids[0, b]) == int(np.argmax(lg[b]))
        print(f"shifted batched decode vs the oracle: worst max-abs {worst:.4g}, top-1 {agree}/{B * steps}",
              flush=True)
        assert m.swiglu_shift() == 8 and worst <= 2e-2 and agree >= B * steps - 1
    finally:
        m.close()
        b_.close()


def test_set_swiglu_shift_ahead(model):
    """A shift set ahead (for a checkpoint whose range is known): on the clean model shift 8 changes only the SwiGLU
    outputs under 2^-6 (kept to 2^-17 absolute instead of fp16's relative precision), so the logits move by a small
    part of the fast path's bound and stay within it against the float32 oracle; the setter refuses values outside
    0 .. 24, and writing a weight sets it back to 0."""
    m, w = model
    ids = synthetic_ids(23, "range/prompt4", 48, CFG.vocab)
    base, _ = m.forward(ids, 0, logits_rows=48)
    m.set_swiglu_shift(8)
    assert m.swiglu_shift() == 8
    lg, _ = m.forward(ids, 0, logits_rows=48)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), CFG.max_pos)
    orc = cpuref.QwenOracle(CFG.oracle_dict(), w, cos, sin)
    ol = orc.forward(orc.new_cache(), 0, ids)
    d, e0, e8 = (float(np.abs(lg - base).max()), metrics.max_abs(base, ol), metrics.max_abs(lg, ol))
    print(f"clean model, shift 8 against shift 0: max-abs {d:.3g}; against the oracle: {e0:.4g} (shift 0), "
          f"{e8:.4g} (shift 8)", flush=True)
    assert 0 < d <= 5e-3 and e8 <= 2e-2 and metrics.top1_agreement(lg, ol) >= 0.99
    for bad in (-1, 25):
        with pytest.raises(Exception, match="outside 0 .. 24"):
            m.set_swiglu_shift(bad)
    assert m.swiglu_shift() == 8
    name = "model.layers.0.mlp.down_proj.weight"
    m.set_weight(name, w[name])
    assert m.swiglu_shift() == 0
    lg0, _ = m.forward(ids, 0, logits_rows=48)
    assert lg0.tobytes() == base.tobytes()


def test_chunked_shifted_prefill_then_decode_match_the_oracle(model):
    """The spike weights with a 150-token prompt (three chunks of max_tokens 64): the whole call reruns shifted and its
    logits meet the bound against the oracle; then one-sequence decode steps (whose SwiGLU output stays float32),
    teacher-forced, against the oracle's rows at those positions. The restored model runs as before."""
    m, w = model
    prompt = synthetic_ids(23, "range/chunked", 150, CFG.vocab)
    cont = synthetic_ids(23, "range/chunked/cont", 6, CFG.vocab)
    bad = _swiglu_spikes(w)
    w2 = dict(w)
    w2.update(bad)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), CFG.max_pos)
    orc = cpuref.QwenOracle(CFG.oracle_dict(), w2, cos, sin)
    ol = orc.forward(orc.new_cache(), 0, np.concatenate([prompt, cont]))
    try:
        for n, v in bad.items():
            m.set_weight(n, v)
        lg, _ = m.forward(prompt, 0, logits_rows=150)
        assert m.swiglu_shift() == 8
        err, top1 = metrics.max_abs(lg, ol[:150]), metrics.top1_agreement(lg, ol[:150])
        worst = 0.0
        for i, tok in enumerate(cont):
            pos = prompt.size + i
            m.decode_set(int(tok), pos)
            m.decode_run(1)
            worst = max(worst, metrics.max_abs(m.read_logits(1), ol[pos:pos + 1]))
        print(f"chunked shifted prefill: max-abs {err:.4g}, top-1 {top1:.4f}; decode after it: worst max-abs "
              f"{worst:.4g}", flush=True)
        assert err <= 2e-2 and top1 >= 0.99 and worst <= 2e-2
    finally:
        for n in bad:
            m.set_weight(n, w[n])
    assert m.swiglu_shift() == 0
    _clean_forward(m, prompt[:48])
