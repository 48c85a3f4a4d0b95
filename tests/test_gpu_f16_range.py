"""The fast path's fp16 range monitor: a value it narrows to fp16 (normed hidden rows, q, the K/V cache, the attention
and SwiGLU outputs) that overflows makes the forward or decode call fail with Fp16RangeError naming the site, instead
of passing inf on into logits the caller would take as results. The overflows are forced from the host through the
weights (data only: every kernel still runs to its end), and the same model then runs clean again, bit for bit.
"""
import numpy as np
import pytest

from oracle import cpuref
from rosylnalive_amd.gpu_core import Fp16RangeError, HipBackend
from rosylnalive_amd.qwen import QwenConfig, QwenModel, synthetic_ids, synthetic_weights

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


def test_swiglu_outlier_fails_the_forward_and_names_the_site(model):
    """gate and up rows 0 .. 63 all +1 and rows 64 .. 127 all -1 in layer 1, after a post-attention norm of 30: for
    either sign of a row's sum one half of those columns has gate = up ~ 30 * sum(normed x), so silu(gate) * up runs
    far past 65,504 while h (|h| ~ 30) and the float32 reference stay finite."""
    m, w = model
    ids = synthetic_ids(23, "range/prompt", 48, CFG.vocab)
    base, am = _clean_forward(m, ids)
    gname, uname = "model.layers.1.mlp.gate_proj.weight", "model.layers.1.mlp.up_proj.weight"
    nname = "model.layers.1.post_attention_layernorm.weight"
    g, u = w[gname].copy(), w[uname].copy()
    for a in (g, u):
        a[:64] = bf16(1.0, (64, CFG.hidden))
        a[64:128] = bf16(-1.0, (64, CFG.hidden))
    try:
        m.set_weight(gname, g)
        m.set_weight(uname, u)
        m.set_weight(nname, bf16(30.0, (CFG.hidden,)))
        with pytest.raises(Fp16RangeError) as e:
            m.forward(ids, 0)
        print(e.value, flush=True)
        assert "SwiGLU output (a)" in str(e.value)
    finally:
        for n in (gname, uname, nname):
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
