"""Checkpoint load through the executor (lrm_qwen_load_safetensors): a synthetic file of the Qwen3-0.6B layout (311
BF16 entries including the stored copy of the tied lm_head, header N = 35,552 as the real file's,
tests/Lrm.Tensor.Tests/ModelTests.fs:16-29) loads bit for bit and gives the same logits as the same weights set one by
one; the committed tiny golden model loads too; files of another layout are refused with the reason.
"""
import os

import numpy as np
import pytest

from conftest import TINY
from rosylnalive_amd import safetensors_io as st
from rosylnalive_amd.gpu_core import HipBackend, LrmError
from rosylnalive_amd.qwen import QwenConfig, QwenModel, synthetic_ids, synthetic_weights
from rosylnalive_amd.safetensors_io import SafetensorsFormatError

pytestmark = pytest.mark.gpu


def test_qwen3_0_6b_layout_loads_bit_for_bit(tmp_path):
    cfg = QwenConfig.qwen3_0_6b(max_pos=256)
    w = synthetic_weights(cfg, seed=31)
    path = str(tmp_path / "model.safetensors")
    tensors = [(n, "BF16", a) for n, a in w.items()] + [("lm_head.weight", "BF16", w["model.embed_tokens.weight"])]
    st.save(path, tensors, [("format", "pt")])
    with st.SafetensorsFile.open(path) as f:
        assert len(f.entries) == 311 and f.header_length == 35_552 and f.data_offset == 35_560 and f.is_aligned
    ids = synthetic_ids(31, "ckpt/prompt", 24, cfg.vocab)
    out = []
    for from_file in (True, False):  # one model per backend (a backend creates its heap once)
        b = HipBackend(0)
        m = QwenModel(b, cfg, mode="fast", max_tokens=64)
        try:
            if from_file:
                m.load_safetensors(path)
                for n in ("model.embed_tokens.weight", "model.layers.0.self_attn.q_proj.weight",
                          "model.layers.27.mlp.down_proj.weight", "model.norm.weight"):
                    assert m.read_weight(n).tobytes() == w[n].tobytes(), n
            else:
                m.load_weights(w)
            out.append(m.forward(ids, 0))
        finally:
            m.close()
            b.close()
    (l1, a1), (l2, a2) = out
    assert l1.tobytes() == l2.tobytes() and a1 == a2
    print(f"0.6B layout: 311 entries loaded, logits equal, argmax {a1}", flush=True)


def _tiny_cfg(tiny):
    c = tiny["cfg"]
    return QwenConfig(c["layers"], c["hidden"], c["heads"], c["kv_heads"], c["head_dim"], c["intermediate"],
                      c["vocab"], c["max_pos"], c["eps"])


def test_tiny_golden_model_loads_and_other_layouts_are_refused(tiny, tmp_path):
    cfg = _tiny_cfg(tiny)
    golden = os.path.join(TINY, "model", "model.safetensors")
    w = st.load(golden)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fp32", max_tokens=16, inv_freq=tiny["rope"]["inv_freq.bits"])
    try:
        m.load_safetensors(golden)
        for n, a in w.items():
            assert m.read_weight(n).tobytes() == a.tobytes(), n

        def write(tensors):
            p = str(tmp_path / "bad.safetensors")
            st.save(p, tensors, [("format", "pt")])
            return p

        base = [(n, "BF16", a) for n, a in w.items()]
        emb = w["model.embed_tokens.weight"]
        cases = [
            ("no tensor model.norm.weight", [t for t in base if t[0] != "model.norm.weight"]),
            ("is not a weight", base + [("model.extra", "BF16", np.zeros(4, np.uint16))]),
            ("is f32, not bf16", [t if t[0] != "model.norm.weight" else (t[0], "F32", t[2].astype(np.float32))
                                  for t in base]),
            ("has shape", [t if t[0] != "model.norm.weight" else (t[0], "BF16", t[2][:-1]) for t in base]),
            ("differs from model.embed_tokens.weight", base + [("lm_head.weight", "BF16", emb ^ np.uint16(1))]),
        ]
        for what, tensors in cases:
            with pytest.raises(LrmError) as e:
                m.load_safetensors(write(tensors))
            assert what in str(e.value), (what, str(e.value))
        m.load_safetensors(write(base + [("lm_head.weight", "BF16", emb.copy())]))  # a stored tied copy is fine
        p = str(tmp_path / "torn.safetensors")
        with open(p, "wb") as f:
            f.write(open(golden, "rb").read()[:-2])
        with pytest.raises(SafetensorsFormatError):
            m.load_safetensors(p)
    finally:
        m.close()
        b.close()
