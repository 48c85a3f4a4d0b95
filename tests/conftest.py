import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")
TINY = os.path.join(GOLDEN, "tiny_g1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the HIP C-ABI library")
    config.addinivalue_line("markers", "slow: longer CPU test")


@pytest.fixture(scope="session")
def tiny():
    """The reference's committed tiny Qwen3 (goldens/tiny/g1): config, bf16 weights, T_spec table."""
    import json

    from oracle import cpuref
    from rosylnalive_amd import safetensors_io as st

    cfgj = json.load(open(os.path.join(TINY, "model", "config.json")))
    cfg = dict(
        layers=cfgj["num_hidden_layers"],
        hidden=cfgj["hidden_size"],
        heads=cfgj["num_attention_heads"],
        kv_heads=cfgj["num_key_value_heads"],
        head_dim=cfgj["head_dim"],
        intermediate=cfgj["intermediate_size"],
        vocab=cfgj["vocab_size"],
        max_pos=cfgj["max_position_embeddings"],
        eps=cfgj["rms_norm_eps"],
    )
    weights = st.load(os.path.join(TINY, "model", "model.safetensors"))
    rope = st.load(os.path.join(TINY, "rope.safetensors"))
    cos, sin = cpuref.rope_table(rope["inv_freq.bits"], cfg["max_pos"])
    return {"cfg": cfg, "weights": weights, "rope": rope, "cos": cos, "sin": sin,
            "oracle": cpuref.QwenOracle(cfg, weights, cos, sin)}


def golden(name):
    from rosylnalive_amd import safetensors_io as st

    return st.load(os.path.join(TINY, name))
