"""The Qwen3 decoder on the HIP device: the counterpart of the reference's planned Lrm.Models.Qwen (Qwen3Config.load,
Forward.runStage, Greedy.run; docs/dev-plan.md:166-170,289) over the executor in liblrm_hip.so.

The reference's only working composition is tests/Lrm.Tensor.Tests/TinyModel.fs:144-236; the names here (forward,
greedy, the ActivationNames taps, the per-layer caches) follow it.
"""
from __future__ import annotations

import ctypes as C
import json
import os
from dataclasses import asdict, dataclass
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import _native as N
from ._native import check, lib, u32s
from .gpu_core import HipBackend

# torch's float32 inv_freq for theta 1e6 and head_dim 128 (the Qwen3 family), as pinned by the reference
# (tests/Lrm.Tensor.Tests/RopeTests.fs:36-101, SHA-256 138c99b1...). Word j of a head_dim d that divides 128 is word
# j * 128 / d here: theta^(-2j/d) is the same float32 exponent as theta^(-2 (j 128/d) / 128).
QWEN3_INV_FREQ_HD128 = [
    0x3F800000, 0x3F4E4BAD, 0x3F263DE0, 0x3F05F6EF, 0x3ED7E89B, 0x3EADFCFF, 0x3E8C3504, 0x3E61F835,
    0x3E361887, 0x3E12BD91, 0x3DEC7FD6, 0x3DBE94C6, 0x3D99940D, 0x3D778513, 0x3D47763F, 0x3D20BC1D,
    0x3D0186E3, 0x3CD0C1A8, 0x3CA8398B, 0x3C879008, 0x3C5A7BF2, 0x3C301052, 0x3C0DE12D, 0x3BE4AA46,
    0x3BB8449C, 0x3B947DAE, 0x3B6F520E, 0x3B40DAC5, 0x3B1B690D, 0x3AFA78F0, 0x3AC9D75C, 0x3AA2A6F7,
    0x3A83126F, 0x3A533F28, 0x3A2A3B44, 0x3A092E02, 0x39DD1725, 0x39B229FB, 0x398F9272, 0x39676492,
    0x393A7753, 0x39164324, 0x38F22CE2, 0x38C327B5, 0x389D43A4, 0x387D75D4, 0x384C3FBE, 0x382497AB,
    0x3804A2B2, 0x37D5C441, 0x37AC431D, 0x378AD0ED, 0x375FBA4F, 0x37344A0E, 0x371148E3, 0x36EA2732,
    0x36BCB0C1, 0x36980E02, 0x36751070, 0x36457BAB, 0x361F23E4, 0x36003DEC, 0x35CEAF79, 0x35A68E4C,
]


def inv_freq_bits(head_dim: int) -> np.ndarray:
    """The pinned theta-1e6 inverse frequencies for a head_dim dividing 128."""
    if head_dim < 2 or 128 % head_dim:
        raise ValueError(f"no pinned inverse frequencies for head_dim {head_dim}")
    step = 128 // head_dim
    return np.array(QWEN3_INV_FREQ_HD128[::step], dtype=np.uint32)


LAYER_WEIGHTS = (
    "input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
    "self_attn.o_proj.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight",
    "post_attention_layernorm.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
)


@dataclass
class QwenConfig:
    """Qwen3Config (the fields TinyModel.loadModel reads from config.json, TinyModel.fs:60-74)."""

    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    max_pos: int
    eps: float = 1e-6

    @classmethod
    def from_hf(cls, path_or_dict, max_pos: Optional[int] = None) -> "QwenConfig":
        d = path_or_dict if isinstance(path_or_dict, dict) else json.load(open(path_or_dict))
        return cls(d["num_hidden_layers"], d["hidden_size"], d["num_attention_heads"], d["num_key_value_heads"],
                   d["head_dim"], d["intermediate_size"], d["vocab_size"],
                   max_pos or d["max_position_embeddings"], d["rms_norm_eps"])

    @classmethod
    def qwen3_0_6b(cls, max_pos: int = 4096) -> "QwenConfig":
        return cls(28, 1024, 16, 8, 128, 3072, 151936, max_pos)

    @classmethod
    def qwen3_1_7b(cls, max_pos: int = 4096) -> "QwenConfig":
        return cls(28, 2048, 16, 8, 128, 6144, 151936, max_pos)

    @classmethod
    def tiny_plumbing(cls, max_pos: int = 64) -> "QwenConfig":
        """2 layers, hidden 64, 4/2 heads, head_dim 16, SwiGLU 192, vocab 512, tied embeddings."""
        return cls(2, 64, 4, 2, 16, 192, 512, max_pos)

    def weight_shapes(self) -> Dict[str, tuple]:
        QC, KC = self.heads * self.head_dim, self.kv_heads * self.head_dim
        shapes = {"model.embed_tokens.weight": (self.vocab, self.hidden), "model.norm.weight": (self.hidden,)}
        per = {
            "input_layernorm.weight": (self.hidden,), "self_attn.q_proj.weight": (QC, self.hidden),
            "self_attn.k_proj.weight": (KC, self.hidden), "self_attn.v_proj.weight": (KC, self.hidden),
            "self_attn.o_proj.weight": (self.hidden, QC), "self_attn.q_norm.weight": (self.head_dim,),
            "self_attn.k_norm.weight": (self.head_dim,), "post_attention_layernorm.weight": (self.hidden,),
            "mlp.gate_proj.weight": (self.intermediate, self.hidden), "mlp.up_proj.weight": (self.intermediate, self.hidden),
            "mlp.down_proj.weight": (self.hidden, self.intermediate),
        }
        for i in range(self.layers):
            for n in LAYER_WEIGHTS:
                shapes[f"model.layers.{i}.{n}"] = per[n]
        return shapes

    def param_count(self) -> int:
        return int(sum(np.prod(s) for s in self.weight_shapes().values()))

    def oracle_dict(self) -> dict:
        return dict(asdict(self))


def synthetic_weights(cfg: QwenConfig, seed: int, std: float = 0.02) -> Dict[str, np.ndarray]:
    """Random-init weights as bf16 bits: every matrix N(0, std) (float32, then bf16 round-to-nearest-even), every norm
    weight 1.0 (0x3F80), each tensor from its own counter-based stream keyed by its name."""
    out = {}
    for name, shape in cfg.weight_shapes().items():
        if len(shape) == 1:
            out[name] = np.full(shape, 0x3F80, np.uint16)
        else:
            a = np.empty(shape, np.uint16)
            check(lib().lrm_synth_normal_bf16(seed, lib().lrm_stream_of(name.encode()), a.size, std, a.ctypes.data))
            out[name] = a
    return out


def synthetic_normal_f32(seed: int, name: str, shape, std: float = 1.0) -> np.ndarray:
    a = np.empty(shape, np.float32)
    check(lib().lrm_synth_normal_f32(seed, lib().lrm_stream_of(name.encode()), a.size, std, a.ctypes.data))
    return a


def synthetic_ids(seed: int, name: str, n: int, vocab: int) -> np.ndarray:
    """Token ids uniform in [0, vocab) from a seed (numpy PCG64)."""
    rng = np.random.default_rng([seed, int(lib().lrm_stream_of(name.encode())) & 0xFFFFFFFF])
    return rng.integers(0, vocab, n, dtype=np.int64).astype(np.int32)


def rope_table(head_dim: int, max_pos: int):
    """The product's T_spec table (float32 cos, sin [max_pos, head_dim / 2])."""
    inv = inv_freq_bits(head_dim)
    half = head_dim // 2
    cos = np.empty((max_pos, half), np.float32)
    sin = np.empty((max_pos, half), np.float32)
    check(lib().lrm_rope_table(u32s(inv), half, max_pos, cos.ctypes.data, sin.ctypes.data))
    return cos, sin


class QwenModel:
    """A Qwen3 decoder resident on one HIP device. mode "fp32" runs the reference catalog kernels (the parity path);
    mode "fast" (alias "bf16": the model's weights stay bf16) runs the fast path: fp16-operand MFMA GEMMs with fused
    epilogues for prefill, an fp16 KV cache, bf16-weight GEMVs and on-device greedy decode."""

    MODES = {"fp32": 0, "fast": 1, "bf16": 1}

    def __init__(self, backend: Optional[HipBackend], cfg: QwenConfig, mode: str = "fast", max_tokens: int = 512,
                 taps: bool = False, inv_freq: Optional[Sequence[int]] = None, batch: int = 1):
        """batch: sequences held together (fast mode, 1..16): one KV cache each, prefilled one at a time with
        forward(seq=b) and decoded together by decode_batch."""
        self.backend = backend or HipBackend(0)
        self.cfg = cfg
        self.mode = mode
        self.batch = batch
        c = N.QwenConfigC(cfg.layers, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.intermediate, cfg.vocab,
                          cfg.max_pos, cfg.eps, self.MODES[mode], max_tokens, batch, 1 if taps else 0)
        inv = np.asarray(inv_freq if inv_freq is not None else inv_freq_bits(cfg.head_dim), np.uint32)
        self._h = C.c_void_p()
        check(lib().lrm_qwen_create(self.backend.handle, C.byref(c), u32s(inv), len(inv), C.byref(self._h)))
        self.max_tokens = max_tokens

    def close(self):
        if getattr(self, "_h", None):
            check(lib().lrm_qwen_destroy(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # weights
    def set_weight(self, name: str, bits: np.ndarray) -> None:
        a = np.ascontiguousarray(bits, dtype=np.uint16)
        check(lib().lrm_qwen_set_weight(self._h, name.encode(), a.ctypes.data, a.size))

    def load_safetensors(self, path: str) -> None:
        """Every weight from a Qwen3 checkpoint through the library's validating reader: each weight of this
        configuration as BF16 with its exact shape, nothing else but an optional lm_head.weight equal to the tied
        embedding byte for byte."""
        check(lib().lrm_qwen_load_safetensors(self._h, os.fsencode(path)))

    def load_weights(self, weights: Dict[str, np.ndarray]) -> None:
        for name in self.cfg.weight_shapes():
            self.set_weight(name, weights[name])

    def read_weight(self, name: str) -> np.ndarray:
        shape = self.cfg.weight_shapes()[name]
        a = np.empty(shape, np.uint16)
        check(lib().lrm_qwen_read_weight(self._h, name.encode(), a.ctypes.data, a.size))
        return a

    # forward / greedy (TinyModel.forward / greedy)
    def forward(self, ids, pos0: int = 0, logits_rows: Optional[int] = None, seq: int = 0):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        t = ids.size
        rows = t if logits_rows is None else logits_rows
        logits = np.empty((rows, self.cfg.vocab), np.float32)
        am = C.c_uint32()
        check(lib().lrm_qwen_forward(self._h, seq, pos0, ids.ctypes.data, t, logits.ctypes.data if rows else None,
                                     rows, C.byref(am)))
        return logits, am.value

    def greedy(self, prompt, steps: int) -> np.ndarray:
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(steps, np.int32)
        check(lib().lrm_qwen_greedy(self._h, prompt.ctypes.data, prompt.size, steps, out.ctypes.data))
        return out

    def decode_set(self, token, pos) -> None:
        """The next token and its position, for every sequence (scalars when batch is 1)."""
        a = np.ascontiguousarray(np.broadcast_to(np.asarray(token, np.int32), (self.batch,)))
        p = np.ascontiguousarray(np.broadcast_to(np.asarray(pos, np.int32), (self.batch,)))
        check(lib().lrm_qwen_decode_set(self._h, a.ctypes.data, p.ctypes.data))

    def decode_batch(self, tokens, pos, steps: int) -> np.ndarray:
        """steps greedy decode steps of every sequence on device; returns ids [steps, batch]."""
        a = np.ascontiguousarray(tokens, np.int32)
        p = np.ascontiguousarray(pos, np.int32)
        if a.shape != (self.batch,) or p.shape != (self.batch,):
            raise ValueError(f"tokens and pos must hold {self.batch} entries")
        out = np.empty((steps, self.batch), np.int32)
        check(lib().lrm_qwen_decode_batch(self._h, a.ctypes.data, p.ctypes.data, steps, out.ctypes.data))
        return out

    def decode_run(self, steps: int) -> None:
        check(lib().lrm_qwen_decode_run(self._h, steps))

    def decode_ids(self, count: int) -> np.ndarray:
        out = np.empty(count, np.int32)
        check(lib().lrm_qwen_decode_ids(self._h, out.ctypes.data, count))
        return out

    def read_logits(self, rows: int = 1) -> np.ndarray:
        out = np.empty((rows, self.cfg.vocab), np.float32)
        check(lib().lrm_qwen_read_logits(self._h, out.ctypes.data, rows))
        return out

    def last_ms(self) -> float:
        return lib().lrm_qwen_last_ms(self._h)

    def persistent_decode(self) -> bool:
        """True when decode steps run as the single persistent launch (decode_step_persistent); set
        LRM_HIP_DECODE=kernels before construction for the per-stage kernel list."""
        return lib().lrm_qwen_persistent_decode(self._h) == 1

    def swiglu_shift(self) -> int:
        """Fast mode: the binades s the SwiGLU output is shifted down by before its fp16 store (0 until a forward
        overflowed there and ran again with s = 8, then 16; back to 0 when a weight is written)."""
        return lib().lrm_qwen_swiglu_shift(self._h)

    def set_swiglu_shift(self, shift: int) -> None:
        """Sets the SwiGLU shift (0 .. 24) for the calls that follow (until a weight is written)."""
        check(lib().lrm_qwen_set_swiglu_shift(self._h, int(shift)))

    def token(self, name: str) -> int:
        t = C.c_uint32()
        check(lib().lrm_qwen_token(self._h, name.encode(), C.byref(t)))
        return t.value

    # taps and caches
    def taps(self, rows: int) -> Dict[str, np.ndarray]:
        out = {}
        for i in range(lib().lrm_qwen_tap_count(self._h)):
            name = C.create_string_buffer(96)
            w = C.c_int()
            check(lib().lrm_qwen_tap_info(self._h, i, name, 96, C.byref(w)))
            a = np.empty((rows, w.value), np.float32)
            check(lib().lrm_qwen_read_tap(self._h, i, a.ctypes.data, rows))
            out[name.value.decode()] = a
        return out

    def read_cache(self, layer: int, which: str, row0: int, rows: int, seq: int = 0) -> np.ndarray:
        out = np.empty((rows, self.cfg.kv_heads * self.cfg.head_dim), np.float32)
        check(lib().lrm_qwen_read_cache(self._h, seq, layer, 0 if which == "k" else 1, row0, rows, out.ctypes.data))
        return out

    def write_cache(self, layer: int, which: str, row0: int, data: np.ndarray, seq: int = 0) -> None:
        a = np.ascontiguousarray(data, np.float32)
        check(lib().lrm_qwen_write_cache(self._h, seq, layer, 0 if which == "k" else 1, row0, a.shape[0],
                                         a.ctypes.data))

    def fill_cache_random(self, seed: int, rows: int) -> None:
        check(lib().lrm_qwen_fill_cache_random(self._h, seed, rows))
