"""numpy front end of the oracle library (liblrm_oracle.so, built from cpuref.c by oracle/Makefile).

Test infrastructure only: the tests, the smoke check and the bench's CPU-baseline leg use it as the checker. The
product (rosylnalive_amd) never imports it. Each function names the reference function it restates; the arithmetic
is in cpuref_ops.inc.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblrm_oracle.so")

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _lib.orc_last_error.restype = C.c_char_p
        _lib.orc_attention_scale_f32.restype = C.c_float
        _lib.orc_attention_scale_f64.restype = C.c_double
        _lib.orc_bf16_narrow_rne.restype = C.c_uint16
        _lib.orc_bf16_narrow_rne.argtypes = [C.c_float]
    return _lib


class OracleError(ValueError):
    pass


def _check(rc: int) -> None:
    if rc != 0:
        raise OracleError(lib().orc_last_error().decode())


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _mode(dtype) -> tuple:
    dt = np.dtype(dtype)
    if dt == np.float32:
        return "f32", C.c_float, np.float32
    if dt == np.float64:
        return "f64", C.c_double, np.float64
    raise OracleError(f"the oracle computes in float32 or float64, not {dt}")


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def threads() -> int:
    return lib().orc_get_threads()


def bf16_narrow(x: np.ndarray) -> np.ndarray:
    """Bf16.narrowRne (src/Lrm.Core/Numerics.fs:35-45), vectorised in numpy: RNE, NaN -> 7fc0 / ffc0 by sign."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = np.where((u[nan] & 0x80000000) != 0, 0xFFC0, 0x7FC0).astype(np.uint16)
    return r


def bf16_widen(bits: np.ndarray) -> np.ndarray:
    """Bf16.widen (Numerics.fs:24-33): the bits become the top half of a float32, exactly."""
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def cos_sin_exact(x: float) -> tuple:
    """ExactTrig.cosSin (Rope.fs:146-161): correctly rounded float64 (cos x, sin x) of a float32 x."""
    c, s = C.c_double(), C.c_double()
    _check(lib().orc_cos_sin_exact(C.c_float(x), C.byref(c), C.byref(s)))
    return c.value, s.value


def rope_table(inv_freq_bits: np.ndarray, max_pos: int) -> tuple:
    """RopeTable.create (Rope.fs:218-251): float32 cos, sin [max_pos, half]."""
    inv = np.ascontiguousarray(inv_freq_bits, dtype=np.uint32)
    half = inv.size
    cos = np.empty((max_pos, half), np.float32)
    sin = np.empty((max_pos, half), np.float32)
    _check(lib().orc_rope_table(_p(inv), C.c_int(half), C.c_int(max_pos), _p(cos), _p(sin)))
    return cos, sin


def attention_scale(head_dim: int, dtype=np.float32):
    """CpuRef.attentionScale (CpuRef.fs:56-60)."""
    s, _, _ = _mode(dtype)
    return getattr(lib(), f"orc_attention_scale_{s}")(C.c_int(head_dim))


def embed(table: np.ndarray, ids, dtype=np.float32) -> np.ndarray:
    """CpuRef.embed (CpuRef.fs:113-132)."""
    s, _, npt = _mode(dtype)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    vocab, cols = table.shape
    y = np.empty((ids.size, cols), npt)
    _check(getattr(lib(), f"orc_embed_{s}")(_p(table), vocab, cols, _p(ids), ids.size, _p(y)))
    return y


def embed_gather(table: np.ndarray, ids, dtype=np.float32) -> np.ndarray:
    """CpuRef.embedGather (CpuRef.fs:136-146)."""
    s, _, npt = _mode(dtype)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    vocab, cols = table.shape
    y = np.empty((ids.size, cols), npt)
    _check(getattr(lib(), f"orc_embed_gather_{s}")(_p(table), vocab, cols, _p(ids), ids.size, _p(y)))
    return y


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """CpuRef.rmsNorm (CpuRef.fs:150-178); eps is rounded once to the mode's type."""
    s, ct, npt = _mode(x.dtype)
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    y = np.empty_like(x)
    _check(getattr(lib(), f"orc_rmsnorm_{s}")(_p(x), C.c_int64(x.size), _p(w), C.c_int(w.size), ct(eps), _p(y)))
    return y


def matmul_bf16w(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """CpuRef.matmulBf16W (CpuRef.fs:186-221): x [m, k] times widen(w [n, k])^T."""
    s, _, npt = _mode(x.dtype)
    x = np.ascontiguousarray(x)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    m, k = x.shape
    n, k2 = w.shape
    if k != k2:
        raise OracleError(f"x is [{m}, {k}] but w is [{n}, {k2}]")
    y = np.empty((m, n), npt)
    _check(getattr(lib(), f"orc_matmul_bf16w_{s}")(_p(x), m, k, _p(w), n, _p(y)))
    return y


def rope_apply(cos: np.ndarray, sin: np.ndarray, x: np.ndarray, heads: int, pos0: int) -> np.ndarray:
    """CpuRef.ropeApply (CpuRef.fs:225-267)."""
    s, _, npt = _mode(x.dtype)
    x = np.ascontiguousarray(x)
    max_pos, half = cos.shape
    rows = x.shape[0]
    if x.shape[1] != heads * 2 * half:
        raise OracleError(f"x is {x.shape}, not [T, {heads} * {2 * half}]")
    y = np.empty_like(x)
    _check(getattr(lib(), f"orc_rope_apply_{s}")(_p(cos), _p(sin), max_pos, half, _p(x), rows, heads, pos0, _p(y)))
    return y


def attention(q, k_cache, v_cache, q_heads, kv_heads, head_dim, past, scale) -> np.ndarray:
    """CpuRef.attention (CpuRef.fs:274-332)."""
    s, ct, npt = _mode(q.dtype)
    q = np.ascontiguousarray(q)
    k_cache = np.ascontiguousarray(k_cache, dtype=npt)
    v_cache = np.ascontiguousarray(v_cache, dtype=npt)
    rows = q.shape[0]
    y = np.empty((rows, q_heads * head_dim), npt)
    _check(
        getattr(lib(), f"orc_attention_{s}")(
            _p(q), rows, _p(k_cache), _p(v_cache), k_cache.shape[0], q_heads, kv_heads, head_dim, past, ct(scale), _p(y)
        )
    )
    return y


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """CpuRef.siluMul (CpuRef.fs:335-355)."""
    s, _, npt = _mode(g.dtype)
    g = np.ascontiguousarray(g)
    u = np.ascontiguousarray(u, dtype=npt)
    y = np.empty_like(g)
    _check(getattr(lib(), f"orc_silu_mul_{s}")(_p(g), _p(u), C.c_int64(g.size), _p(y)))
    return y


def add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """CpuRef.add (CpuRef.fs:358-378)."""
    s, _, npt = _mode(a.dtype)
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b, dtype=npt)
    y = np.empty_like(a)
    _check(getattr(lib(), f"orc_add_{s}")(_p(a), _p(b), C.c_int64(a.size), _p(y)))
    return y


def argmax_rows(x: np.ndarray) -> np.ndarray:
    """CpuRef.argmaxRows (CpuRef.fs:453-467): u32 index per row, 0xFFFFFFFF for a row with a NaN."""
    s, _, _ = _mode(x.dtype)
    x = np.ascontiguousarray(x)
    rows, cols = x.shape
    y = np.empty(rows, np.uint32)
    _check(getattr(lib(), f"orc_argmax_rows_{s}")(_p(x), rows, cols, _p(y)))
    return y


def softmax_rows(x: np.ndarray) -> np.ndarray:
    """CpuRef.softmax (CpuRef.fs:405-420) with Rows.softmax (Rows.fs:101-110): a NaN anywhere makes the row NaN."""
    s, _, _ = _mode(x.dtype)
    x = np.ascontiguousarray(x)
    y = np.empty_like(x)
    _check(getattr(lib(), f"orc_softmax_rows_{s}")(_p(x), x.shape[0], x.shape[1], _p(y)))
    return y


def logsumexp_rows(x: np.ndarray) -> np.ndarray:
    """Rows.logSumExp (Rows.fs:112-135) per row: an infinite row maximum is the answer, a NaN gives NaN."""
    s, _, npt = _mode(x.dtype)
    x = np.ascontiguousarray(x)
    y = np.empty(x.shape[0], npt)
    _check(getattr(lib(), f"orc_logsumexp_rows_{s}")(_p(x), x.shape[0], x.shape[1], _p(y)))
    return y


def kl_rows(p: np.ndarray, q: np.ndarray) -> np.ndarray:
    """CpuRef.kl (CpuRef.fs:470-502) with Rows.kl."""
    s, _, npt = _mode(p.dtype)
    p = np.ascontiguousarray(p)
    q = np.ascontiguousarray(q, dtype=npt)
    y = np.empty(p.shape[0], npt)
    _check(getattr(lib(), f"orc_kl_rows_{s}")(_p(p), _p(q), p.shape[0], p.shape[1], _p(y)))
    return y


# ---- the Qwen3 forward (tests/Lrm.Tensor.Tests/TinyModel.fs:144-236) ----

LAYER_WEIGHTS = (
    "input_layernorm.weight",
    "self_attn.q_proj.weight",
    "self_attn.k_proj.weight",
    "self_attn.v_proj.weight",
    "self_attn.o_proj.weight",
    "self_attn.q_norm.weight",
    "self_attn.k_norm.weight",
    "post_attention_layernorm.weight",
    "mlp.gate_proj.weight",
    "mlp.up_proj.weight",
    "mlp.down_proj.weight",
)

LAYER_TAPS = (
    "input_layernorm.out",
    "attn.q_proj.out",
    "attn.k_proj.out",
    "attn.v_proj.out",
    "attn.q_norm.out",
    "attn.k_norm.out",
    "attn.q_rope",
    "attn.k_rope",
    "attn.v_cache",
    "attn.o_proj.in",
    "attn.o_proj.out",
    "resid_mid",
    "post_attention_layernorm.out",
    "mlp.gate.out",
    "mlp.up.out",
    "mlp.down.in",
    "mlp.down.out",
    "out",
)


def tap_names(layers: int) -> list:
    """ActivationNames.all (src/Lrm.Tensor/Goldens.fs:314-322): 18 * layers + 3 names in canonical order."""
    return ["embed.out"] + [f"L{i}.{t}" for i in range(layers) for t in LAYER_TAPS] + ["final_norm.out", "logits"]


class _Config(C.Structure):
    _fields_ = [
        ("layers", C.c_int),
        ("hidden", C.c_int),
        ("heads", C.c_int),
        ("kv_heads", C.c_int),
        ("head_dim", C.c_int),
        ("intermediate", C.c_int),
        ("vocab", C.c_int),
        ("max_pos", C.c_int),
        ("eps", C.c_double),
    ]


class QwenOracle:
    """CpuRef composition of a Qwen3 decoder (TinyModel.fs). `weights` maps HF names to bf16 uint16 arrays;
    `cos`/`sin` is the T_spec table [max_pos, head_dim / 2]."""

    def __init__(self, cfg: dict, weights: dict, cos: np.ndarray, sin: np.ndarray):
        self.cfg = dict(cfg)
        self._c = _Config(
            cfg["layers"], cfg["hidden"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["intermediate"],
            cfg["vocab"], cfg["max_pos"], cfg["eps"],
        )
        names = ["model.embed_tokens.weight", "model.norm.weight"] + [
            f"model.layers.{i}.{n}" for i in range(cfg["layers"]) for n in LAYER_WEIGHTS
        ]
        self._w = [np.ascontiguousarray(weights[n], dtype=np.uint16) for n in names]
        self._wp = (C.c_void_p * len(self._w))(*[a.ctypes.data for a in self._w])
        self.cos = np.ascontiguousarray(cos, dtype=np.float32)
        self.sin = np.ascontiguousarray(sin, dtype=np.float32)
        if self.cos.shape[0] < cfg["max_pos"]:
            raise OracleError("the RoPE table is shorter than max_pos")

    def new_cache(self, dtype=np.float32):
        c = self.cfg
        shape = (c["layers"], c["max_pos"], c["kv_heads"] * c["head_dim"])
        return np.zeros(shape, dtype), np.zeros(shape, dtype)

    def forward(self, cache, pos0: int, ids, dtype=np.float32, taps: bool = False):
        """TinyModel.forward: returns logits [T, vocab] (and the tap dict when taps=True); writes the cache."""
        s, _, npt = _mode(dtype)
        kc, vc = cache
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        t = ids.size
        c = self.cfg
        logits = np.empty((t, c["vocab"]), npt)
        tap_arrays = None
        tp = None
        if taps:
            widths = {
                "embed.out": c["hidden"],
                "final_norm.out": c["hidden"],
                "logits": c["vocab"],
            }
            qc, kvc = c["heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"]
            per = {
                "input_layernorm.out": c["hidden"], "attn.q_proj.out": qc, "attn.k_proj.out": kvc,
                "attn.v_proj.out": kvc, "attn.q_norm.out": qc, "attn.k_norm.out": kvc, "attn.q_rope": qc,
                "attn.k_rope": kvc, "attn.v_cache": kvc, "attn.o_proj.in": qc, "attn.o_proj.out": c["hidden"],
                "resid_mid": c["hidden"], "post_attention_layernorm.out": c["hidden"],
                "mlp.gate.out": c["intermediate"], "mlp.up.out": c["intermediate"],
                "mlp.down.in": c["intermediate"], "mlp.down.out": c["hidden"], "out": c["hidden"],
            }
            names = tap_names(c["layers"])
            tap_arrays = {}
            for n in names:
                wdt = widths.get(n) or per[n.split(".", 1)[1]]
                tap_arrays[n] = np.empty((t, wdt), npt)
            tp = (C.c_void_p * len(names))(*[tap_arrays[n].ctypes.data for n in names])
        _check(
            getattr(lib(), f"orc_qwen_forward_{s}")(
                C.byref(self._c), self._wp, _p(self.cos), _p(self.sin), _p(kc), _p(vc), pos0, _p(ids), t,
                _p(logits), tp,
            )
        )
        return (logits, tap_arrays) if taps else logits

    def greedy(self, prompt, steps: int, dtype=np.float32) -> np.ndarray:
        """TinyModel.greedy (TinyModel.fs:219-236)."""
        s, _, _ = _mode(dtype)
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(steps, np.int32)
        _check(
            getattr(lib(), f"orc_qwen_greedy_{s}")(
                C.byref(self._c), self._wp, _p(self.cos), _p(self.sin), _p(prompt), prompt.size, steps, _p(out)
            )
        )
        return out
