"""The entry point that allocates nothing: lrm_hip_dispatch_decode_attention_static records attention_decode_f16 and
attention_combine with the split partials in the library's static scratch (no counterpart in the reference; for callers
that cannot allocate device memory). Checked against the same two kernels dispatched with a partials tensor of the
heap, bit for bit (the same kernels and arithmetic), on two calls in a row, the second with a smaller batch and
context, then as a reusable list replayed as a HIP graph, and its size limit.
"""
import numpy as np
import pytest

from gpu_session import POISON_F32, Session
from oracle import cpuref
from rosylnalive_amd.gpu_core import DType, GpuContractException, TensorFlags
from rosylnalive_amd.qwen import inv_freq_bits, synthetic_normal_f32

pytestmark = pytest.mark.gpu

F32, BF16, F16, U32 = DType.F32, DType.BF16, DType.F16, DType.U32
RO = TensorFlags.READ_ONLY
MAX_POS, BMAX = 2048, 4


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


@pytest.fixture(scope="module")
def sess():
    r = np.random.default_rng(71)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), MAX_POS)
    kc = _f16(synthetic_normal_f32(71, "noalloc/k", (BMAX * 8, MAX_POS, 128)))
    vc = _f16(synthetic_normal_f32(71, "noalloc/v", (BMAX * 8, 128, MAX_POS)))
    qkv = (r.standard_normal((BMAX, 4096)) * 1.5).astype(np.float32)
    s = Session({"qkv": (F32, qkv.shape, RO, qkv), "qn": (BF16, (128,), RO, cpuref.bf16_narrow(np.ones(128))),
                 "kn": (BF16, (128,), RO, cpuref.bf16_narrow(np.ones(128))),
                 "cos": (F32, cos.shape, RO, cos), "sin": (F32, sin.shape, RO, sin),
                 "kc": (F16, kc.shape, 0, kc), "vc": (F16, vc.shape, 0, vc),
                 "part": (F32, (BMAX * 16 * (MAX_POS // 64) * 130,), 0, None),
                 "y": (F32, (BMAX, 2048), 0, None), "state": (U32, (2 * BMAX + 2,), 0, None)})
    s.kc0, s.vc0 = kc, vc
    yield s
    s.close()


def _fields(positions, splits, partials):
    B = len(positions)
    return dict(qkv="qkv", q_norm="qn", k_norm="kn", cos_table="cos", sin_table="sin", k_cache="kc", v_cache="vc",
                partials=partials, state="state", q_heads=16, kv_heads=8, max_pos=MAX_POS, eps=1e-6,
                scale=float(cpuref.attention_scale(128, np.float32)), batch=B, chunks=0 if splits else 1,
                splits=splits)


def _reset(s, positions):
    s.write("kc", s.kc0)
    s.write("vc", s.vc0)
    st = np.zeros(2 * BMAX + 2, np.uint32)
    st[:len(positions)] = positions
    s.write("state", st)
    s.write("y", s.poison("y"))


def _with_heap_partials(s, positions, splits):
    _reset(s, positions)
    B = len(positions)
    cl = s.backend.begin()
    cl.dispatch("attention_decode_f16", s.fields("attention_decode_f16", **_fields(positions, splits, "part")))
    cl.dispatch("attention_combine", s.fields("attention_combine", partials="part", y="y", state="state", q_heads=16,
                                              max_pos=MAX_POS, batch=B, chunks=0 if splits else 1, splits=splits))
    s.backend.wait(s.backend.submit(cl))
    cl.release()
    return s.read("y")[:B].copy(), s.read("kc").copy()


def _static(s, positions, splits, cl=None):
    B = len(positions)
    own = cl is None
    if own:
        _reset(s, positions)
        cl = s.backend.begin()
    cl.dispatch_decode_attention_static(s.fields("attention_decode_f16", **_fields(positions, splits, 0)), s.tok["y"])
    if own:
        s.backend.wait(s.backend.submit(cl))
        cl.release()
        return s.read("y")[:B].copy(), s.read("kc").copy()


def test_static_scratch_equals_heap_partials_on_two_calls(sess):
    """Call 1: four sequences at positions 5, 64, 700, 2000, one 64-key chunk per split (32 splits); call 2: a smaller
    input, two sequences at 3 and 300 with 3 even splits each. Each against the heap-partials dispatch of the same
    inputs, bit for bit, with the caches' appended rows equal too."""
    for positions, splits in (([5, 64, 700, 2000], 0), ([3, 300], 3)):
        ref, kref = _with_heap_partials(sess, positions, splits)
        got, kgot = _static(sess, positions, splits)
        assert np.isfinite(ref).all() and not np.any(got.view(np.uint32) == POISON_F32)
        assert got.tobytes() == ref.tobytes(), positions
        assert kgot.tobytes() == kref.tobytes()


def test_static_scratch_in_a_replayed_graph(sess):
    """A reusable list (captured into a HIP graph at its first submission) holding the static-scratch attention,
    replayed three times with eager work on the same heap between the replays: every replay equals the heap-partials
    result."""
    positions = [17, 900]
    ref, _ = _with_heap_partials(sess, positions, 0)
    cl = sess.backend.begin(reusable=True)
    _static(sess, positions, 0, cl=cl)
    try:
        for _ in range(3):
            _reset(sess, positions)
            sess.backend.wait(sess.backend.submit(cl))
            assert sess.read("y")[:2].tobytes() == ref.tobytes()
            _with_heap_partials(sess, [5, 6, 7, 8], 0)  # eager work between replays
    finally:
        cl.release()


def test_static_scratch_rejects_more_partials_than_it_holds(sess):
    """4 MiB holds batch * 16 heads * splits * 130 floats up to 8065 (batch, split) rows of 16 heads: four sequences
    at 32 splits fit, 4 x 1024 splits do not (max_pos 65536 would need 34 MB)."""
    words = sess.fields("attention_decode_f16", **dict(_fields([1, 2, 3, 4], 0, 0), max_pos=65536))
    cl = sess.backend.begin()
    try:
        with pytest.raises(GpuContractException, match="static scratch holds"):
            cl.dispatch_decode_attention_static(words, sess.tok["y"])
        with pytest.raises(GpuContractException, match="library supplies"):
            cl.dispatch_decode_attention_static(
                sess.fields("attention_decode_f16", **_fields([1], 0, "part")), sess.tok["y"])
    finally:
        cl.release()
