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


def test_static_scratch_rejects_more_partials_than_it_holds():
    """4 MiB holds batch * 16 heads * splits * 130 floats up to 504 (batch, split) pairs: 16 sequences at max_pos
    2048 and 32 splits (4,259,840 bytes) do not fit, 15 do. The bound is computed from the contract-checked words, and
    a refused call records nothing."""
    B, mp = 16, 2048
    s = Session({"qkv": (F32, (B, 4096), RO, None), "qn": (BF16, (128,), RO, None), "kn": (BF16, (128,), RO, None),
                 "cos": (F32, (mp, 64), RO, None), "sin": (F32, (mp, 64), RO, None),
                 "kc": (F16, (B * 8, mp, 128), 0, None), "vc": (F16, (B * 8, 128, mp), 0, None),
                 "part": (F32, (B * 16 * (mp // 64) * 130,), 0, None),
                 "y": (F32, (B, 2048), 0, None), "state": (U32, (2 * B + 2,), 0, None)})
    try:
        def words(batch, partials=0):
            return s.fields("attention_decode_f16", qkv="qkv", q_norm="qn", k_norm="kn", cos_table="cos",
                            sin_table="sin", k_cache="kc", v_cache="vc", partials=partials, state="state", q_heads=16,
                            kv_heads=8, max_pos=mp, eps=1e-6, scale=0.08838834764831845, batch=batch, chunks=1,
                            splits=0)

        cl = s.backend.begin()
        try:
            with pytest.raises(GpuContractException, match="static scratch holds"):
                cl.dispatch_decode_attention_static(words(16), s.tok["y"])
            with pytest.raises(GpuContractException, match="library supplies"):
                cl.dispatch_decode_attention_static(words(1, "part"), s.tok["y"])
            c = s.backend.wait(s.backend.submit(cl))
            assert c.dispatches == 0  # the refused calls recorded neither kernel
        finally:
            cl.release()
        cl = s.backend.begin()
        try:
            cl.dispatch_decode_attention_static(words(15), s.tok["y"])  # 3,993,600 bytes: fits (recorded, not run)
        finally:
            cl.release()
    finally:
        s.close()


def test_refused_combine_leaves_the_list_and_caches_unchanged(sess):
    """The combine's own contract check (here: y too small for the batch, then y of the wrong dtype) refuses the call
    after the attention's check passed: neither kernel is recorded, so submitting the list runs nothing and the K/V
    caches keep their bits (an orphan attention launch would append rows)."""
    positions = [5, 64, 700, 2000]
    _reset(sess, positions)
    words = sess.fields("attention_decode_f16", **_fields(positions, 0, 0))
    cl = sess.backend.begin()
    try:
        with pytest.raises(GpuContractException):
            cl.dispatch_decode_attention_static(words, sess.tok["qn"])  # bf16 [128]: wrong dtype and too small
        with pytest.raises(GpuContractException):
            cl.dispatch_decode_attention_static(words, 0)  # token 0: the null tensor
        c = sess.backend.wait(sess.backend.submit(cl))
        assert c.dispatches == 0
    finally:
        cl.release()
    assert sess.read("kc").tobytes() == sess.kc0.tobytes()
    assert sess.read("vc").tobytes() == sess.vc0.tobytes()
