"""Full-size parity of the fast path against the oracle (CpuRef F32), at the shapes the throughput is quoted on.

- Qwen3-0.6B shape (28 layers, hidden 1024, 16/8 heads, head_dim 128, SwiGLU 3072, vocab 151,936, tied embeddings),
  random N(0, 0.02) bf16 weights, norms 1:
  * a 512-token prefill, every one of the 512 x 151,936 logits against the oracle;
  * a 2048-token prefill, the last 64 rows' logits and a sample of the K / V cache rows against the oracle;
  * a 128-token prompt then 256 greedy tokens: the device's greedy ids are the oracle's greedy ids (the oracle's
    argmax along the device's sequence equals the device's id at every step, up to near-ties), and teacher-forced
    decode steps along that sequence match the oracle's logits.
  * the 4K-context regime of the batch-1 decode: a 4096-token prefill (two 2048-row chunks), then 8 persistent decode
    steps at context 4097..4104 (22 attention splits of three 64-key chunks each), every step's logits against the
    oracle run over the device's own prefill caches, and the cache rows the device wrote against the oracle's.
- Qwen3-1.7B shape (hidden 2048, SwiGLU 6144), 16 sequences whose caches hold 8192 positions of N(0, 1) fp16 values
  (written on the device), two batched decode steps: sequences 0, 7 and 15 against the oracle run over the same
  caches read back from the device.

Bounds (bf16 weights; fp16 MFMA operands and KV cache; fp32 accumulation, norms and residual stream): logits max-abs
<= 2e-2, top-1 agreement >= 99 %, and every top-1 flip a near-tie (the device's pick within twice the measured
max-abs of the oracle's maximum in the oracle's own logits). The reference states these at tiny scale in
tests/Lrm.Tensor.Tests/TinyModelTests.fs:243-334; its tiny goldens pin the oracle.
"""
import numpy as np
import pytest

from oracle import cpuref, metrics
from rosylnalive_amd.gpu_core import HipBackend
from rosylnalive_amd.qwen import QwenConfig, QwenModel, inv_freq_bits, synthetic_ids, synthetic_weights

pytestmark = pytest.mark.gpu

MAX_ABS, TOP1 = 2e-2, 0.99


def _near_ties(lg, ol, err):
    gaps = metrics.top1_flip_gaps(lg, ol)
    return bool(np.all(gaps <= 2 * err)), gaps


@pytest.fixture(scope="module")
def qwen06b():
    cfg = QwenConfig.qwen3_0_6b(max_pos=512)
    w = synthetic_weights(cfg, seed=21)
    cos, sin = cpuref.rope_table(inv_freq_bits(128), cfg.max_pos)
    orc = cpuref.QwenOracle(cfg.oracle_dict(), w, cos, sin)
    print(f"Qwen3-0.6B shape, {cfg.param_count()} parameters, oracle threads {cpuref.threads()}", flush=True)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fast", max_tokens=512)
    m.load_weights(w)
    yield cfg, orc, m
    m.close()
    b.close()


def test_qwen3_0_6b_prefill_512_all_logits(qwen06b):
    """Config C: batch 1, 512 prompt ids uniform in [0, 151936); all 512 x 151,936 logits."""
    cfg, orc, m = qwen06b
    ids = synthetic_ids(21, "fullsize/prefill512", 512, cfg.vocab)
    lg, am = m.forward(ids, 0, logits_rows=512)
    ol = orc.forward(orc.new_cache(), 0, ids)
    err, top1 = metrics.max_abs(lg, ol), metrics.top1_agreement(lg, ol)
    ok, gaps = _near_ties(lg, ol, err)
    print(f"0.6B prefill 512, all logits: max-abs {err:.4g} (range {ol.min():.3g}..{ol.max():.3g}), "
          f"top-1 {top1:.4f}, flip gaps {np.round(gaps, 5).tolist()}", flush=True)
    assert np.isfinite(lg).all()
    assert err <= MAX_ABS and top1 >= TOP1 and ok
    assert am == int(np.argmax(lg[-1]))


def test_qwen3_0_6b_greedy_128_plus_256(qwen06b):
    """Config D: a 128-token prompt, then 256 greedy tokens on the device (one persistent launch per token, the KV
    cache growing to 384 positions). The oracle's logits along the device's sequence come from one oracle prefill of
    prompt + ids[:-1] (the oracle's prefill equals its token-by-token decode bit for bit): where the oracle's argmax
    equals the device's id at every step, the device's sequence is the oracle's greedy sequence. Then the same steps
    teacher-forced on the device, each step's logits against the oracle's row."""
    cfg, orc, m = qwen06b
    prompt = synthetic_ids(22, "fullsize/greedy/prompt", 128, cfg.vocab)
    steps = 256
    g = m.greedy(prompt, steps)
    seq = np.concatenate([prompt, g[:-1]]).astype(np.int32)
    ol = orc.forward(orc.new_cache(), 0, seq)[prompt.size - 1:]  # the 256 rows that choose g[0..255]
    oracle_ids = np.argmax(ol, axis=1)
    same = oracle_ids == g
    # teacher-forced: the prefill row, then each decode step fed the device's previous id
    lg0, am0 = m.forward(prompt, 0, logits_rows=1)
    rows = [lg0[0]]
    for s in range(1, steps):
        m.decode_set(int(g[s - 1]), prompt.size + s - 1)
        m.decode_run(1)
        rows.append(m.read_logits(1)[0])
        assert int(m.decode_ids(1)[0]) == int(np.argmax(rows[-1])), s
    lg = np.stack(rows)
    err, top1 = metrics.max_abs(lg, ol), metrics.top1_agreement(lg, ol)
    ok, gaps = _near_ties(lg, ol, err)
    first_flip = int(np.argmin(same)) if not same.all() else None
    print(f"0.6B greedy 128 + 256: device ids equal the oracle's argmax at {int(same.sum())}/{steps} steps "
          f"(first flip {first_flip}); teacher-forced max-abs {err:.4g}, top-1 {top1:.4f}, flip gaps "
          f"{np.round(gaps, 5).tolist()}", flush=True)
    assert am0 == g[0]
    assert err <= MAX_ABS and top1 >= TOP1 and ok
    assert same.mean() >= TOP1
    # every step where the device's greedy id is not the oracle's argmax is a near-tie in the oracle's logits
    assert np.all(ol[~same, oracle_ids[~same]] - ol[~same, g[~same]] <= 2 * err)


def _row_err(dev, ref):
    """Largest |dev - ref| of any row relative to max(1, that row's largest |ref|): fp16 storage of the device's
    cache rows against the oracle's float32 rows."""
    scale = np.maximum(1.0, np.max(np.abs(ref), axis=-1, keepdims=True))
    return float(np.max(np.abs(dev - ref) / scale))


def test_qwen3_0_6b_prefill_2048_against_the_oracle():
    """The 2048-token prefill the MFMA bar is quoted at (one 2048-row forward from position 0: every GEMM on the
    direct-to-LDS loop, the k-split residual GEMMs on three stages, the attention's long tiles split over two
    workgroups): the last 64 rows' logits and the K / V cache rows of layers 0, 14 and 27 (every 64th row and the last
    eight) against the oracle's prefill of the same 2048 ids."""
    cfg = QwenConfig.qwen3_0_6b(max_pos=2048)
    T, rows = 2048, 64
    w = synthetic_weights(cfg, seed=41)
    ids = synthetic_ids(41, "fullsize/prefill2048", T, cfg.vocab)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fast", max_tokens=T)
    try:
        m.load_weights(w)
        lg, am = m.forward(ids, 0, logits_rows=rows)
        picked = np.r_[np.arange(0, T, 64), np.arange(T - 8, T)]
        dev = {(l, which): m.read_cache(l, which, 0, T)[picked] for l in (0, 14, 27) for which in ("k", "v")}
    finally:
        m.close()
        b.close()
    cos, sin = cpuref.rope_table(inv_freq_bits(128), cfg.max_pos)
    orc = cpuref.QwenOracle(cfg.oracle_dict(), w, cos, sin)
    kc, vc = orc.new_cache()
    ol = orc.forward((kc, vc), 0, ids)[-rows:]
    err, top1 = metrics.max_abs(lg, ol), metrics.top1_agreement(lg, ol)
    ok, gaps = _near_ties(lg, ol, err)
    cache = max(_row_err(dev[(l, which)], (kc if which == "k" else vc)[l][picked]) for (l, which) in dev)
    print(f"0.6B prefill 2048, last {rows} rows: max-abs {err:.4g} (range {ol.min():.3g}..{ol.max():.3g}), top-1 "
          f"{top1:.4f}, flip gaps {np.round(gaps, 5).tolist()}; cache rows within {cache:.3g}", flush=True)
    assert np.isfinite(lg).all()
    assert err <= MAX_ABS and top1 >= TOP1 and ok
    assert am == int(np.argmax(lg[-1])) and cache <= 1e-2


def test_qwen3_0_6b_decode_at_4k_context():
    """The 4K regime of batch-1 decode (the context the decode roofline bar is quoted at): a 4096-token prompt
    prefilled on the device in two 2048-row chunks, then 8 greedy decode steps through the persistent step at context
    4097..4104, where each of a KV head's 22 attention splits holds three 64-key chunks.

    - The decode steps: the oracle is run over the device's own K/V caches for positions 0..4095 (read back), fed the
      device's ids, and each step's logits are compared with the device's (max-abs, top-1, near-ties); the rows the
      steps append to every layer's caches are compared with the oracle's.
    - The prefill: the oracle's own prefill of the first 256 tokens gives every layer's cache rows 0..255 exactly;
      the oracle's forward of tokens 4032..4095 over the device's rows 0..4031 gives rows 4032..4095 (the end of the
      second chunk) and the last row's logits, compared with the device's."""
    cfg = QwenConfig.qwen3_0_6b(max_pos=4160)
    T, steps, tail = 4096, 8, 4032
    w = synthetic_weights(cfg, seed=41)
    ids = synthetic_ids(41, "fullsize/ctx4k", T, cfg.vocab)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fast", max_tokens=2048)
    try:
        m.load_weights(w)
        assert m.persistent_decode()
        print("0.6B 4K: prefill of 4096 tokens, then 8 persistent decode steps", flush=True)
        lg_pre, nxt = m.forward(ids, 0, logits_rows=1)
        m.decode_set(int(nxt), T)
        dev_rows, dev_ids = [], []
        for s in range(steps):
            m.decode_run(1)
            dev_rows.append(m.read_logits(1)[0])
            dev_ids.append(int(m.decode_ids(s + 1)[s]))
            assert dev_ids[-1] == int(np.argmax(dev_rows[-1])), s
        kd = np.stack([m.read_cache(l, "k", 0, T + steps) for l in range(cfg.layers)])
        vd = np.stack([m.read_cache(l, "v", 0, T + steps) for l in range(cfg.layers)])
    finally:
        m.close()
        b.close()
    assert np.isfinite(kd).all() and np.isfinite(vd).all()

    cos, sin = cpuref.rope_table(inv_freq_bits(128), cfg.max_pos)
    orc = cpuref.QwenOracle(cfg.oracle_dict(), w, cos, sin)
    # the prefill's first rows: the oracle's own prefill of the first 256 tokens
    kc, vc = orc.new_cache()
    orc.forward((kc, vc), 0, ids[:256])
    head = max(_row_err(kd[:, :256], kc[:, :256]), _row_err(vd[:, :256], vc[:, :256]))
    # the end of the second chunk over the device's rows 0..4031
    kc[:, :tail], vc[:, :tail] = kd[:, :tail], vd[:, :tail]
    ol_tail = orc.forward((kc, vc), tail, ids[tail:])
    tail_rows = max(_row_err(kd[:, tail:T], kc[:, tail:T]), _row_err(vd[:, tail:T], vc[:, tail:T]))
    pre_err = metrics.max_abs(lg_pre, ol_tail[-1:])
    pre_ok, pre_gaps = _near_ties(lg_pre, ol_tail[-1:], max(pre_err, 1e-6))
    # the decode steps over the device's prefill rows, fed the device's ids
    kc[:, :T], vc[:, :T] = kd[:, :T], vd[:, :T]
    feed = [int(nxt)] + dev_ids[:-1]
    ol = np.concatenate([orc.forward((kc, vc), T + s, np.array([feed[s]], np.int32)) for s in range(steps)])
    lg = np.stack(dev_rows)
    err, top1 = metrics.max_abs(lg, ol), metrics.top1_agreement(lg, ol)
    ok, gaps = _near_ties(lg, ol, err)
    appended = max(_row_err(kd[:, T:], kc[:, T:T + steps]), _row_err(vd[:, T:], vc[:, T:T + steps]))
    print(f"0.6B 4K: prefill cache rows 0..255 within {head:.3g}, rows 4032..4095 within {tail_rows:.3g}; last "
          f"prefill row max-abs {pre_err:.4g} (id {nxt}, oracle {int(np.argmax(ol_tail[-1]))}); decode at "
          f"4097..4104: max-abs {err:.4g}, top-1 {top1:.4f} (ids {dev_ids}, oracle {np.argmax(ol, axis=1).tolist()}), "
          f"flip gaps {np.round(gaps, 5).tolist()}; appended rows within {appended:.3g}", flush=True)
    assert head <= 1e-2 and tail_rows <= 1e-2 and appended <= 1e-2
    assert pre_err <= MAX_ABS and pre_ok
    assert err <= MAX_ABS and top1 >= TOP1 and ok


def test_qwen3_1_7b_batch16_context_8192():
    """Config E: Qwen3-1.7B shape, 16 sequences each with 8192 cached positions of N(0, 1) values, two batched greedy
    decode steps (two attention splits per sequence and KV head: one block per CU). Sequences 0, 7 and 15 against the
    oracle over the same caches, read back from the device; the rows the steps append to the caches against the
    oracle's, within fp16 rounding."""
    cfg = QwenConfig.qwen3_1_7b(max_pos=8256)
    B, ctx = 16, 8192
    w = synthetic_weights(cfg, seed=31)
    b = HipBackend(0)
    m = QwenModel(b, cfg, mode="fast", max_tokens=16, batch=B)
    try:
        m.load_weights(w)
        m.fill_cache_random(31, ctx)
        toks = synthetic_ids(31, "fullsize/batch16", B, cfg.vocab)
        ids1 = m.decode_batch(toks, np.full(B, ctx, np.int32), 1)[0]
        lg1 = m.read_logits(B)
        ids2 = m.decode_batch(ids1, np.full(B, ctx + 1, np.int32), 1)[0]
        lg2 = m.read_logits(B)
        assert ids1.tolist() == np.argmax(lg1, axis=1).tolist() and ids2.tolist() == np.argmax(lg2, axis=1).tolist()
        cos, sin = cpuref.rope_table(inv_freq_bits(128), cfg.max_pos)
        orc = cpuref.QwenOracle(cfg.oracle_dict(), w, cos, sin)
        kc, vc = orc.new_cache()
        worst, agree, n, worst_row = 0.0, 0, 0, 0.0
        for s in (0, 7, 15):
            for layer in range(cfg.layers):
                kc[layer, :ctx] = m.read_cache(layer, "k", 0, ctx, seq=s)
                vc[layer, :ctx] = m.read_cache(layer, "v", 0, ctx, seq=s)
            o1 = orc.forward((kc, vc), ctx, [int(toks[s])])
            o2 = orc.forward((kc, vc), ctx + 1, [int(ids1[s])])
            for lg, o in ((lg1[s:s + 1], o1), (lg2[s:s + 1], o2)):
                e = metrics.max_abs(lg, o)
                worst = max(worst, e)
                agree += int(np.argmax(lg[0]) == np.argmax(o[0]))
                n += 1
                assert _near_ties(lg, o, max(e, 1e-6))[0], s
            for layer in (0, cfg.layers // 2, cfg.layers - 1):
                for which, c in (("k", kc), ("v", vc)):
                    dev = m.read_cache(layer, which, ctx, 2, seq=s)
                    ref = c[layer, ctx:ctx + 2]
                    worst_row = max(worst_row, float(np.max(np.abs(dev - ref)) / max(1.0, np.max(np.abs(ref)))))
        print(f"1.7B batch 16 at 8192: sequences 0, 7, 15 x 2 steps: worst logits max-abs {worst:.4g}, top-1 "
              f"{agree}/{n}; appended cache rows within {worst_row:.3g} (relative to max(1, |row|))", flush=True)
        assert worst <= MAX_ABS and agree >= n - 1
        assert worst_row <= 1e-2
    finally:
        m.close()
        b.close()
