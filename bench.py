"""Benchmark of the Qwen3 forward hot path on one MI355X, printing one JSON line.

Headline (value): batch-1 greedy decode tok/s of a Qwen3-0.6B-shaped decoder (28 layers, hidden 1024, 16/8 heads,
head_dim 128, SwiGLU 3072, vocab 151936, tied embeddings, random N(0, 0.02) bf16 weights, norm weights 1): a 128-token
prompt, then W warmup steps and exactly K timed decode steps (one step = one token: one launch of the persistent decode
step, replayed as a HIP graph, position and token in device memory). Defaults K = 256, W = 8: context 136 .. 392.

Also measured in the same run (extra keys, skipped by --no-extras): 512-token prefill with all 512 x 151936 logits,
2048-token prefill with last-row logits, decode at 4096 context, the isolated GQA prefill attention at T = 2048, and the
batched decode of 16 sequences of a Qwen3-1.7B-shaped model at 8K context, and the same decode through the per-stage
kernel list (LRM_HIP_DECODE=kernels). The prefill and attention extras warm up for a second of back-to-back runs, then
report the fastest of seven runs (ms / us) and their median (ms_median / us_median). The roofline is that of the dominant decode kernel (decode_step_persistent, timed
with HIP events on the device stream). cpu_baseline is the oracle on the
host cores on a bounded sample of the decode workload (--no-cpu skips it); cpu_configs times the oracle on the other
workloads (tiny model, attention, 512-token prefill, a sample of the batched decode).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
FP32_PEAK_TFLOPS = 157.3
GEMV_SWIGLU_TRAFFIC_BYTES = 12675736  # measured HBM bytes per gemv_swiglu_dec launch at the 0.6B shape
PERSIST_TRAFFIC_BYTES = 1281006770    # measured HBM bytes per decode_step_persistent launch at context 393..424
ROOFLINE_POS0 = 392                   # the roofline launches run at context ROOFLINE_POS0 + 1 .. ROOFLINE_POS0 + 32
COPY_BYTES = 1 << 30                  # the reference copy of the traffic calibration: 4 x the last-level cache
CPU_DECODE_STEPS = 128                # the bounded CPU decode sample (about 10 s on 16 host cores)
CTX4K_CHECK_STEPS = 8                 # decode steps of the 4K-context leg whose ids the oracle checks
WARM_S, RUNS = 1.0, 7                 # the prefill and attention extras: seconds of warm-up, then timed runs


def reference_copy() -> float:
    """scale_f32 (a = 1) over COPY_BYTES on a backend of its own: COPY_BYTES read and COPY_BYTES written, more than the
    256 MB last-level cache holds, so every byte crosses HBM. The HBM byte counters (FETCH_SIZE, WRITE_SIZE) of a
    profiling run are scaled by what they read for it. Returns its duration in microseconds (HIP events)."""
    from rosylnalive_amd.gpu_core import Arena, ArgBlock, DType, HeapPlanner, HipBackend, TensorTable
    b = HipBackend(0)
    try:
        b.load_kernels()
        n = COPY_BYTES // 4
        planner = HeapPlanner()
        px, py = planner.allocate(Arena.ACTIVATIONS, COPY_BYTES), planner.allocate(Arena.ACTIVATIONS, COPY_BYTES)
        layout = planner.build()
        heap = b.create_heap(layout)
        table = TensorTable(layout)
        tx = table.add_placed("copy.x", px, DType.F32, [n])
        ty = table.add_placed("copy.y", py, DType.F32, [n])
        heap.write_table(table.seal())
        cl = b.begin()
        tm = cl.begin_timer("gpu.scale_f32")
        cl.dispatch("scale_f32", ArgBlock.encode("scale_f32", x=tx, y=ty, n=n, a=1.0))
        cl.end_timer(tm)
        comp = b.wait(b.submit(cl))
        cl.release()
        return comp.timers[0].duration_ns / 1e3
    finally:
        b.close()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_configs(seed, cfg06, w06, threads, e_sample):
    """The oracle timed on the other workloads of the hot path (wall clock, one run each): the tiny model's whole
    run, the isolated attention at T = 2048, the 0.6B prefill of 512 tokens with every logit, and a stated sample of
    the batched 1.7B decode (its 15 GB cache does not fit a CPU run: sequence 0 over the device's own caches at
    context 8192, 2 steps, whose greedy ids are compared with the device's)."""
    from oracle import cpuref
    from rosylnalive_amd.qwen import QwenConfig, inv_freq_bits, synthetic_ids, synthetic_normal_f32, synthetic_weights
    res = {"cores": threads, "kind": "port"}
    # A: tiny plumbing model, prompt 16, 8 greedy tokens
    ca = QwenConfig.tiny_plumbing(max_pos=64)
    wa = synthetic_weights(ca, seed=seed)
    cos, sin = cpuref.rope_table(inv_freq_bits(ca.head_dim), 64)
    oa = cpuref.QwenOracle(ca.oracle_dict(), wa, cos, sin)
    ids = synthetic_ids(seed, "bench/tiny", 16, ca.vocab)
    t0 = time.perf_counter()
    oa.greedy(ids, 8)
    res["A_tiny_run_s"] = round(time.perf_counter() - t0, 4)
    # B: attention only, T = 2048, 16/8 heads, head_dim 128, fp32
    cos, sin = cpuref.rope_table(inv_freq_bits(128), 2048)
    q = synthetic_normal_f32(seed, "bench/attn/q", (2048, 16 * 128))
    k = synthetic_normal_f32(seed, "bench/attn/k", (2048, 8 * 128))
    v = synthetic_normal_f32(seed, "bench/attn/v", (2048, 8 * 128))
    ones = np.full(128, 0x3F80, np.uint16)
    qn = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(q, ones, 1e-6), 16, 0)
    kn = cpuref.rope_apply(cos, sin, cpuref.rmsnorm(k, ones, 1e-6), 8, 0)
    scale = float(cpuref.attention_scale(128, np.float32))
    t0 = time.perf_counter()
    cpuref.attention(qn, kn, v, 16, 8, 128, 0, scale)
    tb = time.perf_counter() - t0
    res["B_attention_2048_s"] = round(tb, 4)
    res["B_attention_2048_gflops"] = round(17288970240 / tb / 1e9, 1)
    # C: 0.6B prefill of 512 tokens, all logits
    cos, sin = cpuref.rope_table(inv_freq_bits(128), 512)
    d = cfg06.oracle_dict()
    d["max_pos"] = 512
    oc = cpuref.QwenOracle(d, w06, cos, sin)
    ids = synthetic_ids(seed, "bench/prefill512", 512, cfg06.vocab)
    t0 = time.perf_counter()
    oc.forward(oc.new_cache(), 0, ids)
    tc = time.perf_counter() - t0
    res["C_prefill_512_s"] = round(tc, 3)
    res["C_prefill_512_tok_s"] = round(512 / tc, 1)
    res["C_prefill_512_gflops"] = round(640588005376 / tc / 1e9, 1)
    del oc
    # E (sample): the 1.7B shape, sequence 0 over the 8192 cached positions the device holds (N(0, 1) fp16), 2 steps
    if e_sample is not None:
        ce = e_sample["cfg"]
        we = synthetic_weights(ce, seed=seed)
        cos, sin = cpuref.rope_table(inv_freq_bits(128), ce.max_pos)
        oe = cpuref.QwenOracle(ce.oracle_dict(), we, cos, sin)
        kc, vc = oe.new_cache()
        for l_ in range(ce.layers):
            kc[l_, :8192] = e_sample["k"][l_]
            vc[l_, :8192] = e_sample["v"][l_]
        tok = np.array([e_sample["tok"]], np.int32)
        ids = []
        t0 = time.perf_counter()
        for s_ in range(2):
            lg = oe.forward((kc, vc), 8192 + s_, tok)
            tok = np.array([int(np.argmax(lg[-1]))], np.int32)
            ids.append(int(tok[0]))
        te = time.perf_counter() - t0
        res["E_sample"] = ("sequence 0 x 2 steps at context 8193..8194 over the device's caches (of the 16-sequence, "
                           "64-step workload)")
        res["E_sample_s"] = round(te, 3)
        res["E_tok_s_per_sequence"] = round(2 / te, 3)
        res["E_ids_equal_device"] = ids == e_sample["ids"]
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["prefill_2048", "prefill_512", "attention_2048", "roofline", "decode_batch16",
                                       "decode_4k"],
                    help="run only this workload (for profiling runs) and print its figures as the JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0 or 128 + args.warmup + args.steps > 4096:
        print("steps + warmup must keep the context within 4096", file=sys.stderr)
        sys.exit(2)

    from oracle import cpuref
    from rosylnalive_amd.gpu_core import ArgBlock, HipBackend
    from rosylnalive_amd.qwen import QwenConfig, QwenModel, inv_freq_bits, synthetic_ids, synthetic_weights

    cfg = QwenConfig.qwen3_0_6b(max_pos=4096 + 256)
    L, H, QH, KVH, HD, I, V = cfg.layers, cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.intermediate, cfg.vocab
    weight_bytes = cfg.param_count() * 2
    lin_params_layer = (QH * HD + 2 * KVH * HD) * H + H * QH * HD + 2 * I * H + H * I

    t0 = time.time()
    weights = synthetic_weights(cfg, seed=args.seed)
    log(f"weights generated in {time.time() - t0:.1f} s ({weight_bytes / 1e9:.3f} GB bf16)")
    backend = HipBackend(0)
    model = QwenModel(backend, cfg, mode="fast", max_tokens=2048)
    model.load_weights(weights)
    log(f"model resident after {time.time() - t0:.1f} s on {backend.info.name} ({backend.info.arch})")

    def kv_bytes(ctx):
        return 2 * L * KVH * ctx * HD * 2

    def timed_runs(run):
        """Warm-up for WARM_S seconds of back-to-back runs, then RUNS more: (fastest, median) of their device times."""
        t_end = time.time() + WARM_S
        while time.time() < t_end:
            run()
        times = sorted(run() for _ in range(RUNS))
        return times[0], times[RUNS // 2]

    def prefill(T, rows, name):
        """The forward of T synthetic tokens, logits of the last `rows` rows: the fastest of the timed runs (device
        time), with their median."""
        ids = synthetic_ids(args.seed, name, T, V)
        best, med = timed_runs(lambda: (model.forward(ids, 0, logits_rows=rows), model.last_ms())[1])
        fl = 2 * T * L * lin_params_layer + 2 * rows * V * H + L * QH * (T * (T + 1) // 2) * (4 * HD + 3)
        return {"ms": round(best, 3), "ms_median": round(med, 3), "tok_s": round(T / (best / 1e3), 1),
                "tflops": round(fl / (best / 1e3) / 1e12, 1),
                "mfma_frac": round(fl / (best / 1e3) / 1e12 / BF16_PEAK_TFLOPS, 4), "flop": fl}

    def attention_2048_us():
        """The isolated GQA prefill attention at T = 2048 on the caches a 2048-token prefill wrote, each layer's in
        turn, 28 launches in one list timed with HIP events."""
        tok = model.token
        cl = backend.begin()
        tm = cl.begin_timer("gpu.attention_prefill_f16")
        for i in range(L):
            cl.dispatch("attention_prefill_f16", ArgBlock.encode(
                "attention_prefill_f16", q=tok("q"), k_cache=tok(f"L{i}.k_cache"), v_cache=tok(f"L{i}.v_cache"),
                y=tok("o"), workspace=tok("attn.ws"), rows=2048, past=0, q_heads=QH, kv_heads=KVH,
                max_pos=cfg.max_pos, scale=float(np.float32(HD ** -0.5))))
        cl.end_timer(tm)
        comp = backend.wait(backend.submit(cl))
        cl.release()
        return comp.timers[0].duration_ns / 1e3 / L

    def attention_2048():
        """attention_2048_us's fastest timed run, with their median."""
        a_us, med = timed_runs(attention_2048_us)
        a_fl = QH * (2048 * 2049 // 2) * (4 * HD + 3)
        return {"us": round(a_us, 2), "us_median": round(med, 2), "tflops": round(a_fl / (a_us * 1e-6) / 1e12, 1),
                "mfma_frac": round(a_fl / (a_us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4), "flop": a_fl}

    def decode_batch16(sample):
        """Config E: Qwen3-1.7B shape, 16 sequences whose caches hold 8192 positions of bf16-valued N(0, 1) (stored
        fp16), 2 warmup + 64 timed steps of all 16 sequences. Returns its figures and, when `sample`, sequence 0's
        caches and ids for the oracle's check."""
        cfg_e = QwenConfig.qwen3_1_7b(max_pos=8192 + 128)
        w_e = synthetic_weights(cfg_e, seed=args.seed)
        be_e = HipBackend(0)
        m_e = QwenModel(be_e, cfg_e, mode="fast", max_tokens=16, batch=16)
        try:
            m_e.load_weights(w_e)
            del w_e
            m_e.fill_cache_random(args.seed, 8192)
            toks = synthetic_ids(args.seed, "bench/batch16", 16, cfg_e.vocab)
            e_ids = m_e.decode_batch(toks, [8192] * 16, 2)
            m_e.decode_batch(toks, [8192] * 16, 64)
            e_ms = m_e.last_ms()
            e_w = cfg_e.param_count() * 2
            e_bytes = sum(e_w + 16 * 2 * cfg_e.layers * cfg_e.kv_heads * (8192 + s + 1) * cfg_e.head_dim * 2
                          for s in range(64))
            res = {"tok_s": round(16 * 64 / (e_ms / 1e3), 1), "ms_per_step": round(e_ms / 64, 4),
                   "gbs": round(e_bytes / (e_ms / 1e3) / 1e9, 1),
                   "hbm_frac": round(e_bytes / (e_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                   "bytes_per_step": int(e_bytes / 64),
                   "workload": "Qwen3-1.7B shape, 16 sequences, context 8193..8256, greedy, skinny MFMA GEMMs over "
                               "fp16 weight copies"}
            smp = None
            if sample:  # sequence 0's caches, for the oracle's sample of this workload
                smp = {"cfg": cfg_e, "tok": int(toks[0]), "ids": e_ids[:, 0].tolist(),
                       "k": [m_e.read_cache(l, "k", 0, 8192, seq=0) for l in range(cfg_e.layers)],
                       "v": [m_e.read_cache(l, "v", 0, 8192, seq=0) for l in range(cfg_e.layers)]}
            return res, smp
        finally:
            m_e.close()
            be_e.close()

    def decode_4k(sample):
        """Decode at 4096 context: a real 4096-token prefill (two chunks), then 4 + 64 decode steps (context 4101 ..
        4164), the 64 timed. Returns its figures and, when `sample`, the prefill's caches and the first ids for the
        oracle's check."""
        ids = synthetic_ids(args.seed, "bench/ctx4k", 4096, V)
        _, nxt = model.forward(ids, 0, logits_rows=1)
        model.decode_set(int(nxt), 4096)
        model.decode_run(4)
        model.decode_run(64)
        d_ms = model.last_ms()
        smp = None
        if sample:  # the prefill's caches and the first ids, for the oracle's check of this leg
            smp = {"first": int(nxt), "ids": model.decode_ids(CTX4K_CHECK_STEPS).tolist(),
                   "k": [model.read_cache(l_, "k", 0, 4096) for l_ in range(L)],
                   "v": [model.read_cache(l_, "v", 0, 4096) for l_ in range(L)]}
        b4 = sum(weight_bytes + kv_bytes(4096 + 4 + s + 1) for s in range(64))
        return {"tok_s": round(64 / (d_ms / 1e3), 1), "ms_per_token": round(d_ms / 64, 4),
                "gbs": round(b4 / (d_ms / 1e3) / 1e9, 1), "hbm_frac": round(b4 / (d_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                "bytes_per_token": int(b4 / 64)}, smp

    if args.only == "decode_4k":
        res, _ = decode_4k(False)
        log(args.only, res)
        print(json.dumps({"workload": args.only, **res}), flush=True)
        model.close()
        backend.close()
        return
    if args.only == "decode_batch16":
        res, _ = decode_batch16(False)
        log(args.only, res)
        print(json.dumps({"workload": args.only, **res}), flush=True)
        model.close()
        backend.close()
        return
    if args.only == "attention_2048":
        prefill(2048, 1, "bench/prefill2048")
        res = attention_2048()
        log(args.only, res)
        print(json.dumps({"workload": args.only, **res}), flush=True)
        model.close()
        backend.close()
        return
    if args.only in ("prefill_2048", "prefill_512"):
        T, rows = (2048, 1) if args.only == "prefill_2048" else (512, 512)
        res = prefill(T, rows, "bench/" + args.only.replace("_", ""))
        log(args.only, res)
        print(json.dumps({"workload": args.only, **res}), flush=True)
        model.close()
        backend.close()
        return

    # ---------------------------------------------------------------- dominant kernel roofline
    # The decode step is one launch of decode_step_persistent (the whole token: every layer, the lm_head and the
    # argmax): its duration per launch, from HIP events on the device stream around `reps` launches recorded in one
    # list, against the algorithmic bytes of each launch (every weight once, the KV cache up to its position, the
    # appended K/V rows and the logits row).
    tok = model.token

    def persist_roofline():
        # at a fixed context, 393..424, whatever --steps is (the context the traffic profile was taken at): a prefill
        # of 392 tokens writes the caches the launches read
        reps = 32
        pos0 = ROOFLINE_POS0
        _, nxt = model.forward(synthetic_ids(args.seed, "bench/roofline", pos0, V), 0, logits_rows=1)
        model.decode_set(int(nxt), pos0)
        cl = backend.begin()
        tm = cl.begin_timer("gpu.decode_step_persistent")
        for _ in range(reps):
            cl.dispatch("decode_step_persistent", ArgBlock.encode(
                "decode_step_persistent", embed=tok("model.embed_tokens.weight"), final_norm=tok("model.norm.weight"),
                in_norm=tok("stack.input_layernorm"), qkv=tok("stack.qkv_proj.f16"), q_norm=tok("stack.q_norm"),
                k_norm=tok("stack.k_norm"), o_proj=tok("stack.o_proj.f16"),
                post_norm=tok("stack.post_attention_layernorm"), gate_up=tok("stack.gate_up_proj.f16"),
                down=tok("stack.down_proj.f16"), k_cache=tok("stack.k_cache"), v_cache=tok("stack.v_cache"),
                cos=tok("rope.cos"), sin=tok("rope.sin"), logits=tok("logits"), state=tok("dec.state"),
                out_ids=tok("dec.out_ids"), exchange=tok("dec.exchange"), embed16=tok("embed.f16"), layers=L,
                hidden=H, q_heads=QH, kv_heads=KVH, inter=I, vocab=V, max_pos=cfg.max_pos, max_steps=cfg.max_pos,
                write_logits=1, eps=cfg.eps, scale=float(np.float32(HD ** -0.5)), blocks=256))
        cl.end_timer(tm)
        comp = backend.wait(backend.submit(cl))
        cl.release()
        p_us = comp.timers[0].duration_ns / 1e3 / reps
        p_bytes = sum(weight_bytes + kv_bytes(pos0 + r + 1) + 2 * L * KVH * HD * 2 + V * 4 for r in range(reps)) / reps
        res = {"us": p_us, "bytes": p_bytes, "gbs": p_bytes / (p_us * 1e-6) / 1e9}
        log(f"decode_step_persistent: {p_us:.2f} us per launch at context {pos0 + 1}..{pos0 + reps}, "
            f"{res['gbs']:.0f} GB/s ({res['gbs'] / HBM_PEAK_GBS:.1%} of HBM peak)")
        return res

    persistent = model.persistent_decode()
    if args.only == "roofline":
        pk = persist_roofline() if persistent else None
        c_us = reference_copy()
        log(f"reference copy (scale_f32, 1 GiB read + 1 GiB written): {c_us:.1f} us, "
            f"{2 * COPY_BYTES / (c_us * 1e-6) / 1e9:.0f} GB/s")
        print(json.dumps({"workload": "roofline", "decode_step_persistent_us": round(pk["us"], 3) if pk else None,
                          "bytes_per_launch": int(pk["bytes"]) if pk else None, "copy_us": round(c_us, 2)}),
              flush=True)
        model.close()
        backend.close()
        return

    # ---------------------------------------------------------------- headline: decode, context 128 + ...
    prompt = synthetic_ids(args.seed, "bench/prompt", 128, V)
    _, first = model.forward(prompt, 0, logits_rows=1)
    model.decode_set(int(first), 128)
    if args.warmup:
        model.decode_run(args.warmup)
    ctx0 = 128 + args.warmup
    t1 = time.perf_counter()
    model.decode_run(args.steps)
    wall = time.perf_counter() - t1
    dev_ms = model.last_ms()
    # the greedy ids of the run (the prefill's, then every decode step's), checked against the oracle's below
    gpu_ids = [int(first)] + model.decode_ids(args.warmup + args.steps).tolist()
    tok_s = args.steps / (dev_ms / 1e3)
    step_bytes = sum(weight_bytes + kv_bytes(ctx0 + s + 1) for s in range(args.steps))
    log(f"decode: {args.steps} steps in {dev_ms:.2f} ms device ({wall * 1e3:.2f} ms wall): {tok_s:.1f} tok/s, "
        f"{step_bytes / (dev_ms / 1e3) / 1e9:.0f} GB/s algorithmic")

    pk = persist_roofline() if persistent else None  # the dominant kernel's roofline (defined above)

    # the fused gate/up SwiGLU GEMV of the per-stage decode list (the dominant kernel of that list)
    reps = 4
    cl = backend.begin()
    tm = cl.begin_timer("gpu.gemv_swiglu_dec")
    for _ in range(reps):
        for i in range(L):
            cl.dispatch("gemv_swiglu_dec", ArgBlock.encode(
                "gemv_swiglu_dec", x=tok("dec.x"), norm=tok(f"model.layers.{i}.post_attention_layernorm.weight"),
                w=tok(f"L{i}.gate_up_proj"), y=tok("dec.a"), inter=I, hidden=H, eps=cfg.eps))
    cl.end_timer(tm)
    comp = backend.wait(backend.submit(cl))
    cl.release()
    launches = reps * L
    k_us = comp.timers[0].duration_ns / 1e3 / launches
    k_bytes = 2 * I * H * 2 + H * 4 + H * 2 + I * 4
    k_gbs = k_bytes / (k_us * 1e-6) / 1e9
    log(f"gemv_swiglu_dec: {k_us:.2f} us per launch, {k_gbs:.0f} GB/s ({k_gbs / HBM_PEAK_GBS:.1%} of HBM peak)")

    # a plain copy of known size larger than the last-level cache, the reference that the HBM byte counters of a
    # profiling run are scaled by
    reference_copy()

    out = {
        "metric": "Qwen3-0.6B prefill & decode tok/s on 1 MI355X; % of HBM/MFMA roofline",
        "value": round(tok_s, 2),
        "unit": "tok/s (batch-1 greedy decode)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dev_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 weights; fp16 MFMA operands and KV cache; fp32 accumulate",
        "data": "synthetic (random N(0,0.02) bf16 weights, norm weights 1, uniform token ids; seed %d)" % args.seed,
        "config": {
            "workload": "Qwen3-0.6B-shaped greedy decode with KV cache, batch 1, prompt 128, then %d warmup + %d timed "
                        "tokens (context %d..%d)" % (args.warmup, args.steps, ctx0 + 1, ctx0 + args.steps),
            "layers": L, "hidden": H, "heads": f"{QH}/{KVH}", "head_dim": HD, "intermediate": I, "vocab": V,
            "batch": 1,
        },
        "roofline": ({
            "bound": "hbm",
            "kernel": "decode_step_persistent",
            "achieved": round(pk["gbs"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(pk["gbs"] / HBM_PEAK_GBS, 4),
            # HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled by the same counters on the 1 GiB
            # reference copy (profiles/decode_persistent_qwen3_0.6b.md)
            "traffic": PERSIST_TRAFFIC_BYTES,
            "bytes_per_launch": int(pk["bytes"]),
            "us_per_launch": round(pk["us"], 3),
        } if persistent else {
            "bound": "hbm",
            "kernel": "gemv_swiglu_dec",
            "achieved": round(k_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(k_gbs / HBM_PEAK_GBS, 4),
            "traffic": GEMV_SWIGLU_TRAFFIC_BYTES,
            "bytes_per_launch": k_bytes,
            "us_per_launch": round(k_us, 3),
        }),
        "decode_path": "decode_step_persistent (one launch per token)" if persistent else
                       "per-stage kernel list (171 launches per token, one HIP graph)",
        "gemv_swiglu_dec": {"us_per_launch": round(k_us, 3), "gbs": round(k_gbs, 1),
                            "frac": round(k_gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": k_bytes,
                            # profiles/decode_gemv_traffic_qwen3_0.6b.md
                            "traffic": GEMV_SWIGLU_TRAFFIC_BYTES},
        "decode_step_roofline": {
            "bound": "hbm",
            "achieved": round(step_bytes / (dev_ms / 1e3) / 1e9, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(step_bytes / (dev_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "bytes_per_token": int(step_bytes / args.steps),
        },
    }

    e_sample = ctx4k_sample = None
    if not args.no_extras:
        # 512-token prefill with every logit row (all 512 x 151936 logits)
        out["prefill_512_all_logits"] = prefill(512, 512, "bench/prefill512")
        log("prefill 512:", out["prefill_512_all_logits"])
        # 2048-token prefill, last-row logits
        out["prefill_2048"] = prefill(2048, 1, "bench/prefill2048")
        log("prefill 2048:", out["prefill_2048"])
        # the isolated GQA prefill attention at T = 2048 on the caches the prefill just wrote
        out["attention_prefill_2048"] = attention_2048()
        log("attention 2048:", out["attention_prefill_2048"])
        out["decode_4k"], ctx4k_sample = decode_4k(not args.no_cpu)
        log("decode 4k:", out["decode_4k"])

        # the same decode workload through the per-stage kernel list (171 launches per token in one HIP graph)
        if persistent:
            os.environ["LRM_HIP_DECODE"] = "kernels"
            be_k = HipBackend(0)
            m_k = QwenModel(be_k, cfg, mode="fast", max_tokens=256)
            os.environ.pop("LRM_HIP_DECODE", None)
            m_k.load_weights(weights)
            _, f_k = m_k.forward(prompt, 0, logits_rows=1)
            m_k.decode_set(int(f_k), 128)
            if args.warmup:
                m_k.decode_run(args.warmup)
            m_k.decode_run(args.steps)
            k_ms = m_k.last_ms()
            out["decode_kernel_list"] = {"tok_s": round(args.steps / (k_ms / 1e3), 1),
                                         "ms_per_token": round(k_ms / args.steps, 4),
                                         "workload": "the headline workload, LRM_HIP_DECODE=kernels"}
            log("decode through the kernel list:", out["decode_kernel_list"])
            m_k.close()
            be_k.close()

        out["decode_batch16_1.7b_8k"], e_sample = decode_batch16(not args.no_cpu)
        log("decode batch 16 (1.7B, 8K):", out["decode_batch16_1.7b_8k"])

    if not args.no_cpu:
        # The oracle (CpuRef F32 restated in C, parallel over independent outputs) on the host's cores.
        # Headline baseline: the decode workload itself, bounded: the same 128-token prompt, then CPU_DECODE_STEPS greedy
        # steps of the same model; value = decode tok/s over those steps.
        threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
        cpuref.set_threads(threads)
        cpu_model = _cpu_model()
        cos, sin = cpuref.rope_table(inv_freq_bits(HD), 512)
        ocfg = cfg.oracle_dict()
        ocfg["max_pos"] = 512
        orc = cpuref.QwenOracle(ocfg, weights, cos, sin)
        cache = orc.new_cache()
        t2 = time.perf_counter()
        lg = orc.forward(cache, 0, prompt)
        t_pre = time.perf_counter() - t2
        nxt = int(np.argmax(lg[-1]))
        cpu_ids = [nxt]
        t3 = time.perf_counter()
        steps = CPU_DECODE_STEPS
        for s_ in range(steps):
            lg = orc.forward(cache, 128 + s_, np.array([nxt], np.int32))
            nxt = int(np.argmax(lg[-1]))
            cpu_ids.append(nxt)
        t_dec = time.perf_counter() - t3
        # the oracle's greedy ids against the device's over the ids both runs produced
        n_cmp = min(len(gpu_ids), len(cpu_ids))
        same = [a == b for a, b in zip(gpu_ids[:n_cmp], cpu_ids[:n_cmp])]
        prefix = same.index(False) if False in same else n_cmp
        out["ids_vs_oracle"] = {"compared": n_cmp, "equal": int(sum(same)), "identical_prefix": prefix,
                                "what": "greedy ids of the headline decode (the prefill's id, then each step's) against "
                                        "the oracle's greedy ids from the same prompt"}
        log("greedy ids vs oracle:", out["ids_vs_oracle"])
        out["cpu_baseline"] = {"value": round(steps / t_dec, 4), "unit": "tok/s (batch-1 decode)", "cores": threads,
                               "kind": "port", "cpu": cpu_model,
                               "sample": f"oracle (CpuRef F32 in C) on the same weights: 128-token prefill "
                                         f"({t_pre:.2f} s, {128 / t_pre:.1f} tok/s) then {steps} greedy decode steps, "
                                         f"context 129..{128 + steps} ({t_dec:.2f} s)"}
        log("cpu baseline:", out["cpu_baseline"])
        if ctx4k_sample is not None:
            # the 4K-context leg's first steps: the oracle over the device's own prefill caches (positions 0..4095),
            # fed the device's ids; its argmax at each step against the device's id
            cos4, sin4 = cpuref.rope_table(inv_freq_bits(HD), 4096 + 64)
            ocfg4 = cfg.oracle_dict()
            ocfg4["max_pos"] = 4096 + 64
            o4 = cpuref.QwenOracle(ocfg4, weights, cos4, sin4)
            kc4, vc4 = o4.new_cache()
            for l_ in range(L):
                kc4[l_, :4096] = ctx4k_sample["k"][l_]
                vc4[l_, :4096] = ctx4k_sample["v"][l_]
            feed = [ctx4k_sample["first"]] + ctx4k_sample["ids"][:-1]
            t4 = time.perf_counter()
            o_ids = [int(np.argmax(o4.forward((kc4, vc4), 4096 + s_, np.array([feed[s_]], np.int32))[-1]))
                     for s_ in range(CTX4K_CHECK_STEPS)]
            same4 = [a == b for a, b in zip(ctx4k_sample["ids"], o_ids)]
            out["decode_4k"]["ids_vs_oracle"] = {
                "compared": CTX4K_CHECK_STEPS, "equal": int(sum(same4)), "oracle_s": round(time.perf_counter() - t4, 2),
                "what": "the first %d decode steps' greedy ids (context 4097..%d) against the oracle's argmax, the "
                        "oracle run over the device's prefill caches (read back) and fed the device's ids"
                        % (CTX4K_CHECK_STEPS, 4096 + CTX4K_CHECK_STEPS)}
            log("decode 4k ids vs oracle:", out["decode_4k"]["ids_vs_oracle"])
            del kc4, vc4, o4, ctx4k_sample
        if not args.no_extras:
            out["cpu_configs"] = cpu_configs(args.seed, cfg, weights, threads, e_sample)
            log("cpu configs:", out["cpu_configs"])

    model.close()
    backend.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
