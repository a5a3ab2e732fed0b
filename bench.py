"""Benchmark of the speculative-decoding verify step on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--config c3|c4|c1]
                    [--cpu-baseline auto|skip] [--no-kernel-timing] [--eager]

One step = one verify pass over K+1 rows: embedding, every layer (fused QKV
GEMV + RoPE + paged KV append, paged attention, o_proj + residual, gate/up
GEMV + SwiGLU, down + residual), LM head, greedy acceptance and KV rollback,
replayed from a captured hipGraph with the model, cache and drafts resident in
HBM.  The default workload is c3 (Llama-3.2-1B shape, int8 per-channel
weights, fp16 activations, K=5, a 2048-token context prefilled by the model
itself from random tokens, 16-token pages scattered over the pool).

Drafts are the target's own greedy continuation, so all K drafts are accepted
(the verify work does not depend on the drafts); the same step with random
drafts is timed as well and reported beside it.

Output: one JSON line (metric, value, ... roofline, cpu_baseline, parity).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "opure-voxelengine_amd"))

import opure_hip as H  # noqa: E402
import synth  # noqa: E402

HBM_PEAK_GBS = 8000.0


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


class Verify:
    """Device buffers and argument block for verify steps of one shape."""

    def __init__(self, dev, model, kv_desc, B, R, max_ctx):
        self.dev, self.model, self.B, self.R, self.max_ctx = dev, model, B, R, max_ctx
        V = model.cfg["vocab"]
        self.kv_desc = kv_desc
        self.tokens = dev.alloc(B * R * 4)
        self.seq_len = dev.alloc(B * 4)
        self.new_len = dev.alloc(B * 4)
        self.logits = dev.alloc(B * R * V * 4)
        self.out_tokens = dev.alloc(B * R * 4)
        self.accepted = dev.alloc(B * 4)
        H.check(H.lib().opure_verify_reserve(dev.h, C.byref(model.desc), B, R, max_ctx))

    def args(self, accept):
        a = H.VerifyArgs()
        a.model = C.pointer(self.model.desc)
        a.kv = C.pointer(self.kv_desc)
        a.batch, a.rows, a.max_ctx = self.B, self.R, self.max_ctx
        a.tokens, a.seq_len, a.logits = int(self.tokens), int(self.seq_len), int(self.logits)
        a.accept_mode = accept
        a.out_tokens, a.accepted = int(self.out_tokens), int(self.accepted)
        a.rollback = 1 if accept else 0
        a.new_seq_len = int(self.new_len)
        self._a = a
        return a

    def run(self, tokens, seq_len, accept=H.ACCEPT_NONE):
        self.dev.write(self.tokens, np.ascontiguousarray(tokens, np.int32))
        self.dev.write(self.seq_len, np.ascontiguousarray(seq_len, np.int32))
        H.check(H.lib().opure_verify_step(self.dev.h, C.byref(self.args(accept))))

    def logits_host(self, rows=None):
        V = self.model.cfg["vocab"]
        return self.dev.download(self.logits, np.float32, (self.B, self.R, V))


def build_workload(dev, cfg_name, seed=1234):
    cfg = dict(synth.CONFIGS[cfg_name])
    K, ctx = cfg["K"], cfg["ctx"]
    R = K + 1
    t0 = time.time()
    model = synth.SynthModel(dev, cfg, seed=seed, max_pos=ctx + 64)
    log(f"model {cfg_name} built on device in {time.time() - t0:.1f}s")
    rng = np.random.default_rng(seed)
    n_pages = (ctx + R + 15) // 16 + 8
    kv = H.DeviceKV(dev, cfg, n_pages, 1, n_pages)
    pt = rng.permutation(n_pages).astype(np.int32)[None, :]
    kv.set_page_table(pt)
    # prefill: the model itself writes the context's K/V, 16 rows per step
    prompt = rng.integers(0, cfg["vocab"], size=ctx).astype(np.int32)
    pre = Verify(dev, model, kv.desc, 1, 16, ctx + R)
    t0 = time.time()
    for s in range(0, ctx - 16, 16):
        pre.run(prompt[None, s:s + 16], [s])
    last = ctx - (ctx - 16) // 16 * 16 if ctx > 16 else ctx
    tail = Verify(dev, model, kv.desc, 1, last, ctx + R)
    tail.run(prompt[None, ctx - last:], [ctx - last])
    dev.sync()
    nxt = int(np.argmax(tail.logits_host()[0, -1]))
    log(f"prefilled {ctx} tokens in {time.time() - t0:.2f}s")
    # self-drafts: the target's greedy continuation, one row at a time
    one = Verify(dev, model, kv.desc, 1, 1, ctx + R)
    drafts = []
    tok = nxt
    for j in range(K):
        one.run([[tok]], [ctx + j])
        tok = int(np.argmax(one.logits_host()[0, 0]))
        drafts.append(tok)
    step = Verify(dev, model, kv.desc, 1, R, ctx + R)
    return dict(cfg=cfg, model=model, kv=kv, step=step, tokens=np.array([[nxt] + drafts], np.int32),
                ctx=ctx, R=R, K=K, rng=rng)


def time_graph(dev, step, tokens, ctx, warmup, steps, eager=False):
    """Times `steps` verify steps replayed from one captured hipGraph (or, with
    `eager`, launched one by one; profilers that do not follow graph replays
    see the same kernels that way)."""
    step.dev.write(step.tokens, tokens)
    step.dev.write(step.seq_len, np.array([ctx], np.int32))
    a = step.args(H.ACCEPT_GREEDY)
    if eager:
        def launch():
            H.check(H.lib().opure_verify_step(dev.h, C.byref(a)))
        g = None
    else:
        dev.graph_begin()
        H.check(H.lib().opure_verify_step(dev.h, C.byref(a)))
        g = dev.graph_end()

        def launch():
            dev.graph_launch(g)
    for _ in range(warmup):
        launch()
    dev.sync()
    t0 = time.perf_counter()
    dev.timer_begin()
    for _ in range(steps):
        launch()
    dev.timer_end()
    gpu_ms = dev.timer_ms()
    dev.sync()
    wall_ms = (time.perf_counter() - t0) * 1e3
    acc = dev.download(step.accepted, np.int32, (1,))
    out = dev.download(step.out_tokens, np.int32, (1, step.R))
    if g is not None:
        dev.graph_destroy(g)
    return dict(ms_per_step=gpu_ms / steps, wall_ms_per_step=wall_ms / steps, accepted=int(acc[0]),
                out_tokens=out[0].tolist())


def time_stages(dev, step, tokens, ctx, steps):
    """Per-stage timing of eager verify steps (opure_profile_*): every kernel of
    a stage is launched with start/stop events stamped by its own dispatch, so
    a stage's time is its kernels' execution time -- what a profiler's kernel
    trace reports -- without the gaps between launches."""
    step.dev.write(step.tokens, tokens)
    step.dev.write(step.seq_len, np.array([ctx], np.int32))
    a = step.args(H.ACCEPT_GREEDY)
    for _ in range(3):
        H.check(H.lib().opure_verify_step(dev.h, C.byref(a)))
    dev.sync()
    dev.profile(True)
    for _ in range(steps):
        H.check(H.lib().opure_verify_step(dev.h, C.byref(a)))
    prof = dev.profile_read()
    dev.profile(False)
    cfg = step.model.cfg
    out = {}
    for st, (n, ms) in prof.items():
        if n == 0:
            continue
        avg_us = ms * 1e3 / n
        by = synth.stage_bytes(cfg, st, step.B * step.R, ctx)
        out[st] = dict(launches_per_step=n / steps, avg_us=avg_us, us_per_step=ms * 1e3 / steps,
                       bytes_per_launch=by, gbs=by / (avg_us * 1e-6) / 1e9 if by else None)
    return out


def cpu_threads():
    """Host threads for the all-cores oracle run: the process's CPU affinity,
    at most 16 (a one-GPU share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(dev, w, gpu_logits, gpu_accept):
    """The CPU oracle timed on one verify step of the same workload, after
    downloading the device's model and cache: on all host cores (its GEMVs split
    over output rows, every output computed exactly as on one core), then on
    one core when that is expected to take at most about 30 s.  The one-core
    figure is the baseline when it was measured; the all-cores one is reported
    beside it."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    m, cfg, step = w["model"], w["cfg"], w["step"]
    t0 = time.time()
    host = m.download()
    hm = O.HostModel.from_arrays(cfg, host)
    kvd = w["kv"]
    kv = O.HostKV(hm, n_pages=kvd.n_pages, batch=1, max_pages_per_seq=kvd.max_pages)
    kv.pool[...] = kvd.get_pool()
    kv.page_table[...] = kvd.get_page_table()
    log(f"downloaded model + cache for the oracle in {time.time() - t0:.1f}s")
    sample = f"one {cfg['n_layers']}-layer verify step ({w['R']} rows, ctx {w['ctx']}) of the same workload"
    n_all = cpu_threads()
    O.set_threads(n_all)
    t0 = time.perf_counter()
    want = O.verify_forward(hm, kv, w["tokens"], np.array([w["ctx"]], np.int32))
    dt_all = time.perf_counter() - t0
    out, acc = O.accept_greedy(want, w["tokens"][:, 1:])
    all_cores = dict(value=(int(acc[0]) + 1) / dt_all, unit="accepted tokens/s", cores=n_all, kind="port",
                     sample=f"{sample} through the oracle, GEMVs over {n_all} threads: {dt_all:.1f}s")
    base = dict(all_cores)
    if n_all == 1 or dt_all <= 2.5:
        O.set_threads(1)
        t0 = time.perf_counter()
        want1 = O.verify_forward(hm, kv, w["tokens"], np.array([w["ctx"]], np.int32))
        dt = time.perf_counter() - t0
        assert np.array_equal(want1, want), "the oracle's result depends on its thread count"
        base = dict(value=(int(acc[0]) + 1) / dt, unit="accepted tokens/s", cores=1, kind="port",
                    sample=f"{sample} through the scalar oracle on one core: {dt:.1f}s")
        base["all_cores"] = all_cores
    else:
        base["one_core"] = (f"skipped: {dt_all:.0f}s on {n_all} threads; the all-cores figure is the baseline")
    O.set_threads(1)
    err = float(np.abs(gpu_logits - want).max())
    s = np.sort(want.astype(np.float64), axis=-1)
    gap = float((s[..., -1] - s[..., -2]).min())
    return base, dict(
        logits_max_abs=err, oracle_min_top2_gap=gap, accepted_equal=bool(acc[0] == gpu_accept["accepted"]),
        tokens_equal=bool(out[0].tolist() == gpu_accept["out_tokens"]))


def bench_c5(args):
    """Batched stochastic verify at the 1B int8 shape: 32 sequences with ragged
    contexts ~U[512, 8192] (16-token pages scattered over one pool), K=6 drafts
    each (7 rows, 224 rows in all), drafts sampled at temperature 0.8 from
    synthetic draft logits, rejection sampling at temperature 0.8 with Philox
    keyed by (seed, sequence, position), per-sequence rollback.  The cache
    holds seeded random K/V (the verify work does not depend on its values).
    One step = one verify step of all 32 sequences, replayed from a hipGraph."""
    cfg = dict(synth.CONFIGS["c3"])
    B, K, tau, seed = 32, 6, 0.8, 2025
    R = K + 1
    V, L, nkv, hd = cfg["vocab"], cfg["n_layers"], cfg["n_kv_heads"], cfg["head_dim"]
    dev = H.Dev(0)
    log("device", dev.name)
    peak = measure_peak(dev)
    rng = np.random.default_rng(seed)
    ctx = rng.integers(512, 8193, size=B).astype(np.int32)
    need = (ctx + R + 15) // 16
    n_pages = int(need.sum()) + 64
    maxp = int(need.max()) + 1
    max_ctx = int(ctx.max()) + R
    model = synth.SynthModel(dev, cfg, seed=1234, max_pos=max_ctx + 64)
    kv = H.DeviceKV(dev, cfg, n_pages, B, maxp)
    perm = rng.permutation(n_pages).astype(np.int32)
    pt = np.full((B, maxp), -1, np.int32)
    o = 0
    for b in range(B):
        pt[b, :need[b]] = perm[o:o + need[b]]
        o += need[b]
    kv.set_page_table(pt)
    # seeded random K/V in 64M-element pieces (fp32 staging, converted to fp16)
    L_ = H.lib()
    total = L * n_pages * 2 * nkv * 16 * hd
    piece = 64 << 20
    tmp = dev.alloc(piece * 4)
    for i, off in enumerate(range(0, total, piece)):
        n = min(piece, total - off)
        H.check(L_.opure_synth_normal_f32(dev.h, int(tmp), n, seed, 1000 + i, 1.0, 0.0))
        H.check(L_.opure_convert_f32(dev.h, int(tmp), int(kv.pool) + off * 2, cfg["afmt"], n))
    tmp.free()
    log(f"{B} sequences, contexts {ctx.min()}..{ctx.max()} (sum {int(ctx.sum())}), {n_pages} pages of 16 tokens")
    step = Verify(dev, model, kv.desc, B, R, max_ctx)
    draft = dev.alloc(B * K * V * 4)
    H.check(L_.opure_synth_normal_f32(dev.h, int(draft), B * K * V, seed, 7, 2.0, 0.0))
    pos = dev.upload((ctx[:, None] + np.arange(K)[None]).astype(np.uint32).ravel())
    seqs = dev.upload(np.repeat(np.arange(B, dtype=np.uint32), K))
    dtok = dev.alloc(B * K * 4)
    sa = H.SampleArgs(B * K, V, int(draft), tau, seed, int(pos), int(seqs), 0, int(dtok))
    H.check(L_.opure_sample_rows(dev.h, C.byref(sa)))
    last = rng.integers(0, V, size=B).astype(np.int32)
    drafts = dev.download(dtok, np.int32, (B, K))
    tokens = np.concatenate([last[:, None], drafts], axis=1).astype(np.int32)
    pos_base = dev.upload(ctx.astype(np.uint32))
    dev.write(step.tokens, tokens)
    dev.write(step.seq_len, ctx)
    a = step.args(H.ACCEPT_REJECTION)
    a.draft_logits = int(draft)
    a.temperature = tau
    a.seed = seed
    a.pos_base = int(pos_base)
    H.check(L_.opure_verify_reserve(dev.h, C.byref(model.desc), B, R, max_ctx))

    def launch():
        H.check(L_.opure_verify_step(dev.h, C.byref(a)))

    launch()
    dev.sync()
    if args.eager:
        g = None
        run = launch
    else:
        dev.graph_begin()
        launch()
        g = dev.graph_end()

        def run():
            dev.graph_launch(g)
    for _ in range(args.warmup):
        run()
    dev.sync()
    t0 = time.perf_counter()
    dev.timer_begin()
    for _ in range(args.steps):
        run()
    dev.timer_end()
    ms = dev.timer_ms() / args.steps
    dev.sync()
    wall = (time.perf_counter() - t0) * 1e3 / args.steps
    acc = dev.download(step.accepted, np.int32, (B,))
    value = float(acc.sum() + B) / (ms * 1e-3)
    wbytes = synth.verify_bytes(cfg, B * R, 0)["weights"]
    kvbytes = int(sum(synth.verify_bytes(cfg, R, int(c))["kv"] for c in ctx))
    lbytes = B * R * V * 4 + B * K * V * 4
    step_bytes = wbytes + kvbytes + lbytes
    log(f"c5 verify step {ms * 1e3:.1f} us, accepted {acc.tolist()}, {step_bytes / (ms * 1e-3) / 1e9:.0f} GB/s")
    stages = None
    if not args.no_kernel_timing:
        for _ in range(2):
            launch()
        dev.sync()
        dev.profile(True)
        for _ in range(5):
            launch()
        prof = dev.profile_read()
        dev.profile(False)
        stages = {st: dict(avg_us=msx * 1e3 / n, us_per_step=msx * 1e3 / 5, launches_per_step=n / 5)
                  for st, (n, msx) in prof.items() if n}
        att = stages.get("attention")
        if att:
            att_bytes = kvbytes / L
            att["gbs"] = att_bytes / (att["avg_us"] * 1e-6) / 1e9
            att["bytes_per_launch"] = int(att_bytes)
        for st, d in stages.items():
            log(f"stage {st:10s} x{d['launches_per_step']:4.0f}/step  {d['avg_us']:8.2f} us/launch  "
                f"{d['us_per_step']:8.1f} us/step")
    line = {
        "metric": "accepted tokens/s of the batched stochastic verify step (1B int8, batch 32, K=6)",
        "value": round(value, 1), "unit": "accepted tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 weights, f16 activations, f32 accumulate",
        "data": "synthetic: seeded N(0,0.02) int8 weights, seeded random K/V, N(0,2) draft logits",
        "config": {"workload": f"c5: verify step of 32 sequences x 7 rows (224 rows), Llama-3.2-1B-shape int8/fp16, "
                               f"contexts {int(ctx.min())}..{int(ctx.max())} (sum {int(ctx.sum())}), pages scattered "
                               "over one pool, drafts at T=0.8, rejection sampling at T=0.8 + rollback, "
                               + ("eager launches" if args.eager else "hipGraph replay"),
                   "accepted": acc.tolist(), "step_bytes": int(step_bytes),
                   "step_GBps": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                   "step_frac_of_hbm_peak": round(step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "wall_ms_per_step": round(wall, 4)},
    }
    if stages and "attention" in stages:
        att = stages["attention"]
        line["roofline"] = {"bound": "hbm", "achieved": round(att["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(att["gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                            "kernel": "paged attention (k_attn_mfma + k_attn_combine) of one layer, K/V bytes",
                            "bytes_per_launch": att["bytes_per_launch"], "avg_us": round(att["avg_us"], 2),
                            "measured_peak_GBps": peak["read_GBps"],
                            "frac_of_measured_peak": round(att["gbs"] / peak["read_GBps"], 4), "measured_peak": peak}
        line["stages_us_per_step"] = {st: round(d["us_per_step"], 1) for st, d in stages.items()}
    if args.cpu_baseline == "auto":
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        got = step.logits_host()
        host = model.download()
        hm = O.HostModel.from_arrays(cfg, host)
        # sequence 0 alone through the oracle: its pages copied into a small host pool
        n0 = int(need[0])
        kvh = O.HostKV(hm, n_pages=n0, batch=1, max_pages_per_seq=n0)
        page_bytes = 2 * nkv * 16 * hd * 2
        for layer in range(L):
            for i in range(n0):
                src = (layer * n_pages + int(pt[0, i])) * page_bytes
                kvh.pool[layer, i] = dev.download(kv.pool, np.uint16, (2, nkv, 16, hd), offset=src)
        kvh.page_table[0] = np.arange(n0)
        O.set_threads(1)
        t0 = time.perf_counter()
        want0 = O.verify_forward(hm, kvh, tokens[:1], ctx[:1])
        dt = time.perf_counter() - t0
        q = dev.download(draft, np.float32, (B, K, V))
        w_out, w_acc, _ = O.accept_rejection(got, q, tokens[:, 1:], tau, seed, ctx.astype(np.uint32))
        out = dev.download(step.out_tokens, np.int32, (B, R))
        line["cpu_baseline"] = {"value": round((int(w_acc[0]) + 1) / dt, 4), "unit": "accepted tokens/s", "cores": 1,
                                "kind": "port",
                                "sample": f"sequence 0 alone ({R} rows over its {int(ctx[0])}-token context) through the "
                                          f"scalar oracle: {dt:.1f}s"}
        line["parity"] = {"seq0_logits_max_abs": float(np.abs(got[0] - want0[0]).max()),
                          "accepted_equal": bool(np.array_equal(w_acc, acc)),
                          "tokens_equal": bool(np.array_equal(w_out, out))}
        log("cpu baseline", line["cpu_baseline"], "parity", line["parity"])
    print(json.dumps(line), flush=True)
    if g is not None:
        dev.graph_destroy(g)
    dev.close()


def bench_c1(args):
    """Greedy speculative generation through the native engine
    (libopure_engine.so): SmolLM-135M-shaped fp32 target (30 layers) and a
    2-layer draft of the same width, both seeded N(0,0.02), a 32-token random
    prompt, K=4 drafts per verify step, 64 new tokens.  A step is one whole
    generation of 64 tokens (prefill excluded); value = new tokens / s."""
    import opure_engine as E
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import spec_loop
    cfg = synth.CONFIGS["c1"]
    n_new, K, P = 64, 4, 32
    dev = H.Dev(0)
    log("device", dev.name)
    max_pos = P + n_new + 2 * K + 16
    tgt = synth.SynthModel(dev, cfg, seed=1234, max_pos=max_pos)
    drf = synth.SynthModel(dev, dict(cfg, n_layers=2), seed=4321, max_pos=max_pos)
    prompt = np.random.default_rng(7).integers(0, cfg["vocab"], P).astype(np.int32)
    eng = E.Engine(dev, tgt.desc, drf.desc, max_positions=max_pos, draft_tokens=K, use_graphs=not args.eager)
    for _ in range(max(1, args.warmup // 5)):
        eng.generate_speculative(prompt, n_new)
        eng.generate(prompt, n_new)
    runs = max(1, args.steps // 10)
    spec_ms, greedy_ms, hist = [], [], None
    for _ in range(runs):
        out, hist, st = eng.generate_speculative(prompt, n_new)
        spec_ms.append(st.ms_generate)
        g, gst = eng.generate(prompt, n_new)
        greedy_ms.append(gst.ms_generate)
    ms = float(np.median(spec_ms))
    gms = float(np.median(greedy_ms))
    value = n_new / (ms * 1e-3)
    log(f"speculative: {ms:.2f} ms for {n_new} tokens ({st.verify_steps} verify + {st.draft_steps} draft steps, "
        f"accepted per step {hist.tolist()}); greedy: {gms:.2f} ms")
    wbytes = synth.verify_bytes(cfg, 1, P + n_new // 2)["weights"]
    line = {
        "metric": "new tokens/s of greedy speculative generation (SmolLM-135M-shape fp32 + 2-layer draft, K=4)",
        "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": runs, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic: seeded N(0,0.02) target and draft, uniform random 32-token prompt",
        "config": {"workload": "c1: native engine GenerateSpeculative, 30-layer target + 2-layer draft, 32-token "
                               "prompt, K=4, 64 new tokens, one step = the whole generation (prefill excluded), "
                               + ("eager launches" if args.eager else "one hipGraph per speculative iteration"),
                   "accepted_per_verify_step": hist.tolist(), "verify_steps": int(st.verify_steps),
                   "draft_steps": int(st.draft_steps), "greedy_ms": round(gms, 4),
                   "greedy_tokens_per_s": round(n_new / (gms * 1e-3), 1),
                   "target_weight_bytes": int(wbytes),
                   "speculative_acceptance": round(eng.metrics().speculative_acceptance, 4)},
    }
    if args.cpu_baseline == "auto":
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        hm = O.HostModel.from_arrays(tgt.cfg, tgt.download())
        npg = (max_pos + 15) // 16
        kv = O.HostKV(hm, n_pages=npg, batch=1, max_pages_per_seq=npg)
        kv.page_table[0] = np.arange(npg)
        O.set_threads(1)
        n_cpu = 4

        def step(_k, toks, ctx):
            return O.verify_forward(hm, kv, toks, np.array([ctx], np.int32))

        t0 = time.perf_counter()
        want, _ = spec_loop.greedy(step, list(prompt), n_cpu)
        dt = time.perf_counter() - t0
        line["cpu_baseline"] = {"value": round(n_cpu / dt, 3), "unit": "tokens/s", "cores": 1, "kind": "port",
                                "sample": f"greedy decoding of {n_cpu} tokens after the 32-token prompt through the "
                                          f"scalar oracle (prefill included): {dt:.1f}s"}
        line["parity"] = {"speculative_equals_greedy": bool(np.array_equal(out, g)),
                          "first_tokens_equal_oracle": bool(g[:n_cpu].tolist() == want)}
        log("cpu baseline", line["cpu_baseline"], "parity", line["parity"])
    print(json.dumps(line), flush=True)
    eng.close()
    dev.close()


def bench_c2(args):
    """The isolated acceptance stage: rejection sampling over target logits
    [64][9][49152] and draft logits [64][8][49152] (fp32, N(0,3) from Philox),
    drafts sampled from the draft softmax at temperature 1 (Philox stream 0),
    accept uniforms on stream 1, residual / bonus draws on stream 2.  Three
    input sets (226 MB each) rotate so the 256 MB last-level cache cannot
    serve a set twice in a row.  One step = one opure_accept_rejection call
    that also writes the [64][49152] distribution of each final draw."""
    B, K, V, tau, seed = 64, 8, 49152, 1.0, 2024
    dev = H.Dev(0)
    log("device", dev.name)
    peak = measure_peak(dev)
    L = H.lib()
    sets = []
    for i in range(3):
        t = dev.alloc(B * (K + 1) * V * 4)
        q = dev.alloc(B * K * V * 4)
        H.check(L.opure_synth_normal_f32(dev.h, int(t), B * (K + 1) * V, seed + i, 0, 3.0, 0.0))
        H.check(L.opure_synth_normal_f32(dev.h, int(q), B * K * V, seed + i, 1, 3.0, 0.0))
        pos = dev.upload(np.tile(np.arange(K, dtype=np.uint32), B))
        seq = dev.upload(np.repeat(np.arange(B, dtype=np.uint32), K))
        d = dev.alloc(B * K * 4)
        sa = H.SampleArgs(B * K, V, int(q), tau, seed + i, int(pos), int(seq), 0, int(d))
        H.check(L.opure_sample_rows(dev.h, C.byref(sa)))
        pb = dev.upload(np.full(B, 0, np.uint32))
        ot, ac, di = dev.alloc(B * (K + 1) * 4), dev.alloc(B * 4), dev.alloc(B * V * 4)
        a = H.AcceptArgs(B, K, V, int(t), int(q), int(d), K, tau, seed + i, int(pb), int(ot), int(ac), int(di))
        sets.append(dict(t=t, q=q, d=d, pos=pos, seq=seq, pb=pb, ot=ot, ac=ac, di=di, a=a))
    dev.sync()

    def launch(i):
        H.check(L.opure_accept_rejection(dev.h, C.byref(sets[i % 3]["a"])))

    for i in range(args.warmup):
        launch(i)
    dev.sync()
    t0 = time.perf_counter()
    dev.timer_begin()
    for i in range(args.steps):
        launch(i)
    dev.timer_end()
    ms = dev.timer_ms() / args.steps
    dev.sync()
    wall = (time.perf_counter() - t0) * 1e3 / args.steps
    accs = [dev.download(st["ac"], np.int32, (B,)) for st in sets]
    tokens = float(np.mean([a.sum() + B for a in accs]))     # accepted drafts + the final token, per sequence
    value = tokens / (ms * 1e-3)
    # bytes the stage moves for these inputs: the row statistics read target
    # and draft row 0 of every sequence and the other rows only where draft 0
    # was accepted; the residual pass reads target row n (and draft row n when
    # n < K) and writes the draw weights, which the draw pass reads before it
    # writes the distribution
    def stage_read(acc):
        rows = 0
        for n in acc.tolist():
            rows += 2 + (2 * K - 1 if n >= 1 else 0) + (2 if n < K else 1) + 1
        return rows * V * 4
    read = int(np.mean([stage_read(a) for a in accs]))
    written = 2 * B * V * 4 + B * (K + 2) * 4
    gbs = (read + written) / (ms * 1e-3) / 1e9
    log(f"accept_rejection: {ms * 1e3:.2f} us/step, {gbs:.0f} GB/s, mean accepted {np.mean(accs):.3f}")
    line = {
        "metric": "accepted tokens/s of the rejection-sampling acceptance stage (B=64, K=8, V=49152)",
        "value": round(value, 1), "unit": "accepted tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 logits, u64 fixed-point partition sums, u32 Philox",
        "data": "synthetic: logits N(0,3) from Philox (seeds 2024..2026), drafts sampled from the draft softmax",
        "config": {"workload": "c2: opure_accept_rejection, batch 64, K=8, vocab 49152, temperature 1.0, "
                               "residual distributions written, 3 rotating 226 MB input sets",
                   "mean_accepted": round(float(np.mean(accs)), 4), "wall_ms_per_step": round(wall, 5)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "opure_accept_rejection (one launch of k_rej_fused), whole stage; "
                               "bytes = the rows it reads for these inputs (rows past a sequence's first "
                               "rejected draft are never read) + the distributions written",
                     "bytes_per_launch": read + written, "avg_us": round(ms * 1e3, 2),
                     "measured_peak_GBps": peak["read_GBps"], "frac_of_measured_peak": round(gbs / peak["read_GBps"], 4),
                     "measured_peak": peak},
    }
    if args.cpu_baseline == "auto":
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        st = sets[0]
        t = dev.download(st["t"], np.float32, (B, K + 1, V))
        q = dev.download(st["q"], np.float32, (B, K, V))
        d = dev.download(st["d"], np.int32, (B, K))
        O.set_threads(1)
        t0 = time.perf_counter()
        w_out, w_acc, w_dist = O.accept_rejection(t, q, d, tau, seed, np.zeros(B, np.uint32))
        dt = time.perf_counter() - t0
        got_out = dev.download(st["ot"], np.int32, (B, K + 1))
        got_dist = dev.download(st["di"], np.float32, (B, V))
        w_tokens = float(w_acc.sum() + B)
        line["cpu_baseline"] = {"value": round(w_tokens / dt, 1), "unit": "accepted tokens/s", "cores": 1,
                                "kind": "port", "sample": f"one full acceptance stage (64 sequences) of input set 0 "
                                                          f"through the scalar oracle: {dt:.2f}s"}
        line["parity"] = {"accepted_equal": bool(np.array_equal(w_acc, accs[0])),
                          "tokens_equal": bool(np.array_equal(w_out, got_out)),
                          "dist_max_abs": float(np.abs(got_dist - w_dist).max())}
        log("cpu baseline", line["cpu_baseline"], "parity", line["parity"])
    print(json.dumps(line), flush=True)
    dev.close()


def copy_calibration():
    """Five copies of 64 MiB (16 Mi fp32 read, 16 Mi fp32 written) by
    k_convert_f32 into f32: under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE,
    counter KiB / 65536 is the factor that turns a counter into bytes."""
    dev = H.Dev(0)
    n = 16 << 20
    src, dst = dev.alloc(n * 4), dev.alloc(n * 4)
    L = H.lib()
    H.check(L.opure_synth_normal_f32(dev.h, int(src), n, 1, 0, 1.0, 0.0))
    for _ in range(5):
        H.check(L.opure_convert_f32(dev.h, int(src), int(dst), H.A_F32, n))
    dev.sync()
    print(json.dumps({"copy_calibration": {"bytes_read": n * 4, "bytes_written": n * 4, "launches": 5}}), flush=True)
    dev.close()


def measure_peak(dev, read_gib=2, reps=5):
    """The box's streaming peak, timed with the library's HIP events: `reps`
    read-only passes over read_gib GiB and copies of read_gib/2 GiB (both far
    above the 256 MB last-level cache), 16-byte nontemporal accesses
    (opure_bw_measure).  The roofline fractions are also given against the
    read figure, beside the published 8 TB/s."""
    n = read_gib << 30
    src = dev.alloc(n)
    try:
        dev.fill_u32(src, 0x3C003C00, n // 4)
        read = dev.bw_measure(H.BW_READ, src, None, n, reps)
        half = n // 2
        copy = dev.bw_measure(H.BW_COPY, src, int(src) + half, half, reps)
    finally:
        src.free()
    log(f"measured peak: read {read:.0f} GB/s, copy {copy:.0f} GB/s (read + written)")
    return {"read_GBps": round(read, 1), "copy_GBps": round(copy, 1),
            "method": f"opure_bw_measure: {reps} read-only passes over {read_gib} GiB and {reps} copies of "
                      f"{read_gib / 2:g} GiB, 16-byte nontemporal accesses, 4 x 512-thread workgroups a CU, "
                      "HIP events on the library's stream"}


# Stages of a verify step that run the same kernel instantiation at these
# shapes (the dispatch rules of gemv.hip): a profiler's kernel summary adds
# them into one row, so the roofline reports that row as well.
SHARED_KERNEL = {"c3": {("o_proj", "down"): "k_gemv<1, 1, 1, 16, 1, 1, false, 0> (o_proj and down)"}}


def kernel_rows(config, stages):
    """Per kernel instantiation: algorithmic bytes per step / kernel time per
    step (stages sharing one instantiation combined)."""
    rows = {}
    shared = SHARED_KERNEL.get(config, {})
    seen = set()
    for group, name in shared.items():
        if all(st in stages for st in group):
            by = sum(stages[st]["bytes_per_launch"] * stages[st]["launches_per_step"] for st in group)
            us = sum(stages[st]["us_per_step"] for st in group)
            rows[name] = dict(us_per_step=us, bytes_per_step=by, gbs=by / (us * 1e-6) / 1e9)
            seen.update(group)
    for st, d in stages.items():
        if st in seen or not d.get("gbs"):
            continue
        rows[f"{kernel_of(config, st)} ({st})"] = dict(
            us_per_step=d["us_per_step"], bytes_per_step=d["bytes_per_launch"] * d["launches_per_step"], gbs=d["gbs"])
    return rows


def kernel_of(config, stage):
    """The GEMV kernel a verify-step stage runs at these shapes: loader waves
    for the 8B gate/up (7 tiles a CU), waves owning whole tiles for 1024 tiles
    and more, the K-split kernel below."""
    if stage == "gate_up" and config == "c4":
        return "k_gemv_pc"
    other = {"attention": "k_attn_mfma + k_attn_combine", "embed": "k_embed", "accept": "k_accept_greedy"}
    if stage in other:
        return other[stage]
    return "k_gemv_wpt" if stage in ("gate_up", "lm_head") else "k_gemv"


def traffic_of(config, stage):
    """HBM bytes per launch of a stage's kernel measured by the hardware counters
    (profiles/traffic.json: FETCH_SIZE + WRITE_SIZE of rocprofv3 --pmc runs of
    this benchmark, each scaled by the copy calibration) with the run they came
    from, or None when not measured.  Counters cannot be read inside this
    process, so the figure comes from that separate profiled run."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    doc = json.load(open(path))
    t = doc.get(config, {}).get(stage)
    if not t:
        return None
    return {"bytes": int(t["bytes"]), "source": t.get("source", doc.get("source"))}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c3", choices=sorted(synth.CONFIGS) + ["c2", "c5"])
    ap.add_argument("--cpu-baseline", default="auto", choices=["auto", "skip"])
    ap.add_argument("--no-kernel-timing", action="store_true")
    ap.add_argument("--eager", action="store_true", help="launch each step's kernels directly instead of a hipGraph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run five 64 MiB fp32 copies (k_convert_f32 to f32): the known-size kernel that "
                         "calibrates the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration()
    if args.gpus != 1:
        print(f"bench.py: this benchmark measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    if args.config == "c2":
        return bench_c2(args)
    if args.config == "c1":
        return bench_c1(args)
    if args.config == "c5":
        return bench_c5(args)

    dev = H.Dev(0)
    log("device", dev.name)
    peak = measure_peak(dev)
    w = build_workload(dev, args.config)
    cfg, ctx, R, K = w["cfg"], w["ctx"], w["R"], w["K"]
    res = time_graph(dev, w["step"], w["tokens"], ctx, args.warmup, args.steps, args.eager)
    gpu_logits = w["step"].logits_host()
    log(f"self-drafts: {res['ms_per_step'] * 1e3:.1f} us/step, accepted {res['accepted']}/{K}")
    rnd = w["tokens"].copy()
    rnd[0, 1:] = w["rng"].integers(0, cfg["vocab"], K)
    res_r = time_graph(dev, w["step"], rnd, ctx, args.warmup, args.steps, args.eager)
    log(f"random drafts: {res_r['ms_per_step'] * 1e3:.1f} us/step, accepted {res_r['accepted']}/{K}")
    # restore the self-draft step's logits for the parity check (same cache state)
    step_bytes = synth.verify_bytes(cfg, R, ctx)
    step_gbs = step_bytes["total"] / (res["ms_per_step"] * 1e-3) / 1e9
    stages = None if args.no_kernel_timing else time_stages(dev, w["step"], w["tokens"], ctx, 10)
    kern = None
    if stages:
        for st, d in stages.items():
            log(f"stage {st:10s} x{d['launches_per_step']:4.0f}/step  {d['avg_us']:8.2f} us/launch  "
                f"{d['us_per_step']:8.1f} us/step" + (f"  {d['gbs']:6.0f} GB/s" if d["gbs"] else ""))
        # the dominant single-kernel stage (attention is two kernels: chunks + combine)
        gemv_stages = [st for st in ("qkv", "o_proj", "gate_up", "down", "lm_head") if st in stages]
        dom = max(gemv_stages, key=lambda st: stages[st]["us_per_step"])
        kern = dict(stages[dom], stage=dom)
    cpu, parity = None, None
    if args.cpu_baseline == "auto":
        cpu, parity = cpu_baseline(dev, w, gpu_logits, res)
        log("cpu baseline", cpu, "parity", parity)
    value = (res["accepted"] + 1) / (res["ms_per_step"] * 1e-3)
    names = {"c1": "SmolLM-135M-shape fp32", "c3": "Llama-3.2-1B-shape int8-pc/fp16",
             "c4": "Llama-3-8B-shape int4-g128/bf16"}
    line = {
        "metric": "accepted tokens/s @1 GPU (1B int8, K=5); verify-step ms; % HBM peak",
        "value": round(value, 1),
        "unit": "accepted tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": {"c1": "f32", "c3": "int8 weights, f16 activations, f32 accumulate",
                  "c4": "uint4 weights, bf16 activations, f32 accumulate"}[args.config],
        "data": "synthetic: seeded N(0,0.02) weights quantised on device; context prefilled from random ids",
        "config": {"workload": f"{args.config}: verify step, {names[args.config]}, {cfg['n_layers']} layers, "
                               f"batch 1, K={K} ({R} rows), {ctx}-token paged context (16-token pages), greedy "
                               "acceptance + rollback, " + ("eager launches" if args.eager else "hipGraph replay"),
                   "drafts": f"target's greedy continuation ({res['accepted']}/{K} accepted)",
                   "accepted_tokens_per_s_random_drafts": round((res_r["accepted"] + 1) /
                                                                (res_r["ms_per_step"] * 1e-3), 1),
                   "random_drafts_accepted": res_r["accepted"],
                   "step_bytes": step_bytes["total"], "step_GBps": round(step_gbs, 1),
                   "step_frac_of_hbm_peak": round(step_gbs / HBM_PEAK_GBS, 4),
                   "step_frac_of_measured_peak": round(step_gbs / peak["read_GBps"], 4),
                   "wall_ms_per_step": round(res["wall_ms_per_step"], 4)},
    }
    if kern:
        tr = traffic_of(args.config, kern["stage"])
        line["roofline"] = {"bound": "hbm", "achieved": round(kern["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(kern["gbs"] / HBM_PEAK_GBS, 4),
                            "traffic": tr["bytes"] if tr else None,
                            "kernel": f"{kernel_of(args.config, kern['stage'])} ({kern['stage']} stage of the verify step)",
                            "bytes_per_launch": kern["bytes_per_launch"], "avg_us": round(kern["avg_us"], 2),
                            "timing": "kernel execution time from start/stop events stamped by each dispatch "
                                      "(hipExtLaunchKernelGGL) over 10 eager steps, averaged per launch",
                            "traffic_source": tr["source"] if tr else None,
                            "measured_peak_GBps": peak["read_GBps"],
                            "frac_of_measured_peak": round(kern["gbs"] / peak["read_GBps"], 4),
                            "measured_peak": peak}
        krows = kernel_rows(args.config, stages)
        top = max(krows, key=lambda k: krows[k]["us_per_step"])
        line["roofline"]["kernels"] = {
            k: {"us_per_step": round(d["us_per_step"], 1), "GBps": round(d["gbs"], 1),
                "frac": round(d["gbs"] / HBM_PEAK_GBS, 4), "frac_of_measured_peak": round(d["gbs"] / peak["read_GBps"], 4)}
            for k, d in sorted(krows.items(), key=lambda kv: -kv[1]["us_per_step"])}
        line["roofline"]["top_kernel"] = top
        line["stages"] = {st: {"launches_per_step": round(d["launches_per_step"], 2), "us": round(d["avg_us"], 2),
                               "us_per_step": round(d["us_per_step"], 1),
                               "GBps": round(d["gbs"], 1) if d["gbs"] else None,
                               "frac": round(d["gbs"] / HBM_PEAK_GBS, 4) if d["gbs"] else None}
                          for st, d in stages.items()}
    if cpu:
        line["cpu_baseline"] = rounded(cpu)
        line["parity"] = parity
    print(json.dumps(line), flush=True)
    dev.close()


def rounded(d):
    """Floats of a (nested) result dict to 4 decimals."""
    return {k: rounded(v) if isinstance(v, dict) else round(v, 4) if isinstance(v, float) else v for k, v in d.items()}


if __name__ == "__main__":
    main()
