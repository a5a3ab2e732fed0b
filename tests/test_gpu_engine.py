"""The native C++20 engine (include/opure_engine.h) on the GPU at the
SmolLM-135M shape: 30-layer fp32 target, 2-layer draft of the same width,
32-token prompt, K=4, 64 new tokens (the greedy speculative-generation
workload).  Checks:
  - speculative output == greedy output of the same engine, bit for bit
    (the defining invariant of greedy speculative decoding);
  - a draft identical to the target accepts all K drafts at every step;
  - hipGraph replay == eager launches;
  - the 64 emitted ids and every verify step's accepted count equal the CPU
    oracle's run of the same speculative loop on the same weights, for the
    2-layer draft (which is rarely accepted) and for a draft that is accepted
    part of the time (the target's first 29 layers).
"""
import numpy as np
import pytest

import opure_engine as E
import opure_hip as H
import oracle as O
import spec_loop
import synth
from gpu_util import say

pytestmark = pytest.mark.gpu

N_NEW, K, PROMPT = 64, 4, 32


@pytest.fixture(scope="module")
def models():
    dev = H.Dev(0)
    cfg = synth.CONFIGS["c1"]
    max_pos = 256                         # cache and RoPE capacity: prompt + 112 new + K + 1, rounded up
    say("building c1 target (30 layers) and draft (2 layers) on the device")
    tgt = synth.SynthModel(dev, cfg, seed=1234, max_pos=max_pos)
    drf = synth.SynthModel(dev, dict(cfg, n_layers=2), seed=4321, max_pos=max_pos)
    prompt = np.random.default_rng(7).integers(0, cfg["vocab"], PROMPT).astype(np.int32)
    yield dev, tgt, drf, prompt, max_pos
    dev.close()


def test_speculative_equals_greedy_c1(models):
    dev, tgt, drf, prompt, max_pos = models
    eng = E.Engine(dev, tgt.desc, drf.desc, max_positions=max_pos, draft_tokens=K)
    greedy, gst = eng.generate(prompt, N_NEW)
    spec, hist, sst = eng.generate_speculative(prompt, N_NEW)
    say("greedy", greedy[:12].tolist(), "accepted per step", hist.tolist())
    say(f"greedy {gst.ms_generate:.2f} ms, speculative {sst.ms_generate:.2f} ms "
        f"({sst.verify_steps} verify + {sst.draft_steps} draft steps)")
    assert np.array_equal(spec, greedy)
    assert sst.emitted == N_NEW and gst.emitted == N_NEW
    assert int(hist.sum()) == sst.accepted_total
    m = eng.metrics()
    assert (m.generate_calls, m.tokens_emitted) == (2, 2 * N_NEW)
    assert (m.verify_steps, m.drafts_accepted) == (sst.verify_steps, sst.accepted_total)
    assert m.drafts_proposed == K * sst.verify_steps
    assert m.speculative_acceptance == sst.accepted_total / (K * sst.verify_steps)
    eng.close()


def test_identical_draft_accepts_everything(models):
    dev, tgt, _, prompt, max_pos = models
    eng = E.Engine(dev, tgt.desc, tgt.desc, max_positions=max_pos, draft_tokens=K)
    greedy, _ = eng.generate(prompt, N_NEW)
    assert eng.metrics().speculative_acceptance == -1.0     # no speculative step yet
    spec, hist, st = eng.generate_speculative(prompt, N_NEW)
    assert np.array_equal(spec, greedy)
    assert (hist == K).all(), hist.tolist()
    assert st.verify_steps == -(-N_NEW // (K + 1))
    assert eng.metrics().speculative_acceptance == 1.0
    eng.reset_metrics()
    m = eng.metrics()
    assert (m.generate_calls, m.verify_steps, m.speculative_acceptance) == (0, 0, -1.0)
    eng.close()


def test_graph_replay_equals_eager(models):
    dev, tgt, drf, prompt, max_pos = models
    a = E.Engine(dev, tgt.desc, drf.desc, max_positions=max_pos, draft_tokens=K, use_graphs=True)
    b = E.Engine(dev, tgt.desc, drf.desc, max_positions=max_pos, draft_tokens=K, use_graphs=False)
    sa, ha, _ = a.generate_speculative(prompt, 24)
    sb, hb, _ = b.generate_speculative(prompt, 24)
    assert np.array_equal(sa, sb) and np.array_equal(ha, hb)
    a.close()
    b.close()


def oracle_speculative(tgt_cfg, tgt_w, drf_cfg, drf_w, prompt, n_new, max_pos):
    """The same greedy speculative loop run on the CPU oracle (both models)."""
    models = {"t": O.HostModel.from_arrays(tgt_cfg, tgt_w), "d": O.HostModel.from_arrays(drf_cfg, drf_w)}
    mp = (max_pos + 15) // 16
    kvs = {k: O.HostKV(m, n_pages=mp, batch=1, max_pages_per_seq=mp) for k, m in models.items()}
    for kv in kvs.values():
        kv.page_table[0] = np.arange(mp)

    def step(key, toks, ctx):
        return O.verify_forward(models[key], kvs[key], toks, np.array([ctx], np.int32))

    def accept(toks, ctx):
        o, a = O.accept_greedy(step("t", toks, ctx), toks[:, 1:])
        return o[0], int(a[0])

    O.set_threads(16)
    try:
        return spec_loop.speculative(step, accept, list(prompt), n_new, K)
    finally:
        O.set_threads(1)


def test_speculative_matches_oracle_c1(models):
    """The whole C1 workload: 64 emitted ids and the accepted count of every
    verify step equal the oracle's run of the same loop, bit for bit."""
    dev, tgt, drf, prompt, max_pos = models
    eng = E.Engine(dev, tgt.desc, drf.desc, max_positions=max_pos, draft_tokens=K)
    spec, hist, _ = eng.generate_speculative(prompt, N_NEW)
    eng.close()
    want, want_hist = oracle_speculative(tgt.cfg, tgt.download(), drf.cfg, drf.download(), prompt, N_NEW, max_pos)
    say("oracle accepted per step", want_hist)
    assert spec.tolist() == want
    assert hist.tolist() == want_hist


def test_partial_acceptance_matches_oracle_c1(models):
    """A draft that accepts some drafts: the target's first 29 layers (same
    embedding, final norm and LM head).  Ids and per-step accepted counts equal
    the oracle's, and drafts are accepted at some steps and rejected at others."""
    import ctypes as C
    dev, tgt, _, prompt, max_pos = models
    d = H.Model()
    C.memmove(C.byref(d), C.byref(tgt.desc), C.sizeof(H.Model))
    d.n_layers = 29
    n_new = 112
    eng = E.Engine(dev, tgt.desc, d, max_positions=max_pos, draft_tokens=K)
    spec, hist, st = eng.generate_speculative(prompt, n_new)
    # every page of the target's pool is held by the sequence or free, once:
    # the sequence holds exactly the pages of its kept positions, the rollbacks
    # of ~30 steps having returned the rest
    total, avail, row = eng.pages()
    held = row[row >= 0]
    kept = len(prompt) + st.verify_steps + st.accepted_total
    assert len(set(held.tolist())) == len(held) == -(-kept // 16)
    assert avail == total - len(held)
    dt, da, drow = eng.pages(draft=True)
    dheld = drow[drow >= 0]
    assert len(set(dheld.tolist())) == len(dheld) and da == dt - len(dheld)
    eng.close()
    w = tgt.download()
    want, want_hist = oracle_speculative(tgt.cfg, w, dict(tgt.cfg, n_layers=29), dict(w, layers=w["layers"][:29]),
                                         prompt, n_new, max_pos)
    say("29-layer draft accepted per step", hist.tolist(), "oracle", want_hist)
    assert spec.tolist() == want
    assert hist.tolist() == want_hist
    assert len(want_hist) >= 30
    assert 0 < sum(want_hist) < K * len(want_hist)


def test_verify_step_and_rollback_kv_c1(models):
    """The engine's VerifyStep and RollbackKV on their own: rows scored against
    the target's greedy continuation (a K+1-row step equals K+1 decode steps),
    a rejected draft, and the rollback giving the page past the kept length
    back to the pool."""
    dev, tgt, _, prompt, max_pos = models
    eng = E.Engine(dev, tgt.desc, None, max_positions=max_pos, draft_tokens=K)
    p, ctx = prompt[:30], 30
    g, _ = eng.generate(p, K + 2)                 # g[0] after the prompt, g[1..] its continuation
    g = g.tolist()
    bad = [g[0], (g[1] + 1) % 49152] + g[2:K + 1]
    acc, emitted = eng.verify_step(bad, ctx)
    assert (acc, emitted) == (0, [g[1]])
    assert eng.rollback_kv(ctx, acc, K) == ctx + 1
    total, avail, row = eng.pages()
    held = row[row >= 0]
    assert len(held) == 2 and avail == total - 2          # positions 0..30: pages 0 and 1; page 2 went back
    acc, emitted = eng.verify_step(g[:K + 1], ctx)
    assert (acc, emitted) == (K, g[1:K + 2])
    assert eng.rollback_kv(ctx, acc, K) == ctx + K + 1
    total, avail, row = eng.pages()
    assert (row >= 0).sum() == 3 and avail == total - 3
    m = eng.metrics()
    assert (m.verify_steps, m.drafts_proposed, m.drafts_accepted) == (2, 2 * K, K)
    eng.close()


def test_prefill_256_rows_engine():
    """A quantised model's 300-token prompt is prefilled 256 rows a launch
    (16 parts x 16 rows on one page-table row), then 32, then 11 in a 16-row
    step: the greedy continuation equals the oracle's (every decision's top-2
    gap is well above the logit bar)."""
    from test_gpu_verify import small_model
    from gpu_util import device_model
    m = small_model(O.W_I8PC, O.A_F16, max_pos=512)
    prompt = list(np.random.default_rng(0).integers(0, m.cfg["vocab"], 300))
    dev = H.Dev(0)
    try:
        dm = device_model(dev, m)
        eng = E.Engine(dev, dm.desc, None, max_positions=400, draft_tokens=K)
        got, _ = eng.generate(prompt, 4)
        eng.close()
    finally:
        dev.close()
    kv = O.HostKV(m, n_pages=32, batch=1, max_pages_per_seq=32)
    kv.page_table[0] = np.arange(32)

    def step(_key, toks, ctx):
        return O.verify_forward(m, kv, toks, np.array([ctx], np.int32))

    want, gaps = spec_loop.greedy(step, prompt, 4)
    assert min(gaps) > 4e-2
    assert got.tolist() == want
