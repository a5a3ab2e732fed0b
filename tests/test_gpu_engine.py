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
    max_pos = PROMPT + N_NEW + 2 * K + 16
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
    n_new = 24
    eng = E.Engine(dev, tgt.desc, d, max_positions=max_pos, draft_tokens=K)
    spec, hist, _ = eng.generate_speculative(prompt, n_new)
    eng.close()
    w = tgt.download()
    want, want_hist = oracle_speculative(tgt.cfg, w, dict(tgt.cfg, n_layers=29), dict(w, layers=w["layers"][:29]),
                                         prompt, n_new, max_pos)
    say("29-layer draft accepted per step", hist.tolist(), "oracle", want_hist)
    assert spec.tolist() == want
    assert hist.tolist() == want_hist
    assert 0 < sum(want_hist) < K * len(want_hist)
