"""The native C++20 engine (include/opure_engine.h) on the GPU at the
SmolLM-135M shape: 30-layer fp32 target, 2-layer draft of the same width,
32-token prompt, K=4, 64 new tokens (the greedy speculative-generation
workload).  Checks:
  - speculative output == greedy output of the same engine, bit for bit
    (the defining invariant of greedy speculative decoding);
  - a draft identical to the target accepts all K drafts at every step;
  - hipGraph replay == eager launches;
  - the first greedy ids equal the CPU oracle's greedy decoding of the same
    weights (the oracle runs a few tokens of the 30-layer model).
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


def test_greedy_matches_oracle_c1(models):
    dev, tgt, _, prompt, max_pos = models
    eng = E.Engine(dev, tgt.desc, None, max_positions=max_pos, draft_tokens=K)
    greedy, _ = eng.generate(prompt, 3)
    eng.close()
    hm = O.HostModel.from_arrays(tgt.cfg, tgt.download())
    kv = O.HostKV(hm, n_pages=(max_pos + 15) // 16, batch=1, max_pages_per_seq=(max_pos + 15) // 16)
    kv.page_table[0] = np.arange(kv.max_pages)
    O.set_threads(8)

    def step(_key, toks, ctx):
        return O.verify_forward(hm, kv, toks, np.array([ctx], np.int32))

    want, gaps = spec_loop.greedy(step, list(prompt), 3)
    say("oracle greedy", want, "min top-2 gap", float(np.min(gaps)) if gaps else None)
    assert greedy.tolist() == want
