"""Pins orc_verify_forward: an independent numpy forward, row independence,
page-placement invariance, and the greedy speculative-decoding invariant."""
import numpy as np
import pytest

import npref
import oracle as O

CASES = [
    dict(wfmt=O.W_F32, afmt=O.A_F32, tol=2e-5),
    dict(wfmt=O.W_I8PC, afmt=O.A_F16, tol=2e-2),
    dict(wfmt=O.W_I4G128, afmt=O.A_BF16, tol=2e-2),
]


def tiny(wfmt, afmt, seed=21, tied=True, n_layers=2):
    return O.HostModel(n_layers=n_layers, hidden=128, n_heads=4, n_kv_heads=2, head_dim=32, ffn=256,
                       vocab=512, wfmt=wfmt, afmt=afmt, attn_scale=0.17, theta=10000.0, max_pos=256,
                       tied=tied, seed=seed, norm_jitter=0.1)


def make_kv(model, B=2, ctx=(37, 20), pages=24, seed=3):
    kv = O.HostKV(model, n_pages=pages, batch=B, max_pages_per_seq=8)
    rng = np.random.default_rng(seed)
    kv.fill_random(rng, 0.5)
    perm = rng.permutation(pages)
    for b in range(B):
        kv.page_table[b, :6] = perm[b * 6:(b + 1) * 6]
    return kv, np.array(ctx[:B], dtype=np.int32)


@pytest.mark.parametrize("case", CASES, ids=["f32", "i8pc-f16", "i4g128-bf16"])
def test_forward_matches_numpy_restatement(case):
    m = tiny(case["wfmt"], case["afmt"], tied=case["wfmt"] != O.W_I4G128)
    kv, seq_len = make_kv(m)
    tokens = np.random.default_rng(4).integers(0, 512, size=(2, 5)).astype(np.int32)
    pool_np = kv.pool.copy()
    got = O.verify_forward(m, kv, tokens, seq_len)
    want = npref.forward(m, pool_np, kv.page_table, tokens, seq_len)
    err = np.abs(got - want).max()
    assert err <= case["tol"], err
    # the K/V appended by the two sides agree (same rounding points)
    if case["afmt"] == O.A_F32:
        np.testing.assert_allclose(kv.pool, pool_np, rtol=0, atol=1e-5)
    else:
        a = npref.act_to_f32(kv.pool, case["afmt"])
        b = npref.act_to_f32(pool_np, case["afmt"])
        assert np.abs(a - b).max() <= 2e-2


@pytest.mark.parametrize("case", CASES, ids=["f32", "i8pc-f16", "i4g128-bf16"])
def test_rows_equal_sequential_decode(case):
    """Row j of a K+1-row verify equals a one-row decode at position ctx+j."""
    m = tiny(case["wfmt"], case["afmt"])
    kv, seq_len = make_kv(m, B=1)
    pool0 = kv.pool.copy()
    tokens = np.array([[5, 77, 301, 9, 460]], dtype=np.int32)
    multi = O.verify_forward(m, kv, tokens, seq_len)
    kv.pool[...] = pool0
    for j in range(tokens.shape[1]):
        one = O.verify_forward(m, kv, tokens[:, j:j + 1], seq_len + j)
        assert np.array_equal(one[0, 0], multi[0, j])


def test_threads_give_the_same_bits():
    """The oracle's GEMVs (over output rows) and attention (over row, head
    pairs) split over threads compute every output as one thread does."""
    m = tiny(O.W_I4G128, O.A_BF16)
    kv, seq_len = make_kv(m)
    pool0 = kv.pool.copy()
    tokens = np.random.default_rng(6).integers(0, 512, size=(2, 4)).astype(np.int32)
    try:
        O.set_threads(1)
        one = O.verify_forward(m, kv, tokens, seq_len)
        kv.pool[...] = pool0
        O.set_threads(4)
        four = O.verify_forward(m, kv, tokens, seq_len)
    finally:
        O.set_threads(1)
    assert np.array_equal(one, four)


def test_page_placement_invariance():
    m = tiny(O.W_I8PC, O.A_F16)
    kv, seq_len = make_kv(m, B=1)
    tokens = np.array([[1, 2, 3]], dtype=np.int32)
    kv2 = O.HostKV(m, n_pages=kv.n_pages, batch=1, max_pages_per_seq=8)
    perm = np.random.default_rng(8).permutation(kv.n_pages)
    for p in range(6):
        src = kv.page_table[0, p]
        kv2.pool[:, perm[p]] = kv.pool[:, src]
        kv2.page_table[0, p] = perm[p]
    a = O.verify_forward(m, kv, tokens, seq_len)
    b = O.verify_forward(m, kv2, tokens, seq_len)
    assert np.array_equal(a, b)


def test_bad_arguments_rejected():
    m = tiny(O.W_F32, O.A_F32)
    kv, seq_len = make_kv(m, B=1)
    with pytest.raises(ValueError):
        O.verify_forward(m, kv, np.array([[600]], dtype=np.int32), seq_len)   # id >= vocab
    kv.page_table[0, 3] = -1
    with pytest.raises(ValueError):
        O.verify_forward(m, kv, np.array([[1, 2]], dtype=np.int32), np.array([47], dtype=np.int32))


def greedy_generate(m, prompt, n_new, spec_k=0, draft=None):
    """Plain greedy (spec_k=0) or greedy speculative decoding driven by the oracle."""
    ps, maxp = 16, 16
    kv = O.HostKV(m, n_pages=maxp, batch=1, max_pages_per_seq=maxp)
    kv.page_table[0, :] = np.arange(maxp)
    dkv = None
    if draft is not None:
        dkv = O.HostKV(draft, n_pages=maxp, batch=1, max_pages_per_seq=maxp)
        dkv.page_table[0, :] = np.arange(maxp)
    lg = O.verify_forward(m, kv, np.array([prompt], dtype=np.int32), np.array([0], dtype=np.int32))
    nxt = int(np.argmax(lg[0, -1]))
    ctx = len(prompt)
    out = []
    accepted_hist = []
    if draft is not None:
        O.verify_forward(draft, dkv, np.array([prompt], dtype=np.int32), np.array([0], dtype=np.int32))
    dctx = len(prompt)
    pending = [nxt]          # tokens the draft model has not consumed yet
    while len(out) < n_new:
        if spec_k == 0:
            out.append(nxt)
            lg = O.verify_forward(m, kv, np.array([[nxt]], dtype=np.int32), np.array([ctx], dtype=np.int32))
            ctx += 1
            nxt = int(np.argmax(lg[0, 0]))
            continue
        drafts = []
        dl = O.verify_forward(draft, dkv, np.array([pending], dtype=np.int32), np.array([dctx], dtype=np.int32))
        dctx += len(pending)
        d = int(np.argmax(dl[0, -1]))
        drafts.append(d)
        for _ in range(spec_k - 1):
            dl = O.verify_forward(draft, dkv, np.array([[d]], dtype=np.int32), np.array([dctx], dtype=np.int32))
            dctx += 1
            d = int(np.argmax(dl[0, 0]))
            drafts.append(d)
        lg = O.verify_forward(m, kv, np.array([[nxt] + drafts], dtype=np.int32), np.array([ctx], dtype=np.int32))
        toks, acc = O.accept_greedy(lg, np.array([drafts], dtype=np.int32))
        n = int(acc[0])
        accepted_hist.append(n)
        emitted = [nxt] + [int(t) for t in toks[0, :n]]
        out.extend(emitted)
        ctx += n + 1
        nxt = int(toks[0, n])
        # draft cache: keep what matches the accepted prefix, re-feed the rest
        dctx = min(dctx, ctx - 1 + 0)
        consumed_ok = ctx - 1        # positions < ctx-1 hold tokens the draft saw and that were accepted
        dctx = min(dctx, consumed_ok)
        pending = ([drafts[n - 1]] if n == spec_k else []) + [nxt]
        if n < spec_k:
            dctx = ctx
            pending = [nxt]
    return out[:n_new], accepted_hist


def test_speculative_greedy_equals_greedy():
    m = tiny(O.W_F32, O.A_F32, n_layers=2)
    d = tiny(O.W_F32, O.A_F32, seed=99, n_layers=1)
    prompt = [3, 14, 15, 92, 65, 35, 89, 79]
    ref, _ = greedy_generate(m, prompt, 20)
    spec, hist = greedy_generate(m, prompt, 20, spec_k=4, draft=d)
    assert spec == ref
    self_spec, hist2 = greedy_generate(m, prompt, 20, spec_k=4, draft=m)
    assert self_spec == ref
    assert all(h == 4 for h in hist2)          # draft == target: every draft accepted
