"""Pins the oracle's acceptance rules and KV rollback.

Greedy: longest matching prefix, correction = argmax of the first mismatching
row, bonus = argmax of row K.  Rejection sampling (Leviathan et al. 2023,
Chen et al. 2023): q = p always accepts; p(x) = 0 always rejects; the residual
is normalised and zero wherever q >= p; and the emitted token is distributed
exactly as p (chi-square on small vocabularies).  Rollback: the invariant that
a rolled-back cache behaves exactly like one that only ever held n tokens.
"""
import numpy as np
import pytest
from scipy import stats

import oracle as O
from test_oracle_forward import tiny


def test_greedy_accept_rules():
    V, K = 10, 4
    t = np.full((1, K + 1, V), -1.0, dtype=np.float32)
    am = [3, 5, 7, 1, 9]
    for j, a in enumerate(am):
        t[0, j, a] = 2.0
    out, acc = O.accept_greedy(t, np.array([[3, 5, 7, 1]]))
    assert acc[0] == 4 and list(out[0]) == [3, 5, 7, 1, 9]
    out, acc = O.accept_greedy(t, np.array([[3, 5, 2, 1]]))
    assert acc[0] == 2 and list(out[0]) == [3, 5, 7, -1, -1]
    out, acc = O.accept_greedy(t, np.array([[0, 5, 7, 1]]))
    assert acc[0] == 0 and list(out[0]) == [3, -1, -1, -1, -1]
    t[0, 0, 8] = 2.0     # tie with index 3: lowest index wins
    out, acc = O.accept_greedy(t, np.array([[3, 5, 7, 1]]))
    assert acc[0] == 4


def _softmax(x, tau=1.0):
    z = x.astype(np.float64) / tau
    e = np.exp(z - z.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def test_rejection_q_equals_p_always_accepts():
    rng = np.random.default_rng(1)
    B, K, V = 16, 6, 300
    q = (rng.standard_normal((B, K, V)) * 3).astype(np.float32)
    t = np.concatenate([q, (rng.standard_normal((B, 1, V)) * 3).astype(np.float32)], axis=1)
    drafts = rng.integers(0, V, size=(B, K)).astype(np.int32)
    out, acc, dist = O.accept_rejection(t, q, drafts, 1.0, seed=77)
    assert np.all(acc == K)
    np.testing.assert_allclose(dist, _softmax(t[:, K]), rtol=2e-5, atol=1e-7)


def test_rejection_zero_target_prob_always_rejects():
    rng = np.random.default_rng(2)
    B, K, V = 32, 3, 64
    t = (rng.standard_normal((B, K + 1, V))).astype(np.float32)
    q = (rng.standard_normal((B, K, V))).astype(np.float32)
    drafts = rng.integers(0, V, size=(B, K)).astype(np.int32)
    for b in range(B):
        t[b, 0, drafts[b, 0]] = -1e30           # p(x_0) underflows to exactly 0
    out, acc, dist = O.accept_rejection(t, q, drafts, 1.0, seed=5)
    assert np.all(acc == 0)
    for b in range(B):
        assert dist[b, drafts[b, 0]] == 0.0
        assert out[b, 0] != drafts[b, 0]


def test_residual_normalised_and_zero_where_q_ge_p():
    rng = np.random.default_rng(3)
    B, K, V = 64, 8, 49152 // 16
    t = (rng.standard_normal((B, K + 1, V)) * 3).astype(np.float32)
    q = (rng.standard_normal((B, K, V)) * 3).astype(np.float32)
    drafts = rng.integers(0, V, size=(B, K)).astype(np.int32)
    out, acc, dist = O.accept_rejection(t, q, drafts, 1.0, seed=9)
    assert (acc < K).sum() >= B // 2
    for b in range(B):
        n = acc[b]
        if n == K:      # full accept: the bonus is drawn from p_K itself
            np.testing.assert_allclose(dist[b], _softmax(t[b, K]), rtol=0, atol=1e-6)
            continue
        p, qq = _softmax(t[b, n]), _softmax(q[b, n])
        want = np.maximum(p - qq, 0)
        want /= want.sum()
        np.testing.assert_allclose(dist[b], want, rtol=0, atol=1e-6)
        assert np.all(dist[b][qq >= p * (1 + 1e-5)] == 0)
        assert abs(dist[b].astype(np.float64).sum() - 1) < 1e-4
        assert dist[b, out[b, n]] > 0


def test_rejection_is_deterministic_and_keyed():
    rng = np.random.default_rng(4)
    B, K, V = 8, 4, 200
    t = (rng.standard_normal((B, K + 1, V))).astype(np.float32)
    q = (rng.standard_normal((B, K, V))).astype(np.float32)
    d = rng.integers(0, V, size=(B, K)).astype(np.int32)
    a = O.accept_rejection(t, q, d, 1.0, seed=11)
    b = O.accept_rejection(t, q, d, 1.0, seed=11)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    c = O.accept_rejection(t, q, d, 1.0, seed=12)
    e = O.accept_rejection(t, q, d, 1.0, seed=11, pos_base=np.full(B, 1000))
    assert not np.array_equal(a[0], c[0]) or not np.array_equal(a[0], e[0])


def test_emitted_token_follows_target_distribution():
    """The first emitted token of speculative sampling is distributed as p_0,
    whatever q is (Leviathan et al. 2023, Theorem 3.5).  Chi-square over many
    independent seeds."""
    rng = np.random.default_rng(6)
    V, K, N = 6, 1, 20000
    tl = rng.standard_normal(V).astype(np.float32) * 1.5
    ql = rng.standard_normal(V).astype(np.float32) * 1.5
    p, qq = _softmax(tl), _softmax(ql)
    t = np.broadcast_to(np.stack([tl, tl])[None], (N, K + 1, V)).copy()
    q = np.broadcast_to(ql[None, None], (N, K, V)).copy()
    # drafts sampled from q on Philox stream 0, as the draft model would
    drafts = O.sample_rows(q.reshape(N, V), 1.0, 123, np.zeros(N), np.arange(N), 0).reshape(N, K)
    dh = np.bincount(drafts[:, 0], minlength=V)
    assert stats.chisquare(dh, qq * N).pvalue > 1e-3
    out, acc, _ = O.accept_rejection(t, q, drafts, 1.0, seed=321)
    first = out[:, 0]
    hist = np.bincount(first, minlength=V)
    assert stats.chisquare(hist, p * N).pvalue > 1e-3
    assert 0 < acc.mean() < 1


def test_sample_rows_matches_softmax_at_temperature():
    rng = np.random.default_rng(7)
    V, N, tau = 5, 20000, 0.8
    lg = rng.standard_normal(V).astype(np.float32)
    toks = O.sample_rows(np.broadcast_to(lg, (N, V)).copy(), tau, 99, np.arange(N), np.zeros(N), 0)
    assert stats.chisquare(np.bincount(toks, minlength=V), _softmax(lg, tau) * N).pvalue > 1e-3


def test_low_temperature_limit_is_greedy():
    rng = np.random.default_rng(8)
    B, K, V = 16, 4, 100
    t = (rng.standard_normal((B, K + 1, V)) * 3).astype(np.float32)
    am = t.argmax(-1)
    drafts = am[:, :K].astype(np.int32).copy()
    drafts[::2, 2] = (drafts[::2, 2] + 1) % V
    q = np.full((B, K, V), -50.0, dtype=np.float32)
    q[np.arange(B)[:, None], np.arange(K)[None, :], drafts] = 50.0
    g_out, g_acc = O.accept_greedy(t, drafts)
    r_out, r_acc, _ = O.accept_rejection(t, q, drafts, 1e-3, seed=1)
    assert np.array_equal(g_acc, r_acc) and np.array_equal(g_out, r_out)


def test_rollback_bookkeeping_and_poison():
    m = tiny(O.W_F32, O.A_F32)
    kv = O.HostKV(m, n_pages=8, batch=2, max_pages_per_seq=4)
    kv.page_table[0, :3] = [5, 1, 2]
    kv.page_table[1, :2] = [0, 3]
    seq_len = np.array([14, 9], dtype=np.int32)     # verify wrote 14..19 and 9..14 (K=5)
    acc = np.array([1, 5], dtype=np.int32)
    nan = int(np.float32(np.nan).view(np.uint32))
    new_len, freed, nf = O.kv_rollback(kv, m, 5, seq_len, acc, poison_bits=nan)
    assert list(new_len) == [16, 15]
    # seq 0: positions 16..19 rolled back, page 1 (positions 16..31) released
    assert nf[0] == 1 and freed[0, 0] == 1 and kv.page_table[0, 1] == -1
    Kp, Vp = O.kv_planes(kv.pool)
    assert np.isnan(Kp[:, 1, :, 0:4]).all() and np.isnan(Vp[:, 1, :, 0:4]).all()
    assert not np.isnan(Kp[:, 1, :, 4:]).any() and not np.isnan(Vp[:, 1, :, 4:]).any()
    assert not np.isnan(kv.pool[:, 5]).any()
    assert nf[1] == 0 and kv.page_table[1, 0] == 0


def test_rollback_equals_never_written():
    """After a verify step and a rollback to n accepted tokens, the next step's
    logits equal those of a cache that only ever held the accepted prefix."""
    m = tiny(O.W_I8PC, O.A_F16)
    K = 4
    prompt = np.array([[7, 8, 9, 10, 11, 12, 13]], dtype=np.int32)

    def fresh():
        kv = O.HostKV(m, n_pages=4, batch=1, max_pages_per_seq=4)
        kv.page_table[0, :] = [2, 0, 3, 1]
        O.verify_forward(m, kv, prompt, np.array([0], dtype=np.int32))
        return kv

    kv = fresh()
    ctx = prompt.shape[1]
    drafts = np.array([[100, 200, 300, 400]], dtype=np.int32)
    lg = O.verify_forward(m, kv, np.concatenate([[[42]], drafts], axis=1), np.array([ctx], dtype=np.int32))
    acc = np.array([1], dtype=np.int32)
    nan = int(np.uint16(0x7E00))
    new_len, _, _ = O.kv_rollback(kv, m, K, np.array([ctx]), acc, poison_bits=nan)
    kv.page_table[0, :] = [2, 0, 3, 1]          # re-grant released pages, as the allocator would
    nxt = np.array([[int(lg[0, 1].argmax()), 5, 6]], dtype=np.int32)
    a = O.verify_forward(m, kv, nxt, new_len)

    kv2 = fresh()
    O.verify_forward(m, kv2, np.array([[42, 100]], dtype=np.int32), np.array([ctx], dtype=np.int32))
    b = O.verify_forward(m, kv2, nxt, np.array([ctx + 2], dtype=np.int32))
    assert np.array_equal(a, b)
