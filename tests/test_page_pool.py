"""CPU checks of the page pool (include/opure_engine.h, opure_page_pool_*):
the free list that sequences take 16-token KV pages from as they grow and
that opure_kv_rollback's freed lists return pages to.  Host bookkeeping only,
so everything here runs without a GPU; the rollback in the loop test is the
oracle's restatement of opure_kv_rollback (the GPU test of that entry point
checks the device rollback against the same oracle bit for bit)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import opure_engine as E
import opure_hip as H
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def engine_symbols():
    text = open(os.path.join(ROOT, "include", "opure_engine.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(opure_[a-z0-9_]+)\s*\(", text)))


def test_engine_library_exports_every_declared_symbol():
    L = E.lib()
    names = engine_symbols()
    assert "opure_page_pool_grow_seq" in names and "opure_engine_get_metrics" in names
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    for n in names:
        assert getattr(L, n).argtypes is not None, n


def test_metrics_and_pool_error_paths():
    L = E.lib()
    m = E.Metrics()
    assert L.opure_engine_get_metrics(None, C.byref(m)) == H.E_INVALID
    assert b"null" in L.opure_engine_last_error()
    assert L.opure_engine_reset_metrics(None) == H.E_INVALID
    h = C.c_void_p()
    assert L.opure_page_pool_create(0, C.byref(h)) == H.E_INVALID and not h.value
    assert L.opure_page_pool_alloc(None, 1, None) == H.E_INVALID
    assert L.opure_page_pool_destroy(None) == H.OK


def state(p):
    """(free count, sorted ids handed out by draining the pool) without changing it."""
    k = p.available()
    ids = p.alloc(k)
    p.release(ids[::-1])            # back in the same stack order
    return k, sorted(ids.tolist())


def test_fresh_pool_order_and_all_or_none():
    p = E.PagePool(6)
    assert p.available() == 6
    assert p.alloc(3).tolist() == [0, 1, 2]
    with pytest.raises(H.OpureError) as e:
        p.alloc(4)
    assert e.value.code == H.E_CAPACITY
    assert p.available() == 3
    assert p.alloc(3).tolist() == [3, 4, 5]
    assert p.available() == 0
    assert p.alloc(0).size == 0


def test_release_is_lifo_and_skips_padding():
    p = E.PagePool(8)
    p.alloc(5)                                  # 0..4
    p.release(np.array([1, -1, 3, -1], np.int32))
    assert p.available() == 5
    assert p.alloc(2).tolist() == [3, 1]        # last released first
    assert p.alloc(1).tolist() == [5]           # then pages never used
    p.release([])


@pytest.mark.parametrize("bad", [[2, 9], [2, 2], [7], [-1, 2, 40]])
def test_bad_release_changes_nothing(bad):
    p = E.PagePool(8)
    p.alloc(4)                                  # 0..3 in use; 7 never handed out; 9, 40 past the pool
    before = state(p)
    with pytest.raises(H.OpureError) as e:
        p.release(np.array(bad, np.int32))
    assert e.value.code == H.E_INVALID
    assert state(p) == before
    p.release([0, 1, 2, 3])
    assert p.available() == 8


def test_grow_seq():
    p = E.PagePool(10)
    row = np.full(4, -1, np.int32)
    assert p.grow_seq(row, 17) == 2 and row.tolist() == [0, 1, -1, -1]
    assert p.grow_seq(row, 32) == 0                          # 32 tokens still fit in 2 pages
    assert p.grow_seq(row, 33) == 1 and row.tolist() == [0, 1, 2, -1]
    with pytest.raises(H.OpureError) as e:                   # 65 tokens need 5 pages, the row holds 4
        p.grow_seq(row, 65)
    assert e.value.code == H.E_CAPACITY and row.tolist() == [0, 1, 2, -1]
    q = E.PagePool(2)
    r2 = np.full(4, -1, np.int32)
    with pytest.raises(H.OpureError):                        # the pool holds 2 of the 3 pages needed
        q.grow_seq(r2, 40)
    assert r2.tolist() == [-1] * 4 and q.available() == 2


def test_speculative_loop_with_rollback_returns_every_page():
    """Sequences of a batch grow by K+1 positions per verify step (pages taken
    from the pool) and are rolled back to ctx + accepted + 1 (the oracle's
    rollback lists the pages wholly past that, which go back to the pool).
    After every step each row holds exactly ceil(len/16) distinct pages and
    the pool's free count is the rest."""
    hm = O.HostModel(n_layers=1, hidden=64, n_heads=4, n_kv_heads=2, head_dim=32, ffn=64, vocab=64,
                     wfmt=O.W_I8PC, afmt=O.A_F16, seed=5)
    B, K, n_pages, mpps = 4, 7, 64, 16
    kv = O.HostKV(hm, n_pages=n_pages, batch=B, max_pages_per_seq=mpps)
    p = E.PagePool(n_pages)
    rng = np.random.default_rng(11)
    seq_len = rng.integers(1, 40, B).astype(np.int32)
    for b in range(B):
        p.grow_seq(kv.page_table[b], int(seq_len[b]))
    for step in range(30):
        for b in range(B):                                   # room for the verify step's K+1 rows
            p.grow_seq(kv.page_table[b], int(seq_len[b]) + K + 1)
        acc = rng.integers(0, K + 1, B).astype(np.int32)
        new_len, freed, n_freed = O.kv_rollback(kv, hm, K, seq_len, acc, freed_stride=8)
        assert np.array_equal(new_len, seq_len + acc + 1)
        for b in range(B):
            assert (freed[b, n_freed[b]:] == -1).all()
        p.release(freed)
        seq_len = new_len
        if seq_len.max() + K + 1 > mpps * 16:                # a sequence ends: all its pages go back
            b = int(np.argmax(seq_len))
            p.release(kv.page_table[b])
            kv.page_table[b] = -1
            seq_len[b] = 1
            p.grow_seq(kv.page_table[b], 1)
        held = []
        for b in range(B):
            need = -(-int(seq_len[b]) // 16)
            row = kv.page_table[b]
            assert (row[:need] >= 0).all() and (row[need:] == -1).all(), (step, b, row.tolist())
            held += row[:need].tolist()
        assert len(set(held)) == len(held)
        assert p.available() == n_pages - len(held)
