"""opure_accept_rejection_noalloc (the acceptance entry point that allocates
nothing: its scratch is a device array built into the library) against
opure_accept_rejection on the same inputs: ids, accepted lengths and the
final-token distributions bit for bit, on two calls in a row -- the second
with a smaller batch and vocabulary, so it runs over what the first left in
the shared array -- and a shape beyond the array is refused."""
import ctypes as C

import numpy as np
import pytest

import opure_hip as H
import oracle as O
from gpu_util import say

pytestmark = pytest.mark.gpu


def call(dev, fn, t, q, drafts, tau, seed):
    B, K1, V = t.shape
    tb, qb, db = dev.upload(t), dev.upload(q), dev.upload(np.ascontiguousarray(drafts, np.int32))
    ot, ac, di = dev.alloc(B * K1 * 4), dev.alloc(B * 4), dev.alloc(B * V * 4)
    a = H.AcceptArgs(B, K1 - 1, V, int(tb), int(qb), int(db), K1 - 1, tau, seed, None, int(ot), int(ac), int(di))
    rc = fn(dev.h, C.byref(a))
    if rc == H.OK:
        dev.sync()
        res = (dev.download(ot, np.int32, (B, K1)), dev.download(ac, np.int32, (B,)), dev.download(di, np.float32, (B, V)))
    else:
        res = rc
    for b in (tb, qb, db, ot, ac, di):
        b.free()
    return res


def inputs(B, K, V, seed):
    rng = np.random.default_rng(seed)
    t = (rng.standard_normal((B, K + 1, V)) * 3.0).astype(np.float32)
    q = (rng.standard_normal((B, K, V)) * 3.0).astype(np.float32)
    pos = np.repeat(np.arange(K)[None], B, 0).ravel()
    seqs = np.repeat(np.arange(B)[:, None], K, 1).ravel()
    d = O.sample_rows(q.reshape(-1, V), 1.0, seed, pos, seqs, 0).reshape(B, K)
    q[: B // 2] = t[: B // 2, :K]          # half the batch accepts every draft
    return t, q, d


def test_noalloc_equals_allocating_entry_point():
    dev = H.Dev(0)
    try:
        L = H.lib()
        for (B, K, V, seed) in [(64, 8, 49152, 5), (7, 3, 1000, 6)]:
            say("noalloc rejection", B, K, V)
            t, q, d = inputs(B, K, V, seed)
            want = call(dev, L.opure_accept_rejection, t, q, d, 1.0, 99)
            got = call(dev, L.opure_accept_rejection_noalloc, t, q, d, 1.0, 99)
            assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
            assert np.array_equal(got[2], want[2])
            assert (got[1][: B // 2] == K).all()
        # a batch whose scratch exceeds the array is refused, and nothing runs
        t, q, d = inputs(80, 2, 128256, 7)
        assert call(dev, L.opure_accept_rejection_noalloc, t, q, d, 1.0, 99) == H.E_CAPACITY
        assert b"scratch" in L.opure_last_error()
    finally:
        dev.close()
