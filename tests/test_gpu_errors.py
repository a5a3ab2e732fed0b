"""Failures that only a kernel can see reach the host as error codes at the
next sync, and the device keeps working afterwards.  Every condition is forced
from the host; every kernel still runs to its end (no fault, no hang):

- a token id outside the vocabulary (its embedding row is NaN)  -> OPURE_E_INVALID
- a row position at or past max_ctx and the page table          -> OPURE_E_CAPACITY
- a bounded wait between waves that gives up (wait limit 0)     -> OPURE_E_DEVICE
- a workspace that grows while a captured graph points into the old one
  leaves the graph replaying correctly (the old buffer is kept until the last
  graph is destroyed).
"""
import ctypes as C

import numpy as np
import pytest

import opure_hip as H
import oracle as O
from gpu_util import VerifyRunner, device_kv, device_model, say
from test_gpu_verify import random_cache, small_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = H.Dev(0)
    yield d
    d.close()


def sync_code(dev):
    try:
        dev.sync()
        return H.OK
    except H.OpureError as e:
        say("reported:", e)
        return e.code


def small_step(dev, B=1, R=4, max_ctx=256, fmt=(O.W_I8PC, O.A_F16)):
    m = small_model(*fmt)
    kv = random_cache(m, B, max_ctx, 32 * B, seed=3)
    dm, dkv = device_model(dev, m), device_kv(dev, m, kv)
    return m, kv, dkv, VerifyRunner(dev, dm, dkv, B, R, max_ctx)


def launch(dev, run, tokens, seq_len, **kw):
    dev.write(run.tokens, np.ascontiguousarray(tokens, np.int32))
    dev.write(run.seq_len, np.ascontiguousarray(seq_len, np.int32))
    a = run.args(**kw)
    H.check(H.lib().opure_verify_step(dev.h, C.byref(a)))


def test_token_outside_vocabulary_is_reported(dev):
    m, kv, dkv, run = small_step(dev)
    V = m.cfg["vocab"]
    launch(dev, run, [[1, 2, V + 5, 3]], [40])
    assert sync_code(dev) == H.E_INVALID
    assert b"vocabulary" in H.lib().opure_last_error()
    assert np.isnan(run.get_logits()[0, 2]).all()
    # cleared: the next good step syncs clean
    launch(dev, run, [[1, 2, 4, 3]], [40])
    assert sync_code(dev) == H.OK
    assert np.isfinite(run.get_logits()).all()


@pytest.mark.parametrize("fmt", [(O.W_I8PC, O.A_F16), (O.W_F32, O.A_F32)], ids=["i8-f16", "f32"])
def test_position_past_max_ctx_is_reported(dev, fmt):
    """Matrix-core attention + combine (f16), and the fp32 short-context
    kernel that merges its chunks itself: both report the row past max_ctx."""
    m, kv, dkv, run = small_step(dev, max_ctx=256, fmt=fmt)
    # the last row sits at 254 + 3 = 257, past max_ctx = 256 and the 16 pages of the table
    launch(dev, run, [[1, 2, 3, 4]], [254])
    assert sync_code(dev) == H.E_CAPACITY
    assert b"max_ctx" in H.lib().opure_last_error()
    launch(dev, run, [[1, 2, 3, 4]], [250])
    assert sync_code(dev) == H.OK


def test_gemv_wait_that_gives_up_is_reported(dev):
    """The 8B gate/up shape (1792 tiles) at 8 rows runs the loader-wave GEMV.
    With a wait limit of 0 sleeps, every wait not already met gives up at
    once: the launch completes, its results are wrong, and the sync says so.
    With the default limit the same launch is clean and matches a reference
    run bit for bit."""
    rng = np.random.default_rng(8)
    out, inn, M = 2 * 14336, 4096, 8
    lin = O.make_linear(rng, out, inn, O.W_I4G128)
    w, s, z = dev.upload(lin["w"]), dev.upload(lin["scale"]), dev.upload(lin["zero"])
    rm = H.Linear(int(w), int(s), int(z), out, inn, H.LAYOUT_ROWMAJOR)
    tl, keep = dev.tile(H.W_I4G128, rm, H.LAYOUT_TILED_SWIGLU)
    x = O.np_f32_to_bf16_bits(rng.standard_normal((M, inn)).astype(np.float32)).reshape(M, inn)
    xb = dev.upload(x)
    yb = dev.alloc(M * (out // 2) * 2)
    a = H.GemvArgs(tl, int(xb), int(yb), M, H.A_BF16, H.A_BF16, H.EPI_SWIGLU)
    L = H.lib()
    H.check(L.opure_gemv_batched_i4g128(dev.h, C.byref(a)))
    assert sync_code(dev) == H.OK
    ref = dev.download(yb, np.uint16, (M, out // 2))
    H.check(L.opure_debug_set_wait_limit(dev.h, 0))
    try:
        H.check(L.opure_gemv_batched_i4g128(dev.h, C.byref(a)))
        assert sync_code(dev) == H.E_DEVICE
        assert b"gave up" in L.opure_last_error()
    finally:
        H.check(L.opure_debug_set_wait_limit(dev.h, 1 << 22))
    H.check(L.opure_gemv_batched_i4g128(dev.h, C.byref(a)))
    assert sync_code(dev) == H.OK
    assert np.array_equal(dev.download(yb, np.uint16, (M, out // 2)), ref)


def test_rejection_wait_gives_up_then_recovers(dev):
    """The one-launch rejection step's slices wait for each other with the
    same bounded wait.  At 0 sleeps a slice whose wait is not already met
    gives up at once: the launch completes and the sync reports it (unless
    every wait happened to be met).  Either way the sequences' launch counts
    move on, so the next launches at the default limit never take a value
    the failed launch published for one of theirs, and match the oracle bit
    for bit."""
    rng = np.random.default_rng(9)
    B, K, V, tau = 16, 4, 30000, 0.8
    t = (rng.standard_normal((B, K + 1, V)) * 3).astype(np.float32)
    q = (rng.standard_normal((B, K, V)) * 3).astype(np.float32)
    q[: B // 2] = t[: B // 2, :K] + (rng.standard_normal((B // 2, K, V)) * 0.05).astype(np.float32)
    pos = np.repeat(np.arange(K)[None], B, 0).ravel()
    seq = np.repeat(np.arange(B)[:, None], K, 1).ravel()
    drafts = O.sample_rows(q.reshape(B * K, V), tau, 5, pos, seq, 0).reshape(B, K)
    w_out, w_acc, _ = O.accept_rejection(t, q, drafts, tau, 5, None)
    tb, qb, db = dev.upload(t), dev.upload(q), dev.upload(drafts.astype(np.int32))
    ot, ac = dev.alloc(B * (K + 1) * 4), dev.alloc(B * 4)
    a = H.AcceptArgs(B, K, V, int(tb), int(qb), int(db), K, tau, 5, None, int(ot), int(ac), None)
    L = H.lib()
    H.check(L.opure_debug_set_wait_limit(dev.h, 0))
    try:
        H.check(L.opure_accept_rejection(dev.h, C.byref(a)))
        code = sync_code(dev)
        assert code in (H.OK, H.E_DEVICE)
        if code == H.E_DEVICE:
            assert b"gave up" in L.opure_last_error()
    finally:
        H.check(L.opure_debug_set_wait_limit(dev.h, 1 << 22))
    for _ in range(2):
        H.check(L.opure_accept_rejection(dev.h, C.byref(a)))
        assert sync_code(dev) == H.OK
        assert np.array_equal(dev.download(ac, np.int32, (B,)), w_acc)
        assert np.array_equal(dev.download(ot, np.int32, (B, K + 1)), w_out)
    for buf in (tb, qb, db, ot, ac):
        buf.free()


def test_graph_survives_workspace_growth(dev):
    """A step captured into a graph, then an eager call that needs a larger
    workspace: the graph still replays to the eager result of its own shape."""
    m, kv, dkv, run = small_step(dev, B=1, R=4, max_ctx=256)
    tokens, seq = [[5, 6, 7, 8]], [100]
    launch(dev, run, tokens, seq, accept=H.ACCEPT_GREEDY)
    assert sync_code(dev) == H.OK
    eager = run.get_logits()
    a = run.args(accept=H.ACCEPT_GREEDY)
    dev.graph_begin()
    H.check(H.lib().opure_verify_step(dev.h, C.byref(a)))
    g = dev.graph_end()
    ws, before = C.c_void_p(), C.c_uint64()
    H.check(H.lib().opure_debug_workspace(dev.h, C.byref(ws), C.byref(before)))
    # a much larger eager call: the workspace is replaced
    big = small_model(O.W_I8PC, O.A_F16, vocab=65536)
    bkv = random_cache(big, 8, 1024, 8 * 64 + 8, seed=4)
    brun = VerifyRunner(dev, device_model(dev, big), device_kv(dev, big, bkv), 8, 16, 1024)
    brun.step(np.random.default_rng(0).integers(0, 65536, size=(8, 16)), [900] * 8)
    after = C.c_uint64()
    H.check(H.lib().opure_debug_workspace(dev.h, C.byref(ws), C.byref(after)))
    assert after.value > before.value
    for _ in range(3):
        dev.fill_u32(run.logits, 0x7FC00000, 4 * m.cfg["vocab"])
        dkv.set_pool(kv.pool)
        dev.graph_launch(g)
        assert sync_code(dev) == H.OK
        assert np.array_equal(run.get_logits(), eager)
    dev.graph_destroy(g)
