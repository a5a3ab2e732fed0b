"""Pins the oracle's building blocks.

Known answers: the reference harness's own kernel setups (tests/golden, made by
tests/golden/make_golden.py), judged by the harness's pass rule
Compare() (Opure_TestHarness.cpp:70-101: rms <= 1e-5 * max|ref|).
Closed forms and invariants cover what the harness never tested: per-channel
int8 and group-128 int4 decoding, RoPE, paged GQA attention.
"""
import ctypes as C
import math
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def harness_compare(got, want):
    got = np.asarray(got, dtype=np.float64).ravel()
    want = np.asarray(want, dtype=np.float64).ravel()
    assert not np.isnan(got).any()
    rms = math.sqrt(np.mean((got - want) ** 2))
    scale = max(1e-6, np.abs(want).max())
    return rms <= 1e-5 * scale or rms <= 1e-7


def test_gemv_f32_known_answer():
    g = np.load(os.path.join(GOLD, "gemv_f32.npz"))
    lin = {"w": g["W"], "out": 64, "in": 128}
    y = O.gemv(lin, O.W_F32, g["X"][None, :])[0]
    assert harness_compare(y, g["ref"])
    np.testing.assert_allclose(y, g["W"].astype(np.float64) @ g["X"].astype(np.float64), rtol=0, atol=1e-6)


def test_gemv_quant_known_answer_per_channel():
    g = np.load(os.path.join(GOLD, "gemv_quant.npz"))
    s16 = np.full(64, np.float16(g["sW"][0])).view(np.uint16)
    lin = {"w": g["q"], "scale": s16, "out": 64, "in": 128}
    y = O.gemv(lin, O.W_I8PC, g["X"][None, :])[0]
    # the harness uses a per-tensor fp32 scale; the per-channel format stores it as fp16
    adj = np.float64(np.float16(g["sW"][0])) / np.float64(g["sW"][0])
    assert harness_compare(y, g["ref"].astype(np.float64) * adj)


def test_gemv_i8_per_channel_closed_form():
    rng = np.random.default_rng(11)
    q = rng.integers(-127, 128, size=(48, 96), dtype=np.int8)
    s = (rng.uniform(0.001, 0.1, 48)).astype(np.float16)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    lin = {"w": q, "scale": s.view(np.uint16), "out": 48, "in": 96}
    y = O.gemv(lin, O.W_I8PC, x)
    want = (x.astype(np.float64) @ q.astype(np.float64).T) * s.astype(np.float64)[None, :]
    np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-7)


def test_gemv_i4_integer_special_case_and_nibble_order():
    # all scales 1, zeros 0 -> an integer GEMV; element 2i is the high nibble
    rng = np.random.default_rng(12)
    O_, K = 8, 256
    qv = rng.integers(0, 16, size=(O_, K), dtype=np.uint8)
    packed = ((qv[:, 0::2] << 4) | qv[:, 1::2]).astype(np.uint8)
    one = np.full((O_, K // 128), O.np_f32_to_bf16_bits(np.float32(1.0)))
    zero = np.zeros((O_, K // 128), dtype=np.uint16)
    x = rng.integers(-4, 5, size=(2, K)).astype(np.float32)
    lin = {"w": packed, "scale": one, "zero": zero, "out": O_, "in": K}
    y = O.gemv(lin, O.W_I4G128, x)
    assert np.array_equal(y, (x.astype(np.int64) @ qv.astype(np.int64).T).astype(np.float32))


def test_gemv_i4_group_scale_zero_closed_form():
    rng = np.random.default_rng(13)
    w = rng.standard_normal((16, 384)).astype(np.float32) * 0.02
    lin = O.quant_i4g128(w)
    x = rng.standard_normal((4, 384)).astype(np.float32)
    y = O.gemv(lin, O.W_I4G128, x)
    np.testing.assert_allclose(y, x.astype(np.float64) @ O.dequant(lin, O.W_I4G128).T, rtol=1e-6, atol=1e-7)
    # constant group: q = z exactly -> that group contributes nothing
    lin2 = dict(lin)
    lin2["w"] = lin["w"].copy()
    lin2["zero"] = lin["zero"].copy()
    lin2["w"][:, :64] = 0x77
    lin2["zero"][:, 0] = O.np_f32_to_bf16_bits(np.float32(7.0))
    y2 = O.gemv(lin2, O.W_I4G128, x)
    x0 = x.copy()
    x0[:, :128] = 123.0   # must not matter
    y3 = O.gemv(lin2, O.W_I4G128, x0)
    np.testing.assert_allclose(y2, y3, rtol=1e-6, atol=1e-6)


def test_i4_decode_exhaustive_bytes():
    # one row of 256 bytes = every byte value; decode must give (hi, lo) per byte
    packed = np.arange(256, dtype=np.uint8)[None, :]
    one = np.full((1, 4), O.np_f32_to_bf16_bits(np.float32(1.0)))
    zero = np.zeros((1, 4), dtype=np.uint16)
    lin = {"w": packed, "scale": one, "zero": zero, "out": 1, "in": 512}
    for i in range(0, 512, 37):
        x = np.zeros((1, 512), dtype=np.float32)
        x[0, i] = 1.0
        b = i // 2
        want = (b >> 4) if i % 2 == 0 else (b & 15)
        assert O.gemv(lin, O.W_I4G128, x)[0, 0] == want


def test_rmsnorm_known_answer():
    g = np.load(os.path.join(GOLD, "rmsnorm.npz"))
    y = np.zeros((1, 256), dtype=np.float32)
    X, G = np.ascontiguousarray(g["X"]), np.ascontiguousarray(g["G"])
    O.lib().orc_rmsnorm_rows(X.ctypes.data, G.ctypes.data, y.ctypes.data, 1, 256, 1e-5, O.A_F32)
    assert harness_compare(y, g["ref"])


def test_swiglu_known_answer():
    g = np.load(os.path.join(GOLD, "swiglu.npz"))
    h = np.zeros(64, dtype=np.float32)
    G, U = np.ascontiguousarray(g["G"]), np.ascontiguousarray(g["U"])
    O.lib().orc_swiglu(G.ctypes.data, U.ctypes.data, h.ctypes.data, 64)
    assert harness_compare(h, g["ref"])


def test_argmax_known_answer_and_ties():
    g = np.load(os.path.join(GOLD, "argmax.npz"))
    idx, val = np.zeros(1, np.int32), np.zeros(1, np.float32)
    L = np.ascontiguousarray(g["L"])
    O.lib().orc_argmax_rows(L.ctypes.data, 1, L.size, idx.ctypes.data, val.ctypes.data)
    assert idx[0] == g["idx"][0] and val[0] == g["val"][0]
    t = np.zeros(100, dtype=np.float32)
    t[[17, 42, 99]] = 3.0
    O.lib().orc_argmax_rows(t.ctypes.data, 1, 100, idx.ctypes.data, val.ctypes.data)
    assert idx[0] == 17


def _attn_desc(n_heads, n_kv, hd, afmt=O.A_F32, scale=1.0):
    m = O.OrcModel()
    m.n_heads, m.n_kv_heads, m.head_dim, m.attn_scale, m.afmt, m.n_layers = n_heads, n_kv, hd, scale, afmt, 1
    return m


def _paged(K, V, page_size, perm):
    """Scatter contiguous K/V [kv][seq][hd] into a paged pool following `perm`."""
    n_kv, seq, hd = K.shape
    n_pages = max(perm) + 1 if len(perm) else 1
    pool = np.zeros((1, n_pages, 2, n_kv, page_size, hd), dtype=np.float32)
    Kp, Vp = O.kv_planes(pool)
    for s in range(seq):
        Kp[0, perm[s // page_size], :, s % page_size] = K[:, s]
        Vp[0, perm[s // page_size], :, s % page_size] = V[:, s]
    pt = np.array([perm], dtype=np.int32)
    return pool, pt


def _run_attn(m, pool, pt, ctx, R, q, page_size):
    kv = O.OrcKV(pool.ctypes.data, pool.shape[1], page_size, pt.ctypes.data, pt.shape[1])
    out = np.zeros_like(q)
    O.lib().orc_attention_paged(C.byref(m), C.byref(kv), 0, 0, ctx, R, q.ctypes.data, out.ctypes.data)
    return out


@pytest.mark.parametrize("hd", [32, 64, 96, 128, 160, 192, 224, 256])
def test_attention_known_answer(hd):
    g = np.load(os.path.join(GOLD, f"attention_hd{hd}.npz"))
    m = _attn_desc(4, 2, hd)
    pool, pt = _paged(g["K"], g["V"], 16, [0])
    q = np.ascontiguousarray(g["Q"].reshape(1, 4 * hd))
    out = _run_attn(m, pool, pt, 6, 1, q, 16)
    assert harness_compare(out, g["ref"].reshape(1, -1))


def test_attention_paged_invariants():
    rng = np.random.default_rng(5)
    nh, nkv, hd, seq, ps = 8, 2, 32, 53, 16
    K = rng.standard_normal((nkv, seq, hd)).astype(np.float32)
    V = rng.standard_normal((nkv, seq, hd)).astype(np.float32)
    m = _attn_desc(nh, nkv, hd, scale=0.25)
    R = 3
    q = rng.standard_normal((R, nh * hd)).astype(np.float32)
    pool_a, pt_a = _paged(K, V, ps, [0, 1, 2, 3])
    pool_b, pt_b = _paged(K, V, ps, [6, 2, 5, 0])
    ctx = seq - R
    a = _run_attn(m, pool_a, pt_a, ctx, R, q, ps)
    b = _run_attn(m, pool_b, pt_b, ctx, R, q, ps)
    assert np.array_equal(a, b)                    # invariant to page placement
    # closed form, float64, with GQA map h -> h // (nh / nkv) and causal rows
    grp = nh // nkv
    for j in range(R):
        for h in range(nh):
            s = 0.25 * (K[h // grp, :ctx + j + 1].astype(np.float64) @ q[j, h * hd:(h + 1) * hd].astype(np.float64))
            p = np.exp(s - s.max())
            want = (p / p.sum()) @ V[h // grp, :ctx + j + 1].astype(np.float64)
            np.testing.assert_allclose(a[j, h * hd:(h + 1) * hd], want, rtol=2e-5, atol=2e-6)
    # one cached token: the softmax has one term, so the output is V exactly
    one = _run_attn(m, pool_a, pt_a, 0, 1, q[:1], ps)
    for h in range(nh):
        assert np.array_equal(one[0, h * hd:(h + 1) * hd], V[h // grp, 0])


@pytest.mark.parametrize("mode", [O.ROPE_GPU, O.ROPE_CPUREF])
def test_rope_table_closed_form(mode):
    theta, hd, mp = 10000.0, 64, 300
    cos, sin = O.rope_table(theta, hd, mp, mode)
    for pos in (0, 1, 7, 299):
        for p in (0, 1, 5, 31):
            e = (2 * p) if mode == O.ROPE_CPUREF else p
            t = pos * theta ** (-2.0 * e / hd)
            assert cos[pos, p] == np.float32(math.cos(t))
            assert sin[pos, p] == np.float32(math.sin(t))


def test_rope_invariants():
    hd, nh = 64, 3
    cos, sin = O.rope_table(500000.0, hd, 4096)
    rng = np.random.default_rng(9)
    v = rng.standard_normal(nh * hd).astype(np.float32)

    def rot(x, pos):
        y = x.copy()
        O.lib().orc_rope_rows(y.ctypes.data, nh, hd, cos.ctypes.data, sin.ctypes.data, pos)
        return y

    assert np.array_equal(rot(v, 0), v)            # pos 0 is the identity
    r = rot(v, 1234)
    pairs_in = v.reshape(-1, 2).astype(np.float64)
    pairs_out = r.reshape(-1, 2).astype(np.float64)
    np.testing.assert_allclose(np.hypot(*pairs_out.T), np.hypot(*pairs_in.T), rtol=2e-6)
    np.testing.assert_allclose(rot(rot(v, 100), 900), rot(v, 1000), rtol=0, atol=5e-5)
    # interleaved pairs (2p, 2p+1), not rotate-half: pair 0 rotates by pos*1
    x = np.zeros(nh * hd, dtype=np.float32)
    x[0] = 1.0
    y = rot(x, 1)
    assert abs(y[0] - math.cos(1.0)) < 1e-7 and abs(y[1] - math.sin(1.0)) < 1e-7
