"""Regenerates the reference harness's known-answer kernel setups as fixtures.

The reference stores no golden vectors: every kernel test in
src/app/Opure_TestHarness.cpp draws its inputs from a fixed-seed xorshift64
(:36-47) and recomputes the expected output in scalar float in the same run.
This script replays those setups (same seeds, same draw order, same float
arithmetic for the expected values) and writes inputs + expected outputs to
tests/golden/*.npz, so the oracle and the HIP path are checked against the
harness's own numbers.

  gemv_f32.npz        TestGEMV          :1176-1229  64x128, seed 0xC0FFEE01
  gemv_quant.npz      TestGEMVQuant     :1244-1311  64x128, seed 0x9A17BEEF
  rmsnorm.npz         TestRMSNorm       :1314-1361  d=256,  seed 0xBADF00D2
  swiglu.npz          TestSwiGLU        :1364-1400  n=64,   seed 0x5EED1234
  addres.npz          TestAddRes        :1554-1586  n=64,   seed 0xADDE5EED
  argmax.npz          TestArgMax        :1436-1471  49152,  seed 0x13571357
  attention_hdN.npz   TestAttentionAt   :1479-1547  4h/2kv/seq7/max64, N in 32..256

Run:  python tests/golden/make_golden.py
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F = np.float32


class Rng:
    def __init__(self, seed):
        self.s = seed if seed else 1

    def u32(self):
        s = self.s
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        self.s = s
        return s >> 32

    def f(self):
        return F(F(self.u32()) / F(2147483648.0)) - F(1.0)

    def fs(self, n):
        return np.array([self.f() for _ in range(n)], dtype=F)


def fdot_acc(w, x):
    acc = F(0.0)
    for a, b in zip(w, x):
        acc = F(acc + F(a * b))
    return acc


def gemv_f32():
    r = Rng(0xC0FFEE01)
    W = r.fs(64 * 128).reshape(64, 128)
    X = r.fs(128)
    ref = np.array([fdot_acc(W[o], X) for o in range(64)], dtype=F)
    np.savez(os.path.join(HERE, "gemv_f32.npz"), W=W, X=X, ref=ref)


def gemv_quant():
    r = Rng(0x9A17BEEF)
    q = np.array([np.int8(np.int32(F(r.f() * F(127.0))) - 63) for _ in range(64 * 128)],
                 dtype=np.int8).reshape(64, 128)
    X = np.array([F(F(r.f() * F(2.0)) - F(1.0)) for _ in range(128)], dtype=F)
    sW = F(0.0137)
    ref = np.zeros(64, dtype=F)
    for o in range(64):
        acc = F(0.0)
        for i in range(128):
            acc = F(acc + F(F(q[o, i]) * X[i]))
        ref[o] = F(F(acc * sW) * F(1.0))
    np.savez(os.path.join(HERE, "gemv_quant.npz"), q=q, X=X, sW=np.array([sW]), ref=ref)


def rmsnorm():
    r = Rng(0xBADF00D2)
    X = r.fs(256)
    G = np.array([F(r.f() * F(0.5)) for _ in range(256)], dtype=F)
    ss = 0.0
    for v in X:
        ss += float(v) * float(v)
    inv = F(1.0) / F(np.sqrt(F(F(ss / 256) + F(1e-5))))
    ref = np.array([F(F(X[i] * inv) * G[i]) for i in range(256)], dtype=F)
    np.savez(os.path.join(HERE, "rmsnorm.npz"), X=X, G=G, ref=ref)


def swiglu():
    r = Rng(0x5EED1234)
    G = np.array([F(r.f() * F(3.0)) for _ in range(64)], dtype=F)
    U = r.fs(64)
    ref = np.zeros(64, dtype=F)
    for i in range(64):
        s = F(F(1.0) / F(F(1.0) + np.exp(-G[i], dtype=F)))
        ref[i] = F(F(G[i] * s) * U[i])
    np.savez(os.path.join(HERE, "swiglu.npz"), G=G, U=U, ref=ref)


def addres():
    r = Rng(0xADDE5EED)
    X = np.array([F(F(r.f() * F(2.0)) - F(1.0)) for _ in range(64)], dtype=F)
    R = np.array([F(F(r.f() * F(2.0)) - F(1.0)) for _ in range(64)], dtype=F)
    np.savez(os.path.join(HERE, "addres.npz"), X=X, R=R, ref=(X + R).astype(F))


def argmax():
    r = Rng(0x13571357)
    Lg = np.array([F(r.f() * F(5.0)) for _ in range(49152)], dtype=F)
    best, bi = F(-1e30), 0
    for i, v in enumerate(Lg):
        if v > best:
            best, bi = v, i
    np.savez(os.path.join(HERE, "argmax.npz"), L=Lg, idx=np.array([bi]), val=np.array([best], dtype=F))


def attention(hd):
    heads, kv, seq, mx = 4, 2, 7, 64
    r = Rng((0xABCDEF01 ^ ((hd * 2654435761) & 0xFFFFFFFF)) & 0xFFFFFFFF)
    Q = r.fs(heads * hd).reshape(heads, hd)
    K = r.fs(kv * mx * hd).reshape(kv, mx, hd)
    V = r.fs(kv * mx * hd).reshape(kv, mx, hd)
    ref = np.zeros((heads, hd), dtype=F)
    grp = heads // kv
    for h in range(heads):
        kvh = h // grp
        m, l = F(-1e30), F(0.0)
        acc = np.zeros(hd, dtype=F)
        for s in range(seq):
            score = F(0.0)
            for d in range(hd):
                score = F(score + F(Q[h, d] * K[kvh, s, d]))
            nm = m if m > score else score
            corr = F(0.0) if m <= F(-1e29) else np.exp(F(m - nm), dtype=F)
            pv = np.exp(F(score - nm), dtype=F)
            l = F(F(l * corr) + pv)
            acc = (acc * corr + pv * V[kvh, s]).astype(F)
            m = nm
        ref[h] = (acc / l).astype(F)
    np.savez(os.path.join(HERE, f"attention_hd{hd}.npz"), Q=Q, K=K[:, :seq], V=V[:, :seq], ref=ref)


if __name__ == "__main__":
    gemv_f32()
    gemv_quant()
    rmsnorm()
    swiglu()
    addres()
    argmax()
    for hd in (32, 64, 96, 128, 160, 192, 224, 256):
        attention(hd)
    print("fixtures written to", HERE)
