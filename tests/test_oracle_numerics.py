"""Pins the oracle's scalar numerics against independent definitions.

- fp16 widening: exhaustive over all 65536 patterns against numpy's IEEE float16.
- fp16 / bf16 narrowing: edge cases and random values against numpy / torch RNE.
- Philox4x32-10: the Random123 known-answer vectors (kat_vectors, philox4x32 R=10).
- exp: accuracy against the correctly rounded double exp, and special values.
- xorshift64: the reference harness RNG (Opure_TestHarness.cpp:36-47), restated
  independently here with Python integers.
"""
import math

import numpy as np
import pytest

import oracle as O


def test_f16_widen_exhaustive():
    L = O.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([L.orc_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_narrow_matches_ieee_rne():
    rng = np.random.default_rng(7)
    edge = np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 2.0**-24, 2.0**-25,
                     1.5 * 2.0**-25, 2.0**-14, 2.0**-14 * (1 - 2.0**-11), 6.1e-5, 3e-8, np.inf, -np.inf,
                     0.33325195, 1.0009765625, 1.00048828125, 1.000732421875],
                    dtype=np.float32)
    vals = np.concatenate([edge, rng.standard_normal(20000).astype(np.float32) * 10,
                           (rng.standard_normal(5000) * 1e-5).astype(np.float32),
                           rng.uniform(-70000, 70000, 2000).astype(np.float32)])
    got = O.f32_to_f16_bits(vals)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_narrow_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(8)
    vals = np.concatenate([np.array([0.0, -0.0, 1.0, 3.0e38, -3.4e38, 1e-40, np.inf, -np.inf], dtype=np.float32),
                           rng.standard_normal(20000).astype(np.float32) * 50,
                           (rng.standard_normal(2000) * 1e-39).astype(np.float32)])
    got = O.f32_to_bf16_bits(vals)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    # the numpy helper the tests use for bf16 packing must agree too
    assert np.array_equal(O.np_f32_to_bf16_bits(vals), want)


@pytest.mark.parametrize("ctr,key,want", [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
])
def test_philox_known_answers(ctr, key, want):
    assert [int(v) for v in O.philox(ctr, key)] == want


def test_philox_u32_keying():
    L = O.lib()
    seed = 0x0123456789ABCDEF
    got = L.orc_philox_u32(seed, 5, 7, 2)
    want = O.philox([5, 7, 2, 0], [seed & 0xFFFFFFFF, seed >> 32])[0]
    assert got == want


def _ulp_dist(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


def test_expf_accuracy():
    L = O.lib()
    xs = np.concatenate([np.linspace(-87.3, 88.7, 20001), np.linspace(-1, 1, 4001),
                         np.random.default_rng(3).uniform(-30, 0, 20000)]).astype(np.float32)
    got = np.array([L.orc_expf(float(x)) for x in xs], dtype=np.float32)
    want = np.array([math.exp(float(x)) for x in xs], dtype=np.float64).astype(np.float32)
    d = _ulp_dist(got, want)
    assert d.max() <= 2, (xs[d.argmax()], got[d.argmax()], want[d.argmax()])


def test_expf_special_values():
    L = O.lib()
    assert L.orc_expf(0.0) == 1.0
    assert L.orc_expf(-100.0) == 0.0
    assert L.orc_expf(-1e30) == 0.0
    assert math.isinf(L.orc_expf(89.0))
    assert math.isnan(L.orc_expf(float("nan")))
    # monotone over a fine grid
    xs = np.linspace(-20, 0, 50001).astype(np.float32)
    ys = np.array([L.orc_expf(float(x)) for x in xs], dtype=np.float32)
    assert np.all(np.diff(ys) >= 0)


def test_xorshift_matches_reference_definition():
    seed = 0xC0FFEE01
    s = seed
    want = []
    for _ in range(1000):
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        want.append(s >> 32)
    got = np.zeros(1000, dtype=np.uint32)
    O.lib().orc_xorshift_u32(seed, got.ctypes.data, 1000)
    assert [int(v) for v in got] == want
    f = np.zeros(1000, dtype=np.float32)
    O.lib().orc_xorshift_fill(seed, f.ctypes.data, 1000, 1.0, 0.0)
    wf = (np.array(want, dtype=np.uint32).astype(np.float32) / np.float32(2147483648.0)) - np.float32(1.0)
    assert np.array_equal(f, wf)
