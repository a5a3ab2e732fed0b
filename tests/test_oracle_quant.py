"""Closed-form pins of the oracle's quantisers, which define every int8 and
int4 benchmark model (oracle.quant_i8pc, oracle.quant_i4g128; the device
quantisers are checked bit for bit against these in the GPU suite).

The reference has only a per-tensor int8 scale (shaders/Opure_GEMV_Quant.usf:
39-95, y = sW * sX * sum int8(W) x) and an int4 widening with element 2i in the
high nibble (src/core/Opure_Streamer.cpp:403-426).  BASELINE's per-channel
int8 and group-128 int4 schemes are therefore pinned here by what the
mathematics fixes, independently of the quantiser's own arithmetic:

int8 per output row o:   s_o = fp16(amax_o / 127), |q| <= 127, q the code
                         nearest to w / s_o (brute force over all 255 codes),
                         |w - s_o q| <= s_o / 2, an all-zero row gives zero codes.
int4 per row and 128-group g:  s = bf16((max - min) / 15), z = bf16(-min / s),
                         q in [0, 15] the code nearest to w / s + z (brute force
                         over all 16), |w - s (q - z)| <= s (1/2 + |dz| + 15 * 2^-8)
                         where dz is z's bf16 rounding, an all-zero group is exact,
                         a constant group is within bf16 precision of its value,
                         element 2i sits in the high nibble of byte i.

Each plausible mistake (a scale of amax/128, codes from the unrounded scale,
swapped nibbles, an unrounded or integer zero point) is planted in a copy of the
quantiser below, and the test shows one of these checks rejects it."""
import numpy as np
import pytest

import oracle as O


# ---------------------------------------------------------------------------
#  independent helpers: rounding neighbourhoods and brute-force codes
# ---------------------------------------------------------------------------
def f16_half_ulp(x: np.ndarray) -> np.ndarray:
    """Half the fp16 spacing at |x| (normal range; subnormal spacing 2^-24)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 0.5 * 2.0 ** (e - 10)


def bf16_half_ulp(x: np.ndarray) -> np.ndarray:
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 0.5 * 2.0 ** (e - 7)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """Byte i of a row holds element 2i in its high nibble, 2i + 1 in its low
    one (the reference's int4 order, Opure_Streamer.cpp:403-426)."""
    O_, H = packed.shape
    q = np.empty((O_, 2 * H), dtype=np.int64)
    q[:, 0::2] = packed >> 4
    q[:, 1::2] = packed & 15
    return q


def nearest_code(target: np.ndarray, codes: np.ndarray) -> np.ndarray:
    """For every target value, the code with the smallest |target - code| by
    exhaustive search (ties cannot occur with continuous data)."""
    d = np.abs(target[..., None] - codes.astype(np.float64))
    return codes[np.argmin(d, axis=-1)]


# ---------------------------------------------------------------------------
#  the checks
# ---------------------------------------------------------------------------
def check_i8pc(w: np.ndarray, lin: dict) -> None:
    w = w.astype(np.float64)
    q = lin["w"].astype(np.int64)
    s = O.f16_bits_to_f32(lin["scale"]).astype(np.float64)
    amax = np.abs(w).max(axis=1)
    live = amax > 1e-3
    assert q.shape == w.shape and lin["scale"].shape == (w.shape[0],)
    assert np.abs(q).max() <= 127
    # the scale is amax / 127 rounded to fp16 (a slop of 1e-3 ulp for the f32 quotient)
    assert np.all(np.abs(s[live] - amax[live] / 127.0) <= f16_half_ulp(amax[live] / 127.0) * 1.001), "scale"
    # every code is the nearest of all 255 to w / s
    bf = nearest_code(w / s[:, None], np.arange(-127, 128))
    assert np.array_equal(q, bf), "codes"
    # reconstruction within half a step, and the row's largest |w| maps to 127
    assert np.all(np.abs(w - s[:, None] * q) <= s[:, None] * 0.5 * (1 + 1e-6)), "reconstruction"
    assert np.all(np.abs(q[live]).max(axis=1) == 127)
    # an all-zero row: zero codes and a finite positive scale
    zero = amax == 0
    assert np.all(q[zero] == 0) and np.all(np.isfinite(s[zero]) & (s[zero] > 0))


def check_i4g128(w: np.ndarray, lin: dict) -> None:
    w = w.astype(np.float64)
    O_, K = w.shape
    G = K // 128
    assert lin["w"].shape == (O_, K // 2) and lin["scale"].shape == (O_, G) and lin["zero"].shape == (O_, G)
    q = unpack_nibbles(lin["w"]).reshape(O_, G, 128)
    s = O.bf16_bits_to_f32(lin["scale"]).astype(np.float64)
    z = O.bf16_bits_to_f32(lin["zero"]).astype(np.float64)
    g = w.reshape(O_, G, 128)
    mn, mx = g.min(axis=2), g.max(axis=2)
    assert q.min() >= 0 and q.max() <= 15
    spread = (mx - mn) > 1e-3
    # s = (max - min) / 15 and z = -min / s, each rounded to bf16
    sr = (mx - mn) / 15.0
    assert np.all(np.abs(s[spread] - sr[spread]) <= bf16_half_ulp(sr[spread]) * 1.001), "scale"
    zr = -mn / s
    assert np.all(np.abs(z[spread] - zr[spread]) <= bf16_half_ulp(zr[spread]) * 1.001), "zero"
    # every code is the nearest of all 16 to w / s + z
    bf = nearest_code(g / s[..., None] + z[..., None], np.arange(16))
    assert np.array_equal(q, bf), "codes"
    # reconstruction: half a step, plus what z's rounding and the clip at 0 / 15 add
    dz = np.abs(z - zr)
    bound = s * (0.5 + dz + 15.0 * 2.0 ** -8)
    err = np.abs(g - s[..., None] * (q - z[..., None]))
    assert np.all(err[spread] <= bound[spread][..., None] * (1 + 1e-6)), "reconstruction"
    # groups without spread: an all-zero group is exact, a constant one is
    # within bf16 precision of its value
    flat = ~spread
    if np.any(flat):
        c = g[flat][:, 0]
        got = (s[..., None] * (q - z[..., None]))[flat]
        assert np.all(np.abs(got - g[flat]) <= np.abs(c)[:, None] * 2.0 ** -8 + 1e-7), "constant group"
        zg = np.all(g[flat] == 0.0, axis=1)
        assert np.all(got[zg] == 0.0), "zero group"


# ---------------------------------------------------------------------------
#  inputs: brute force at 8 x 256, with the special rows and groups
# ---------------------------------------------------------------------------
def matrix(seed: int, out: int = 8, inn: int = 256) -> np.ndarray:
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((out, inn)) * 0.02).astype(np.float32)
    w[1] = 0.0                                   # all-zero row (int8) / groups (int4)
    w[2, :128] = 0.01                            # a constant group
    w[2, 128:] = -0.37                           # another, negative
    w[3] *= 50.0                                 # a wide row
    w[4, 5] = 1.0                                # one outlier
    w[5] = np.abs(w[5])                          # a one-signed row (min > 0)
    w[6] = -np.abs(w[6])                         # (max < 0)
    return w


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quant_i8pc_closed_form(seed):
    w = matrix(seed)
    check_i8pc(w, O.quant_i8pc(w))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quant_i4g128_closed_form(seed):
    w = matrix(seed)
    check_i4g128(w, O.quant_i4g128(w))


def test_quantisers_at_a_benchmark_shape():
    """The same checks over a 64 x 4096 slab of N(0, 0.02) weights (the rows of
    a 1B / 8B linear)."""
    w = (np.random.default_rng(9).standard_normal((64, 4096)) * 0.02).astype(np.float32)
    check_i8pc(w, O.quant_i8pc(w))
    check_i4g128(w, O.quant_i4g128(w))


def test_integer_weights_reduce_to_an_integer_gemv():
    """Special case: rows whose largest |w| is 127 and whose values are integers
    get scale 1 and codes equal to the weights, so the int8 GEMV is an integer
    GEMV; groups spanning exactly 0..15 get scale 1, zero 0, codes = weights."""
    rng = np.random.default_rng(4)
    w = rng.integers(-127, 128, size=(4, 256)).astype(np.float32)
    w[:, 0] = 127.0
    lin = O.quant_i8pc(w)
    assert np.all(O.f16_bits_to_f32(lin["scale"]) == 1.0) and np.array_equal(lin["w"], w.astype(np.int8))
    w4 = rng.integers(0, 16, size=(4, 256)).astype(np.float32)
    w4[:, 0::128] = 0.0
    w4[:, 1::128] = 15.0
    l4 = O.quant_i4g128(w4)
    assert np.all(O.bf16_bits_to_f32(l4["scale"]) == 1.0) and np.all(O.bf16_bits_to_f32(l4["zero"]) == 0.0)
    assert np.array_equal(unpack_nibbles(l4["w"]), w4.astype(np.int64))


# ---------------------------------------------------------------------------
#  planted mistakes: each must fail one of the checks above
# ---------------------------------------------------------------------------
def i8_div128(w):
    lin = O.quant_i8pc(w)
    s16 = (np.maximum(np.abs(w).max(axis=1), 1e-8) / 128.0).astype(np.float16)
    s16[s16 == 0] = np.uint16(1).view(np.float16)
    q = np.clip(np.rint(w / s16.astype(np.float32)[:, None]), -127, 127).astype(np.int8)
    return dict(lin, w=q, scale=s16.view(np.uint16).copy())


def i8_unrounded_scale(w):
    lin = O.quant_i8pc(w)
    s = np.maximum(np.abs(w).max(axis=1), 1e-8) / 127.0                  # codes from the f32 scale
    return dict(lin, w=np.clip(np.rint(w / s[:, None]), -127, 127).astype(np.int8))


def i8_truncating(w):
    lin = O.quant_i8pc(w)
    s = O.f16_bits_to_f32(lin["scale"])
    return dict(lin, w=np.clip(np.trunc(w / s[:, None]), -127, 127).astype(np.int8))


def i4_swapped_nibbles(w):
    lin = O.quant_i4g128(w)
    p = lin["w"]
    return dict(lin, w=((p << 4) | (p >> 4)).astype(np.uint8))


def i4_unrounded_scale(w):
    lin = O.quant_i4g128(w)
    O_, K = w.shape
    g = w.reshape(O_, K // 128, 128)
    s = np.maximum(g.max(axis=2) - g.min(axis=2), 1e-8) / 15.0            # codes from the f32 scale
    z = O.bf16_bits_to_f32(lin["zero"])
    q = np.clip(np.rint(g / s[..., None] + z[..., None]), 0, 15).astype(np.uint8).reshape(O_, K)
    return dict(lin, w=((q[:, 0::2] << 4) | q[:, 1::2]).astype(np.uint8))


def i4_integer_zero(w):
    lin = O.quant_i4g128(w)
    O_, K = w.shape
    g = w.reshape(O_, K // 128, 128)
    s = O.bf16_bits_to_f32(lin["scale"])
    zi = np.rint(O.bf16_bits_to_f32(lin["zero"]))
    q = np.clip(np.rint(g / s[..., None] + zi[..., None]), 0, 15).astype(np.uint8).reshape(O_, K)
    return dict(lin, w=((q[:, 0::2] << 4) | q[:, 1::2]).astype(np.uint8),
                zero=O.np_f32_to_bf16_bits(zi.astype(np.float32)))


def i4_div16(w):
    lin = O.quant_i4g128(w)
    O_, K = w.shape
    g = w.reshape(O_, K // 128, 128)
    mn, mx = g.min(axis=2), g.max(axis=2)
    s_b = O.np_f32_to_bf16_bits(np.maximum(mx - mn, 1e-8) / 16.0)
    s = O.bf16_bits_to_f32(s_b)
    z_b = O.np_f32_to_bf16_bits(-mn / s)
    z = O.bf16_bits_to_f32(z_b)
    q = np.clip(np.rint(g / s[..., None] + z[..., None]), 0, 15).astype(np.uint8).reshape(O_, K)
    return dict(lin, w=((q[:, 0::2] << 4) | q[:, 1::2]).astype(np.uint8), scale=s_b.reshape(O_, -1),
                zero=z_b.reshape(O_, -1))


@pytest.mark.parametrize("mutant", [i8_div128, i8_unrounded_scale, i8_truncating])
def test_planted_int8_mistakes_are_caught(mutant):
    w = matrix(0)
    with pytest.raises(AssertionError):
        check_i8pc(w, mutant(w))


@pytest.mark.parametrize("mutant", [i4_swapped_nibbles, i4_unrounded_scale, i4_integer_zero, i4_div16])
def test_planted_int4_mistakes_are_caught(mutant):
    w = matrix(0)
    with pytest.raises(AssertionError):
        check_i4g128(w, mutant(w))
