"""GPU parity of the individual kernels against the CPU oracle, through the C-ABI.

Bars: integer/index work (argmax, acceptance, sampling, Philox, rollback) is
bit-exact; fp32 GEMV/attention within fp32 accumulation error; fp16/bf16
outputs within one storage ulp plus accumulation error.  Every GEMV is also
checked for row independence (M=1 equals row 0 of M=16, bit for bit) and
run-to-run determinism.
"""
import ctypes as C
import os

import numpy as np
import pytest

import opure_hip as H
import oracle as O
from gpu_util import say

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def dev():
    d = H.Dev(0)
    say("device:", d.name, d.hbm_bytes >> 30, "GiB")
    yield d
    d.close()


def to_act(x, afmt):
    x = np.asarray(x, dtype=np.float32)
    if afmt == H.A_F32:
        return x.copy(), x.copy()
    if afmt == H.A_F16:
        b = x.astype(np.float16).view(np.uint16)
        return b, b.view(np.float16).astype(np.float32)
    b = O.np_f32_to_bf16_bits(x).reshape(x.shape)
    return b, O.bf16_bits_to_f32(b).reshape(x.shape)


def from_act(b, afmt):
    if afmt == H.A_F32:
        return b.astype(np.float32)
    if afmt == H.A_F16:
        return b.view(np.float16).astype(np.float32)
    return O.bf16_bits_to_f32(b).reshape(b.shape)


def dev_linear(dev, lin):
    w = dev.upload(lin["w"])
    s = dev.upload(lin["scale"]) if lin.get("scale") is not None else None
    z = dev.upload(lin["zero"]) if lin.get("zero") is not None else None
    return H.Linear(int(w), int(s) if s else None, int(z) if z else None, lin["out"], lin["in"]), (w, s, z)


def np_tiled(wfmt, lin, layout):
    """numpy restatement of the tiled layout (opure_tile_linear): weight bytes
    and scale words, from the row-major linear."""
    out, inn = lin["out"], lin["in"]
    tiles = out // 16
    t, r = np.divmod(np.arange(out), 16)
    if layout == H.LAYOUT_TILED_SWIGLU:
        perm = np.where(r % 2 == 1, out // 2 + 8 * t + r // 2, 8 * t + r // 2)
    else:
        perm = np.arange(out)
    wb = np.ascontiguousarray(lin["w"]).view(np.uint8).reshape(out, -1)[perm]
    if wfmt == H.W_I8PC:
        wb = wb ^ np.uint8(0x80)
    elif wfmt == H.W_I4G128:
        d = np.ascontiguousarray(wb).view(np.uint32)
        o = np.zeros_like(d)
        for e, pos in enumerate((0, 4, 1, 5, 2, 6, 3, 7)):
            byte = (d >> np.uint32(8 * (e // 2))) & np.uint32(0xFF)
            q = (byte & np.uint32(0xF)) if e % 2 else (byte >> np.uint32(4))
            o |= q << np.uint32(4 * pos)
        o = (o << np.uint32(3)) | (o >> np.uint32(29))          # stored rotated left by 3 bits
        wb = o.view(np.uint8).reshape(out, -1)
    nblk = wb.shape[1] // 64
    tiled = wb.reshape(tiles, 16, nblk, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)
    if wfmt == H.W_F32:
        return tiled, None
    if wfmt == H.W_I8PC:
        return tiled, lin["scale"][perm]
    G = inn // 128
    sc = lin["scale"][perm].reshape(tiles, 16, G).transpose(0, 2, 1).astype(np.uint32)
    zr = lin["zero"][perm].reshape(tiles, 16, G).transpose(0, 2, 1).astype(np.uint32)
    return tiled, (sc | (zr << np.uint32(16))).reshape(-1)


def _rounding_cases():
    """f32 values that pin round-to-nearest-even narrowing: random bit patterns
    over the whole finite range, exact ties (even and odd) for both formats,
    subnormal results, overflow to infinity, signed zeros and infinities."""
    rng = np.random.default_rng(5)
    bits = [rng.integers(0, 0x7F800000, 200000, dtype=np.uint32)]
    hi = rng.integers(0x3000, 0x4780, 20000, dtype=np.uint32) << np.uint32(16)
    bits += [hi | np.uint32(0x8000), hi | np.uint32(0x7FFF), hi | np.uint32(0x8001)]   # bf16 ties and neighbours
    f16e = rng.integers(0x33000000, 0x47800000, 20000, dtype=np.uint32) & np.uint32(0xFFFFE000)
    bits += [f16e | np.uint32(0x1000), f16e | np.uint32(0x0FFF)]                       # f16 ties
    bits += [np.array([0, 0x7F800000, 0x477FF000, 0x477FEFFF, 0x47800000, 0x33000000, 0x33000001,
                       0x00000001, 0x007FFFFF, 0x7F7FFFFF], np.uint32)]
    b = np.concatenate(bits)
    return np.concatenate([b, b | np.uint32(0x80000000)]).view(np.float32)


@pytest.mark.parametrize("afmt", [H.A_F16, H.A_BF16], ids=["f16", "bf16"])
def test_narrowing_rounds_to_nearest_even(dev, afmt):
    """The device's f32 -> f16/bf16 narrowing (hardware conversions used by
    every kernel that stores activations) equals the oracle's round-to-
    nearest-even, bit for bit, on every non-NaN input."""
    x = _rounding_cases()
    src = dev.upload(x)
    dst = dev.alloc(2 * x.size)
    H.check(H.lib().opure_convert_f32(dev.h, int(src), int(dst), afmt, x.size))
    dev.sync()
    got = dev.download(dst, np.uint16, x.shape)
    want = O.f32_to_f16_bits(x) if afmt == H.A_F16 else O.f32_to_bf16_bits(x)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(hex(int(x.view(np.uint32)[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:8]]


def test_branch_free_exp_same_bits(dev):
    """The SwiGLU epilogue's select-based exponential returns the bits of the
    oracle-order exponential on all 2^32 fp32 inputs (NaNs, infinities,
    subnormal results, the 2^127 * 2 overflow step included)."""
    n = C.c_uint64(1)
    H.check(H.lib().opure_debug_exp_check(dev.h, C.byref(n)))
    assert n.value == 0


@pytest.mark.parametrize("wfmt", [H.W_F32, H.W_I8PC, H.W_I4G128])
@pytest.mark.parametrize("layout", [H.LAYOUT_TILED, H.LAYOUT_TILED_SWIGLU])
def test_tile_linear_layout(dev, wfmt, layout):
    rng = np.random.default_rng(11 + wfmt + 3 * layout)
    out, inn = 64, 256
    if wfmt == H.W_F32:
        lin = {"w": rng.standard_normal((out, inn)).astype(np.float32), "out": out, "in": inn}
    elif wfmt == H.W_I8PC:
        lin = {"w": rng.integers(-128, 128, (out, inn), dtype=np.int8),
               "scale": rng.integers(0, 65536, out, dtype=np.uint16), "out": out, "in": inn}
    else:
        lin = {"w": rng.integers(0, 256, (out, inn // 2), dtype=np.uint8),
               "scale": rng.integers(0, 65536, (out, inn // 128), dtype=np.uint16),
               "zero": rng.integers(0, 65536, (out, inn // 128), dtype=np.uint16), "out": out, "in": inn}
    desc, keep = dev_linear(dev, lin)
    tiled, bufs = dev.tile(wfmt, desc, layout)
    dev.sync()
    assert tiled.layout == layout and tiled.out == out and tiled.in_ == inn
    want_w, want_s = np_tiled(wfmt, lin, layout)
    got_w = dev.download(bufs[0], np.uint8, want_w.shape)
    assert np.array_equal(got_w, want_w)
    if want_s is not None:
        got_s = dev.download(bufs[1], want_s.dtype, want_s.shape)
        assert np.array_equal(got_s, want_s)


def run_gemv(dev, wfmt, lin_desc, x_bits, M, xfmt, yfmt, epi, y_init=None):
    out = lin_desc.out // 2 if epi == H.EPI_SWIGLU else lin_desc.out
    eb = 4 if yfmt == H.A_F32 else 2
    xb = dev.upload(x_bits[:M])
    yb = dev.alloc(M * out * eb)
    if y_init is not None:
        dev.write(yb, y_init[:M])
    H.gemv(dev, wfmt, lin_desc, xb, yb, M, xfmt, yfmt, epi)
    dev.sync()
    y = dev.download(yb, np.float32 if yfmt == H.A_F32 else np.uint16, (M, out))
    xb.free()
    yb.free()
    return y


GEMV_CASES = [
    # wfmt, afmt, out, in
    (H.W_F32, H.A_F32, 960, 576),
    (H.W_F32, H.A_F32, 576, 1536),
    (H.W_F32, H.A_F32, 4096, 576),
    (H.W_I8PC, H.A_F16, 3072, 2048),
    (H.W_I8PC, H.A_F16, 2048, 8192),
    (H.W_I8PC, H.A_F16, 8192, 2048),
    (H.W_I4G128, H.A_F16, 1024, 4096),
    (H.W_I4G128, H.A_BF16, 6144, 4096),
    (H.W_I4G128, H.A_BF16, 4096, 14336),
    (H.W_I8PC, H.A_F16, 128256, 2048),       # the 1B LM head
    (H.W_I8PC, H.A_F16, 16384, 8192),        # 1024 tiles whose X fits in LDS below 16 rows only
]


def _ids(c):
    return f"w{c[0]}-a{c[1]}-{c[2]}x{c[3]}"


@pytest.mark.parametrize("case", GEMV_CASES, ids=[_ids(c) for c in GEMV_CASES])
def test_gemv_store_residual_matches_oracle(dev, case):
    wfmt, afmt, out, inn = case
    say("gemv", _ids(case))
    rng = np.random.default_rng(out * 7 + inn)
    lin = O.make_linear(rng, out, inn, wfmt)
    desc, keep = dev_linear(dev, lin)
    x_bits, x_f = to_act(rng.standard_normal((16, inn)), afmt)
    ref = O.gemv(lin, wfmt, x_f)
    absref = np.abs(x_f).astype(np.float64) @ np.abs(O.dequant(lin, wfmt)).T
    slack = 4.0 if (wfmt == H.W_I4G128 and afmt == H.A_BF16) else 1.0
    y16 = run_gemv(dev, wfmt, desc, x_bits, 16, afmt, H.A_F32, H.EPI_STORE)
    err = np.abs(y16 - ref)
    assert np.all(err <= 1e-5 * slack * absref + 1e-6), (err.max(), (err / (absref + 1e-9)).max())
    # independent of M, bit for bit; where X does not fit in LDS, M <= 8 also
    # takes the paired X loads and M = 16 the plain ones
    for M in (1, 6, 8):
        yM = run_gemv(dev, wfmt, desc, x_bits, M, afmt, H.A_F32, H.EPI_STORE)
        assert np.array_equal(yM, y16[:M])
    again = run_gemv(dev, wfmt, desc, x_bits, 16, afmt, H.A_F32, H.EPI_STORE)
    assert np.array_equal(again, y16)                        # deterministic
    y0 = rng.standard_normal((16, out)).astype(np.float32)
    yr = run_gemv(dev, wfmt, desc, x_bits, 5, afmt, H.A_F32, H.EPI_RESIDUAL, y_init=y0)
    assert np.array_equal(yr, (y0[:5] + y16[:5]).astype(np.float32))
    for b in keep:
        if b:
            b.free()


WIDE_CASES = [
    # wfmt, afmt, out, in: one K split (many tiles) and several (few tiles, long K)
    (H.W_I8PC, H.A_F16, 16384, 2048),
    (H.W_I8PC, H.A_F16, 3072, 2048),
    (H.W_I8PC, H.A_F16, 2048, 8192),
    (H.W_I4G128, H.A_BF16, 6144, 4096),
    (H.W_I4G128, H.A_F16, 1024, 4096),
    (H.W_I4G128, H.A_BF16, 4096, 14336),
    (H.W_I8PC, H.A_F16, 128256, 2048),       # the 1B LM head over a batch of 32 x 7 rows
]


@pytest.mark.parametrize("case", WIDE_CASES, ids=[_ids(c) for c in WIDE_CASES])
def test_gemv_wide_matches_reference(dev, case):
    """More than 16 rows (a batch of sequences): the thin-GEMM path against
    the dequantised product in float64; each row is independent of how many
    rows share the call (bit for bit), runs are deterministic, and the
    residual epilogue adds in fp32."""
    wfmt, afmt, out, inn = case
    M = 224
    say("gemv wide", _ids(case), "M", M)
    rng = np.random.default_rng(out * 3 + inn)
    lin = O.make_linear(rng, out, inn, wfmt)
    desc, keep = dev_linear(dev, lin)
    x_bits, x_f = to_act(rng.standard_normal((M, inn)), afmt)
    wd = O.dequant(lin, wfmt).astype(np.float64)
    ref = x_f.astype(np.float64) @ wd.T
    absref = np.abs(x_f).astype(np.float64) @ np.abs(wd).T
    slack = 4.0 if (wfmt == H.W_I4G128 and afmt == H.A_BF16) else 1.0
    y = run_gemv(dev, wfmt, desc, x_bits, M, afmt, H.A_F32, H.EPI_STORE)
    err = np.abs(y - ref)
    assert np.all(err <= 1e-5 * slack * absref + 1e-6), (err.max(), (err / (absref + 1e-9)).max())
    y40 = run_gemv(dev, wfmt, desc, x_bits, 40, afmt, H.A_F32, H.EPI_STORE)
    assert np.array_equal(y40, y[:40])
    assert np.array_equal(run_gemv(dev, wfmt, desc, x_bits, M, afmt, H.A_F32, H.EPI_STORE), y)
    y0 = rng.standard_normal((M, out)).astype(np.float32)
    yr = run_gemv(dev, wfmt, desc, x_bits, 100, afmt, H.A_F32, H.EPI_RESIDUAL, y_init=y0)
    assert np.array_equal(yr, (y0[:100] + y[:100]).astype(np.float32))
    for b in keep:
        if b:
            b.free()


def test_gemv_wide_swiglu(dev):
    wfmt, afmt, out, inn, M = H.W_I8PC, H.A_F16, 16384, 2048, 100
    rng = np.random.default_rng(77)
    lin = O.make_linear(rng, out, inn, wfmt)
    desc, keep = dev_linear(dev, lin)
    x_bits, x_f = to_act(rng.standard_normal((M, inn)), afmt)
    gu = (x_f.astype(np.float64) @ O.dequant(lin, wfmt).astype(np.float64).T).astype(np.float32)
    F = out // 2
    g, u = gu[:, :F].copy(), gu[:, F:].copy()
    h = np.zeros_like(g)
    O.lib().orc_swiglu(g.ctypes.data, u.ctypes.data, h.ctypes.data, g.size)
    y = from_act(run_gemv(dev, wfmt, desc, x_bits, M, afmt, afmt, H.EPI_SWIGLU), afmt)
    np.testing.assert_allclose(y, h, rtol=2e-3, atol=1e-4 * max(1.0, np.abs(h).max()))
    for b in keep:
        if b:
            b.free()


@pytest.mark.parametrize("case", [(H.W_F32, H.A_F32, 3072, 576), (H.W_I8PC, H.A_F16, 16384, 2048),
                                  (H.W_I4G128, H.A_BF16, 2048, 4096)], ids=["f32", "i8", "i4bf16"])
def test_gemv_swiglu_matches_oracle(dev, case):
    wfmt, afmt, out, inn = case
    say("gemv swiglu", case)
    rng = np.random.default_rng(out + inn)
    lin = O.make_linear(rng, out, inn, wfmt)
    desc, keep = dev_linear(dev, lin)
    x_bits, x_f = to_act(rng.standard_normal((16, inn)), afmt)
    gu = O.gemv(lin, wfmt, x_f)
    F = out // 2
    g, u = gu[:, :F].copy(), gu[:, F:].copy()
    h = np.zeros_like(g)
    O.lib().orc_swiglu(g.ctypes.data, u.ctypes.data, h.ctypes.data, g.size)
    y = from_act(run_gemv(dev, wfmt, desc, x_bits, 16, afmt, afmt, H.EPI_SWIGLU), afmt)
    tol = 1e-4 if afmt == H.A_F32 else (2e-3 if afmt == H.A_F16 else 1.6e-2)
    np.testing.assert_allclose(y, h, rtol=tol, atol=1e-4 * max(1.0, np.abs(h).max()))
    for b in keep:
        if b:
            b.free()


VALU_CASES = [(H.W_I8PC, H.A_F16, 3072, 2048), (H.W_I8PC, H.A_F16, 2048, 8192), (H.W_I8PC, H.A_F16, 16384, 2048),
              (H.W_I8PC, H.A_F16, 128256, 2048), (H.W_F32, H.A_F32, 960, 576), (H.W_F32, H.A_F32, 576, 1536),
              (H.W_F32, H.A_F32, 3072, 576), (H.W_I4G128, H.A_BF16, 6144, 4096), (H.W_I4G128, H.A_BF16, 4096, 14336),
              (H.W_I4G128, H.A_F16, 4096, 4096)]
VALU_IDS = [f"{['f32', 'i8', 'i4'][w]}{['', '-f16', '-bf16'][a]}-{o}x{i}" for w, a, o, i in VALU_CASES]


@pytest.mark.parametrize("case", VALU_CASES, ids=VALU_IDS)
def test_gemv_valu_engine_matches_oracle(dev, case):
    """The vector-ALU engine (M <= 8: fp32, int8, uint4 weights) against the
    oracle, to the matrix-core path's bound, for every epilogue it takes."""
    wfmt, afmt, out, inn = case
    say("gemv valu", VALU_IDS[VALU_CASES.index(case)])
    rng = np.random.default_rng(out * 3 + inn + wfmt)
    lin = O.make_linear(rng, out, inn, wfmt)
    desc, keep = dev_linear(dev, lin)
    x_bits, x_f = to_act(rng.standard_normal((16, inn)), afmt)
    ref = O.gemv(lin, wfmt, x_f)
    absref = np.abs(x_f).astype(np.float64) @ np.abs(O.dequant(lin, wfmt)).T
    rel = 1e-5 if wfmt != H.W_I4G128 else 2e-5      # uint4: the group correction subtracts (OFF + MUL z) * sum x
    H.check(H.lib().opure_debug_set_gemv_engine(dev.h, H.GEMV_VALU))
    try:
        for M in (1, 5, 6, 8):
            y = run_gemv(dev, wfmt, desc, x_bits, M, afmt, H.A_F32, H.EPI_STORE)
            err = np.abs(y - ref[:M])
            assert np.all(err <= rel * absref[:M] + 1e-6), (M, err.max())
        y0 = rng.standard_normal((8, out)).astype(np.float32)
        yv = run_gemv(dev, wfmt, desc, x_bits, 6, afmt, H.A_F32, H.EPI_STORE)
        yr = run_gemv(dev, wfmt, desc, x_bits, 6, afmt, H.A_F32, H.EPI_RESIDUAL, y_init=y0)
        assert np.array_equal(yr, (y0[:6] + yv).astype(np.float32))
        if out <= 16384 and out % 32 == 0:
            F = out // 2
            g, u = ref[:6, :F].copy(), ref[:6, F:].copy()
            h = np.zeros_like(g)
            O.lib().orc_swiglu(g.ctypes.data, u.ctypes.data, h.ctypes.data, g.size)
            ys = from_act(run_gemv(dev, wfmt, desc, x_bits, 6, afmt, afmt, H.EPI_SWIGLU), afmt)
            tol = 1e-4 if afmt == H.A_F32 else (2e-3 if afmt == H.A_F16 else 1.6e-2)
            np.testing.assert_allclose(ys, h, rtol=tol, atol=1e-4 * max(1.0, np.abs(h).max()))
        # rows past 8 fall back to the matrix cores
        y16 = run_gemv(dev, wfmt, desc, x_bits, 16, afmt, H.A_F32, H.EPI_STORE)
        assert np.all(np.abs(y16 - ref) <= rel * absref + 1e-6)
    finally:
        H.check(H.lib().opure_debug_set_gemv_engine(dev.h, H.GEMV_MFMA))
    for b in keep:
        if b:
            b.free()


@pytest.mark.parametrize("case", [(H.W_I4G128, H.A_BF16, 28672, 4096), (H.W_I8PC, H.A_F16, 24576, 2048)],
                         ids=["i4bf16-28672x4096", "i8-24576x2048"])
def test_gemv_loader_waves_equal_wave_per_tile(dev, case):
    """6 to 8 tiles a CU run the loader-wave kernel where its LDS rings fit
    beside X: uint4 4096-long rows up to 8 rows (16 rows: the wave-per-tile
    kernel), int8 2048-long rows with 3 slots a wave at 8 rows and 2 at 16.
    Same tiles, blocks and order of sums in every case: the rows agree bit for
    bit, and with the oracle."""
    wfmt, afmt, out, inn = case
    say("gemv loader waves", case)
    rng = np.random.default_rng(out - inn)
    lin = O.make_linear(rng, out, inn, wfmt)
    desc, keep = dev_linear(dev, lin)
    x_bits, x_f = to_act(rng.standard_normal((16, inn)), afmt)
    y16 = run_gemv(dev, wfmt, desc, x_bits, 16, afmt, H.A_F32, H.EPI_STORE)
    for M in (1, 8):
        yM = run_gemv(dev, wfmt, desc, x_bits, M, afmt, H.A_F32, H.EPI_STORE)
        assert np.array_equal(yM, y16[:M]), M
    ref = O.gemv(lin, wfmt, x_f[:2])
    absref = np.abs(x_f[:2]).astype(np.float64) @ np.abs(O.dequant(lin, wfmt)).T
    slack = 4.0 if (wfmt == H.W_I4G128 and afmt == H.A_BF16) else 1.0
    assert np.all(np.abs(y16[:2] - ref) <= 1e-5 * slack * absref + 1e-6)
    for b in keep:
        if b:
            b.free()


@pytest.mark.parametrize("case", [(H.W_I8PC, H.A_F16, 16384, 2048), (H.W_I4G128, H.A_BF16, 16384, 4096)],
                         ids=["i8-16384x2048", "i4bf16-16384x4096"])
def test_gemv_two_waves_a_tile(dev, case):
    """1024 tiles (four a CU): two waves share each tile, half of its blocks
    each, and add the halves at the end.  The rows agree bit for bit at any
    row count, and with the oracle."""
    wfmt, afmt, out, inn = case
    say("gemv two waves a tile", case)
    rng = np.random.default_rng(out + 3 * inn)
    lin = O.make_linear(rng, out, inn, wfmt)
    desc, keep = dev_linear(dev, lin)
    x_bits, x_f = to_act(rng.standard_normal((16, inn)), afmt)
    y16 = run_gemv(dev, wfmt, desc, x_bits, 16, afmt, H.A_F32, H.EPI_STORE)
    for M in (1, 6, 8):
        yM = run_gemv(dev, wfmt, desc, x_bits, M, afmt, H.A_F32, H.EPI_STORE)
        assert np.array_equal(yM, y16[:M]), M
    ref = O.gemv(lin, wfmt, x_f[:3])
    absref = np.abs(x_f[:3]).astype(np.float64) @ np.abs(O.dequant(lin, wfmt)).T
    slack = 4.0 if (wfmt == H.W_I4G128 and afmt == H.A_BF16) else 1.0
    assert np.all(np.abs(y16[:3] - ref) <= 1e-5 * slack * absref + 1e-6)
    for b in keep:
        if b:
            b.free()


def test_gemv_known_answer_fixtures(dev):
    g = np.load(os.path.join(GOLD, "gemv_f32.npz"))
    lin = {"w": g["W"], "out": 64, "in": 128}
    desc, keep = dev_linear(dev, lin)
    y = run_gemv(dev, H.W_F32, desc, g["X"][None, :], 1, H.A_F32, H.A_F32, H.EPI_STORE)[0]
    rms = np.sqrt(np.mean((y.astype(np.float64) - g["ref"]) ** 2))
    assert rms <= 1e-5 * np.abs(g["ref"]).max()
    q = np.load(os.path.join(GOLD, "gemv_quant.npz"))
    s16 = np.full(64, np.float16(q["sW"][0])).view(np.uint16)
    lin = {"w": q["q"], "scale": s16, "out": 64, "in": 128}
    desc, keep2 = dev_linear(dev, lin)
    xb, xf = to_act(q["X"][None, :], H.A_F16)
    y = run_gemv(dev, H.W_I8PC, desc, xb, 1, H.A_F16, H.A_F32, H.EPI_STORE)[0]
    want = O.gemv(lin, H.W_I8PC, xf)[0]     # activations enter as fp16 on this path
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-5)


def test_gemv_rejects_bad_shapes(dev):
    # 24 rows are not a whole number of 16-row tiles: tiling refuses them
    lin = {"w": np.zeros((24, 128), np.float32), "out": 24, "in": 128}
    desc, keep = dev_linear(dev, lin)
    x = dev.upload(np.zeros((17, 128), np.float32))
    y = dev.alloc(17 * 32 * 4)
    with pytest.raises(H.OpureError) as e:
        H.gemv(dev, H.W_F32, desc, x, y, 1, H.A_F32, H.A_F32, H.EPI_STORE)
    assert e.value.code == H.E_INVALID
    lin = {"w": np.zeros((32, 128), np.float32), "out": 32, "in": 128}
    desc, keep = dev_linear(dev, lin)
    # more than 16 rows run as a thin GEMM, built for quantised weights only
    with pytest.raises(H.OpureError) as e:
        H.gemv(dev, H.W_F32, desc, x, y, 17, H.A_F32, H.A_F32, H.EPI_STORE)
    assert e.value.code == H.E_UNSUPPORTED
    with pytest.raises(H.OpureError) as e:
        H.gemv(dev, H.W_F32, desc, x, y, 257, H.A_F32, H.A_F32, H.EPI_STORE)
    assert e.value.code == H.E_CAPACITY
    with pytest.raises(H.OpureError) as e:
        H.gemv(dev, H.W_I8PC, desc, x, y, 1, H.A_F32, H.A_F32, H.EPI_STORE)
    assert e.value.code in (H.E_UNSUPPORTED, H.E_INVALID)
    # a row-major linear handed straight to the kernel entry point is refused
    tiled, bufs = dev.tile(H.W_F32, desc)
    a = H.GemvArgs(desc, int(x), int(y), 1, H.A_F32, H.A_F32, H.EPI_STORE)
    assert H.lib().opure_gemv_batched_f32(dev.h, C.byref(a)) == H.E_INVALID
    a = H.GemvArgs(tiled, int(x), int(y), 1, H.A_F32, H.A_F32, H.EPI_SWIGLU)
    assert H.lib().opure_gemv_batched_f32(dev.h, C.byref(a)) == H.E_INVALID    # SwiGLU needs the paired layout


# ---------------------------------------------------------------------------
def attn_model(n_heads, n_kv, hd, afmt, scale=1.0, n_layers=1):
    m = H.Model()
    m.n_layers, m.n_heads, m.n_kv_heads, m.head_dim, m.afmt, m.attn_scale = n_layers, n_heads, n_kv, hd, afmt, scale
    return m


def run_attn(dev, m, pool_bits, pt, seq_len, R, q_bits, layer=0, max_ctx=None):
    B = pt.shape[0]
    pb = dev.upload(pool_bits)
    ptb = dev.upload(pt.astype(np.int32))
    sl = dev.upload(np.asarray(seq_len, dtype=np.int32))
    qb = dev.upload(q_bits)
    ob = dev.alloc(q_bits.nbytes)
    kv = H.KV(int(pb), pool_bits.shape[1], 16, int(ptb), pt.shape[1])
    a = H.AttnArgs(C.pointer(m), C.pointer(kv), layer, B, R, int(sl), int(max(seq_len)) + R if max_ctx is None else max_ctx,
                   int(qb), int(ob))
    H.check(H.lib().opure_attn_decode_paged(dev.h, C.byref(a)))
    dev.sync()
    out = dev.download(ob, q_bits.dtype, q_bits.shape)
    for b in (pb, ptb, sl, qb, ob):
        b.free()
    return out


@pytest.mark.parametrize("hd", [32, 64, 96, 128, 160, 192, 224, 256])
def test_attention_known_answers(dev, hd):
    g = np.load(os.path.join(GOLD, f"attention_hd{hd}.npz"))
    pool = np.zeros((1, 1, 2, 2, 16, hd), np.float32)
    Kp, Vp = O.kv_planes(pool)
    Kp[0, 0, :, :7] = g["K"]
    Vp[0, 0, :, :7] = g["V"]
    out = run_attn(dev, attn_model(4, 2, hd, H.A_F32), pool, np.zeros((1, 1)), [6], 1,
                   np.ascontiguousarray(g["Q"].reshape(1, -1)))
    rms = np.sqrt(np.mean((out.ravel().astype(np.float64) - g["ref"].ravel()) ** 2))
    assert rms <= 1e-5 * np.abs(g["ref"]).max()


ATTN_CASES = [
    # afmt, head_dim, rows, contexts (several 128/256-token chunks at head_dim 64/128)
    (H.A_F32, 64, 5, [131, 37]),
    (H.A_F16, 64, 5, [131, 37]),
    (H.A_BF16, 64, 5, [131, 37]),
    (H.A_F16, 64, 6, [2100, 700]),           # 17 and 6 chunks: groups of 4 merged by the combine
    (H.A_BF16, 64, 6, [2100, 700]),
    (H.A_F16, 128, 8, [1100, 531]),
    (H.A_BF16, 128, 8, [1100, 531]),
]


@pytest.mark.parametrize("case", ATTN_CASES,
                         ids=[f"{['f32', 'f16', 'bf16'][c[0]]}-hd{c[1]}-r{c[2]}" for c in ATTN_CASES])
def test_attention_paged_matches_oracle(dev, case):
    afmt, hd, R, ctx = case
    say("attention", case)
    rng = np.random.default_rng(31 + afmt + hd)
    nh, nkv, B, ps = 8, 2, 2, 16
    mp = [(c + R + ps - 1) // ps for c in ctx]
    n_pages = sum(mp) + 4
    mcfg = dict(n_layers=2, hidden=64, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=64, vocab=64,
                wfmt=O.W_F32, afmt=afmt)
    hm = O.HostModel(**mcfg, attn_scale=hd ** -0.5, max_pos=max(ctx) + 64, seed=1)
    kv = O.HostKV(hm, n_pages=n_pages, batch=B, max_pages_per_seq=max(mp))
    kv.fill_random(rng, 1.0)
    perm = rng.permutation(n_pages)
    kv.page_table[0, :mp[0]] = perm[:mp[0]]
    kv.page_table[1, :mp[1]] = perm[mp[0]:mp[0] + mp[1]]
    q_bits, q_f = to_act(rng.standard_normal((B * R, nh * hd)) * 1.5, afmt)
    want = np.zeros_like(q_f)
    kv._mk()
    O.set_threads(16)
    try:
        for b in range(B):
            qb = np.ascontiguousarray(q_f[b * R:(b + 1) * R])
            ob = np.zeros_like(qb)
            O.lib().orc_attention_paged(C.byref(hm.desc), C.byref(kv.desc), 1, b, ctx[b], R, qb.ctypes.data,
                                        ob.ctypes.data)
            want[b * R:(b + 1) * R] = ob
    finally:
        O.set_threads(1)
    m = attn_model(nh, nkv, hd, afmt, hd ** -0.5, n_layers=2)
    got = run_attn(dev, m, kv.pool, kv.page_table, ctx, R, q_bits, layer=1)
    got_f = from_act(got, afmt)
    if afmt == H.A_F32:
        np.testing.assert_allclose(got_f, want, rtol=2e-5, atol=2e-5)
    else:
        # within one storage ulp of the oracle's rounded output
        want_r = to_act(want, afmt)[1]
        ulp = 2.0 ** -10 if afmt == H.A_F16 else 2.0 ** -7
        assert (np.abs(got_f - want_r) <= ulp * np.abs(want_r) + 1e-6).all()
        say("storage roundings that differ from the oracle:", int((got_f != want_r).sum()), "of", got_f.size)
    # row j of an R-row call equals a 1-row call at position ctx+j, bit for bit
    for j in range(R):
        one = run_attn(dev, m, kv.pool, kv.page_table[:1], [ctx[0] + j], 1, q_bits[j:j + 1], layer=1)
        assert np.array_equal(one[0], got[j])


# fp32 launches over few chunks of 64 tokens: head_dim, query heads, KV heads,
# rows, contexts (rows ending on either side of chunk boundaries)
FAST_ALL_CASES = [
    (64, 9, 3, 5, [0, 1, 58, 59, 60, 63, 64, 122, 187, 251]),     # 4 chunks
    (64, 8, 2, 3, [5, 130, 191, 255, 256, 300, 447, 509]),        # 8 chunks, an odd row count
    (128, 8, 2, 4, [3, 60, 61, 125, 190, 252]),
]


@pytest.mark.parametrize("hd,nh,nkv,R,ctx", FAST_ALL_CASES, ids=["hd64-4", "hd64-8", "hd128"])
def test_attention_one_workgroup_merge_same_bits(dev, hd, nh, nkv, R, ctx):
    """fp32 over a short context merges a row's chunks inside one workgroup
    (head_dim 64, up to 8 chunks: a workgroup a pair of query rows, a wave a
    chunk; head_dim 128, up to 4 chunks: a workgroup a KV head, the chunks in
    turn); a launch over more chunks (max_ctx 1024) writes one partial a chunk
    and merges them in the combine launch.  Every row has the same bits either
    way (a missing page's NaN included), and stays within fp32 tolerance of
    the oracle."""
    say("attention one-workgroup merge", hd, nh, nkv, R, ctx)
    rng = np.random.default_rng(hd + R)
    B, ps, wide = len(ctx), 16, 64
    mp = [(c + R + ps - 1) // ps for c in ctx]
    n_pages = sum(mp) + 4
    hm = O.HostModel(n_layers=1, hidden=64, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=64, vocab=64,
                     wfmt=O.W_F32, afmt=H.A_F32, attn_scale=hd ** -0.5, max_pos=1100, seed=1)
    kv = O.HostKV(hm, n_pages=n_pages, batch=B, max_pages_per_seq=wide)
    kv.fill_random(rng, 1.0)
    kv.page_table[:] = -1
    perm = rng.permutation(n_pages)
    o = 0
    for b in range(B):
        kv.page_table[b, :mp[b]] = perm[o:o + mp[b]]
        o += mp[b]
    q_bits, q_f = to_act(rng.standard_normal((B * R, nh * hd)) * 1.5, H.A_F32)
    m = attn_model(nh, nkv, hd, H.A_F32, hd ** -0.5)
    assert max(ctx) + R <= (512 if hd == 64 else 256)
    one = run_attn(dev, m, kv.pool, kv.page_table, ctx, R, q_bits)
    many = run_attn(dev, m, kv.pool, kv.page_table, ctx, R, q_bits, max_ctx=1024)
    assert np.array_equal(one.view(np.uint32), many.view(np.uint32))
    kv._mk()
    O.set_threads(16)
    try:
        for b in range(B):
            qb = np.ascontiguousarray(q_f[b * R:(b + 1) * R])
            ob = np.zeros_like(qb)
            O.lib().orc_attention_paged(C.byref(hm.desc), C.byref(kv.desc), 0, b, ctx[b], R, qb.ctypes.data,
                                        ob.ctypes.data)
            np.testing.assert_allclose(from_act(one[b * R:(b + 1) * R], H.A_F32), ob, rtol=2e-5, atol=2e-5)
    finally:
        O.set_threads(1)
    # a missing page inside sequence 3's context (tokens 16..31): its rows read
    # NaN, the others keep their bits, both launches alike
    pt = kv.page_table.copy()
    pt[3, 1] = -1
    one_m = run_attn(dev, m, kv.pool, pt, ctx, R, q_bits)
    many_m = run_attn(dev, m, kv.pool, pt, ctx, R, q_bits, max_ctx=1024)
    assert np.array_equal(one_m.view(np.uint32), many_m.view(np.uint32))
    assert np.isnan(one_m[3 * R:4 * R]).all()
    keep = np.ones(B * R, bool)
    keep[3 * R:4 * R] = False
    assert np.array_equal(one_m[keep].view(np.uint32), one[keep].view(np.uint32))


# ---------------------------------------------------------------------------
def run_accept(dev, fn, t, q, drafts, temperature=1.0, seed=0, pos_base=None, want_dist=False):
    B, K1, V = t.shape
    tb = dev.upload(t)
    qb = dev.upload(q) if q is not None else None
    db = dev.upload(np.ascontiguousarray(drafts, dtype=np.int32))
    pbb = dev.upload(np.asarray(pos_base, dtype=np.uint32)) if pos_base is not None else None
    ot = dev.alloc(B * K1 * 4)
    ac = dev.alloc(B * 4)
    di = dev.alloc(B * V * 4) if want_dist else None
    a = H.AcceptArgs(B, K1 - 1, V, int(tb), int(qb) if qb else None, int(db), K1 - 1, temperature, seed,
                     int(pbb) if pbb else None, int(ot), int(ac), int(di) if di else None)
    H.check(fn(dev.h, C.byref(a)))
    dev.sync()
    res = (dev.download(ot, np.int32, (B, K1)), dev.download(ac, np.int32, (B,)),
           dev.download(di, np.float32, (B, V)) if di else None)
    for b in (tb, qb, db, pbb, ot, ac, di):
        if b:
            b.free()
    return res


@pytest.mark.parametrize("V", [1000, 70000], ids=["registers", "sliced"])
def test_accept_rejection_no_drafts(dev, V):
    """k = 0: nothing to test, the token is drawn from the target row alone,
    whose statistics come from one phase (one workgroup a row, or its
    slices); the ids equal the oracle's."""
    say("rejection without drafts", V)
    rng = np.random.default_rng(V)
    B = 3
    t = (rng.standard_normal((B, 1, V)) * 3).astype(np.float32)
    w_out, w_acc, _ = O.accept_rejection(t, np.zeros((B, 0, V), np.float32), np.zeros((B, 0), np.int32), 0.9, 77)
    tb, db = dev.upload(t), dev.upload(np.zeros(1, np.int32))
    ot, ac = dev.alloc(B * 4), dev.alloc(B * 4)
    a = H.AcceptArgs(B, 0, V, int(tb), None, int(db), 0, 0.9, 77, None, int(ot), int(ac), None)
    H.check(H.lib().opure_accept_rejection(dev.h, C.byref(a)))
    dev.sync()
    out, acc = dev.download(ot, np.int32, (B, 1)), dev.download(ac, np.int32, (B,))
    for b in (tb, db, ot, ac):
        b.free()
    assert np.array_equal(acc, w_acc) and (acc == 0).all()
    assert np.array_equal(out, w_out)


def test_accept_greedy_bit_exact(dev):
    rng = np.random.default_rng(41)
    B, K, V = 6, 5, 50000
    t = rng.standard_normal((B, K + 1, V)).astype(np.float32)
    am = t.argmax(-1)
    drafts = am[:, :K].astype(np.int32).copy()
    for b in range(B):
        if b % 3:
            drafts[b, b % K] = (drafts[b, b % K] + 1) % V
    t[0, 0, 777] = t[0, 0].max()            # exact tie: lowest index must win
    t[1, 2, 5] = np.nan                      # NaN counts as -inf
    out, acc, _ = run_accept(dev, H.lib().opure_accept_greedy, t, None, drafts)
    w_out, w_acc = O.accept_greedy(t, drafts)
    assert np.array_equal(acc, w_acc) and np.array_equal(out, w_out)


def test_attention_folded_grid_same_bits(dev):
    """A batch big enough that the launch folds two chunks into a workgroup
    (head_dim 64, 16 sequences of up to 9000 tokens) gives every sequence
    the bits of that sequence scored alone (one chunk a workgroup)."""
    say("attention folded grid")
    rng = np.random.default_rng(5)
    nh, nkv, hd, R, ps = 8, 2, 64, 3, 16
    ctx = [int(c) for c in rng.integers(100, 9000, size=16)]
    B = len(ctx)
    mp = [(c + R + ps - 1) // ps for c in ctx]
    n_pages = sum(mp) + 4
    hm = O.HostModel(n_layers=1, hidden=64, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=64, vocab=64,
                     wfmt=O.W_F32, afmt=H.A_F16, attn_scale=hd ** -0.5, max_pos=max(ctx) + 64, seed=1)
    kv = O.HostKV(hm, n_pages=n_pages, batch=B, max_pages_per_seq=max(mp))
    kv.fill_random(rng, 1.0)
    perm = rng.permutation(n_pages)
    o = 0
    for b in range(B):
        kv.page_table[b, :mp[b]] = perm[o:o + mp[b]]
        o += mp[b]
    q_bits, _ = to_act(rng.standard_normal((B * R, nh * hd)) * 1.5, H.A_F16)
    m = attn_model(nh, nkv, hd, H.A_F16, hd ** -0.5)
    got = run_attn(dev, m, kv.pool, kv.page_table, ctx, R, q_bits)
    assert np.isfinite(from_act(got, H.A_F16)).all()
    for b in (0, 5, 11, 15):
        one = run_attn(dev, m, kv.pool, kv.page_table[b:b + 1], [ctx[b]], R, q_bits[b * R:(b + 1) * R])
        assert np.array_equal(one, got[b * R:(b + 1) * R]), b


# contexts whose rows end on either side of a 128-token chunk and a 512-token
# group boundary (rows 0..2 of a sequence see different numbers of a group's chunks)
FOLD_EDGES = [126, 127, 128, 510, 511, 512, 1021, 1022, 1023, 2045, 2046, 2047, 4094, 4095, 8189, 8190]


@pytest.mark.parametrize("afmt,case", [(H.A_F16, "edges"), (H.A_BF16, "edges"), (H.A_BF16, "random")])
def test_attention_folded_groups_same_bits(dev, afmt, case):
    """The folded launch (head_dim 64, a grid of many sequences) merges each
    group of 4 chunks (512 tokens) inside its workgroup and writes one partial
    a group; a launch of one sequence writes one partial a chunk and its
    combine merges the same groups.  Every sequence gets the same bits either
    way, also where a row's last chunk is inside a group or the first of one,
    and the rows stay within one storage ulp of the oracle."""
    say("attention folded groups", afmt, case)
    rng = np.random.default_rng(7 + afmt)
    nh, nkv, hd, R, ps = 8, 2, 64, 3, 16
    ctx = FOLD_EDGES if case == "edges" else [int(c) for c in rng.integers(100, 9000, size=16)]
    B = len(ctx)
    assert nkv * -(-(max(ctx) + R) // 128) * B > 8 * 256        # the launch folds
    mp = [(c + R + ps - 1) // ps for c in ctx]
    n_pages = sum(mp) + 4
    hm = O.HostModel(n_layers=1, hidden=64, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=64, vocab=64,
                     wfmt=O.W_F32, afmt=afmt, attn_scale=hd ** -0.5, max_pos=max(ctx) + 64, seed=1)
    kv = O.HostKV(hm, n_pages=n_pages, batch=B, max_pages_per_seq=max(mp))
    kv.fill_random(rng, 1.0)
    perm = rng.permutation(n_pages)
    o = 0
    for b in range(B):
        kv.page_table[b, :mp[b]] = perm[o:o + mp[b]]
        o += mp[b]
    q_bits, q_f = to_act(rng.standard_normal((B * R, nh * hd)) * 1.5, afmt)
    m = attn_model(nh, nkv, hd, afmt, hd ** -0.5)
    got = run_attn(dev, m, kv.pool, kv.page_table, ctx, R, q_bits)
    for b in range(B):
        one = run_attn(dev, m, kv.pool, kv.page_table[b:b + 1], [ctx[b]], R, q_bits[b * R:(b + 1) * R])
        assert np.array_equal(one, got[b * R:(b + 1) * R]), (b, ctx[b])
    kv._mk()
    O.set_threads(16)
    try:
        got_f = from_act(got, afmt)
        ulp = 2.0 ** -10 if afmt == H.A_F16 else 2.0 ** -7
        for b in (0, 5, 10, 15):
            qb = np.ascontiguousarray(q_f[b * R:(b + 1) * R])
            ob = np.zeros_like(qb)
            O.lib().orc_attention_paged(C.byref(hm.desc), C.byref(kv.desc), 0, b, ctx[b], R, qb.ctypes.data,
                                        ob.ctypes.data)
            want_r = to_act(ob, afmt)[1]
            gb = got_f[b * R:(b + 1) * R]
            assert (np.abs(gb - want_r) <= ulp * np.abs(want_r) + 1e-6).all(), (b, ctx[b])
    finally:
        O.set_threads(1)


def test_attention_folded_grid_missing_page(dev):
    """The folded kernel loads every K/V operand unconditionally (a lane whose
    page entry is missing reads page 0) and applies the fill when the operand is
    used: a sequence with a -1 entry inside its context reads NaN there, as the
    one-chunk-a-workgroup kernel does, and its neighbours keep their bits."""
    say("attention folded grid, missing page")
    rng = np.random.default_rng(6)
    nh, nkv, hd, R, ps = 8, 2, 64, 3, 16
    ctx = [int(c) for c in rng.integers(4000, 9000, size=15)] + [8999]   # 71 chunks: 2 x 71 x 16 > 8 x 256
    B = len(ctx)
    mp = [(c + R + ps - 1) // ps for c in ctx]
    n_pages = sum(mp) + 4
    hm = O.HostModel(n_layers=1, hidden=64, n_heads=nh, n_kv_heads=nkv, head_dim=hd, ffn=64, vocab=64,
                     wfmt=O.W_F32, afmt=H.A_F16, attn_scale=hd ** -0.5, max_pos=max(ctx) + 64, seed=1)
    kv = O.HostKV(hm, n_pages=n_pages, batch=B, max_pages_per_seq=max(mp))
    kv.fill_random(rng, 1.0)
    perm = rng.permutation(n_pages)
    o = 0
    for b in range(B):
        kv.page_table[b, :mp[b]] = perm[o:o + mp[b]]
        o += mp[b]
    kv.page_table[5, 3] = -1                          # tokens 48..63 of sequence 5
    q_bits, _ = to_act(rng.standard_normal((B * R, nh * hd)) * 1.5, H.A_F16)
    m = attn_model(nh, nkv, hd, H.A_F16, hd ** -0.5)
    got = run_attn(dev, m, kv.pool, kv.page_table, ctx, R, q_bits)
    vals = from_act(got, H.A_F16).reshape(B, R, -1)
    assert np.isnan(vals[5]).all()
    assert np.isfinite(np.delete(vals, 5, axis=0)).all()
    one = run_attn(dev, m, kv.pool, kv.page_table[5:6], [ctx[5]], R, q_bits[5 * R:6 * R])
    assert np.isnan(from_act(one, H.A_F16)).all()
    for b in (0, 4, 6, 15):
        one = run_attn(dev, m, kv.pool, kv.page_table[b:b + 1], [ctx[b]], R, q_bits[b * R:(b + 1) * R])
        assert np.array_equal(one, got[b * R:(b + 1) * R]), b


# 49152-logit rows fit the one-workgroup-a-row statistics; longer or
# unaligned rows take them from their 4096-logit slices
@pytest.mark.parametrize("B,K,V,tau", [(8, 8, 49152, 1.0), (4, 3, 1000, 0.8), (64, 8, 49152, 1.0),
                                       (8, 5, 128256, 1.0), (6, 4, 50001, 0.8), (5, 1, 65539, 1.0)],
                         ids=["b8k8", "small-t0.8", "c2-full", "sliced-128k", "sliced-odd-t0.8", "sliced-k1"])
def test_accept_rejection_bit_exact(dev, B, K, V, tau):
    say("rejection", B, K, V, tau)
    rng = np.random.default_rng(B * 100 + K)
    t = (rng.standard_normal((B, K + 1, V)) * 3).astype(np.float32)
    q = (rng.standard_normal((B, K, V)) * 3).astype(np.float32)
    # drafts drawn from q on Philox stream 0 (the C2 recipe), one seeded half accepted more often
    q[: B // 2] = t[: B // 2, :K] + (rng.standard_normal((B // 2, K, V)) * 0.3).astype(np.float32)
    pos = np.repeat(np.arange(K)[None], B, 0).ravel()
    seq = np.repeat(np.arange(B)[:, None], K, 1).ravel()
    drafts = O.sample_rows(q.reshape(B * K, V), tau, 2024, pos, seq, 0).reshape(B, K)
    pos_base = rng.integers(0, 4096, size=B)
    out, acc, dist = run_accept(dev, H.lib().opure_accept_rejection, t, q, drafts, tau, 2024, pos_base, True)
    w_out, w_acc, w_dist = O.accept_rejection(t, q, drafts, tau, 2024, pos_base)
    assert np.array_equal(acc, w_acc), (acc, w_acc)
    assert np.array_equal(out, w_out)
    assert np.abs(dist - w_dist).max() <= 1e-6
    say("mean accepted", acc.mean())


REJ_LAUNCH_CASES = [(64, 8, 49152, 1.0), (8, 5, 128256, 0.8), (4, 3, 1000, 0.8), (6, 4, 50001, 0.8), (5, 1, 65539, 1.0)]


@pytest.mark.parametrize("B,K,V,tau", REJ_LAUNCH_CASES, ids=["c2", "sliced-128k", "small", "odd-v", "k1-odd-v"])
def test_accept_rejection_one_launch_same_bits_as_staged(dev, B, K, V, tau):
    """The one-launch rejection step (the slices of a sequence hand each other
    their maxima and sums and wait for each other) against the staged
    launches: ids, accepted lengths and the distribution bit for bit.  Half
    the sequences draft close to the target, so they accept several drafts
    and run several positions' statistics in the one launch."""
    say("rejection one launch vs staged", B, K, V, tau)
    rng = np.random.default_rng(B * 7 + K + V)
    t = (rng.standard_normal((B, K + 1, V)) * 3).astype(np.float32)
    q = (rng.standard_normal((B, K, V)) * 3).astype(np.float32)
    q[: B // 2] = t[: B // 2, :K] + (rng.standard_normal((B // 2, K, V)) * 0.05).astype(np.float32)
    pos = np.repeat(np.arange(K)[None], B, 0).ravel()
    seq = np.repeat(np.arange(B)[:, None], K, 1).ravel()
    drafts = O.sample_rows(q.reshape(B * K, V), tau, 77, pos, seq, 0).reshape(B, K)
    pos_base = rng.integers(0, 4096, size=B)
    L = H.lib()
    got = {}
    try:
        for mode in (H.REJ_STAGED, H.REJ_ONE_LAUNCH):
            H.check(L.opure_debug_set_rejection_launches(dev.h, mode))
            got[mode] = run_accept(dev, L.opure_accept_rejection, t, q, drafts, tau, 77, pos_base, True)
    finally:
        H.check(L.opure_debug_set_rejection_launches(dev.h, H.REJ_ONE_LAUNCH))
    (o1, a1, d1), (o2, a2, d2) = got[H.REJ_STAGED], got[H.REJ_ONE_LAUNCH]
    assert np.array_equal(a1, a2) and np.array_equal(o1, o2)
    assert np.array_equal(d1.view(np.uint32), d2.view(np.uint32))
    say("accepted", a2.tolist()[:16])
    assert a2.max() >= 2 or K < 2                           # some sequence ran several positions


def test_sample_rows_and_philox_bit_exact(dev):
    rng = np.random.default_rng(51)
    rows, V = 37, 32000
    lg = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    pos = rng.integers(0, 1 << 20, rows).astype(np.uint32)
    seq = rng.integers(0, 64, rows).astype(np.uint32)
    lb, pb, sb = dev.upload(lg), dev.upload(pos), dev.upload(seq)
    ob = dev.alloc(rows * 4)
    a = H.SampleArgs(rows, V, int(lb), 0.8, 99, int(pb), int(sb), 0, int(ob))
    H.check(H.lib().opure_sample_rows(dev.h, C.byref(a)))
    dev.sync()
    got = dev.download(ob, np.int32, (rows,))
    assert np.array_equal(got, O.sample_rows(lg, 0.8, 99, pos, seq, 0))
    n = 4096
    pos = rng.integers(0, 1 << 31, n).astype(np.uint32)
    seq = rng.integers(0, 1 << 31, n).astype(np.uint32)
    pb, sb, ob = dev.upload(pos), dev.upload(seq), dev.alloc(n * 4)
    seed = 0xDEADBEEFCAFEF00D
    H.check(H.lib().opure_philox_uniform(dev.h, seed, int(pb), int(sb), 2, n, int(ob)))
    dev.sync()
    got = dev.download(ob, np.uint32, (n,))
    want = np.array([O.lib().orc_philox_u32(seed, int(p), int(s), 2) for p, s in zip(pos, seq)], dtype=np.uint32)
    assert np.array_equal(got, want)


def test_rollback_bit_exact(dev):
    hm = O.HostModel(n_layers=2, hidden=64, n_heads=4, n_kv_heads=2, head_dim=32, ffn=64, vocab=64,
                     wfmt=O.W_I8PC, afmt=O.A_F16, seed=3)
    kv = O.HostKV(hm, n_pages=10, batch=3, max_pages_per_seq=4)
    kv.fill_random(np.random.default_rng(2))
    kv.page_table[0, :3] = [5, 1, 2]
    kv.page_table[1, :2] = [0, 3]
    kv.page_table[2, :2] = [7, 8]
    seq_len = np.array([14, 9, 26], np.int32)
    acc = np.array([1, 5, 0], np.int32)
    pool0, pt0 = kv.pool.copy(), kv.page_table.copy()
    want_len, want_freed, want_nf = O.kv_rollback(kv, hm, 5, seq_len, acc, poison_bits=0x7E00)
    cfg = dict(hm.cfg)
    dkv = H.DeviceKV(dev, cfg, 10, 3, 4)
    dkv.set_pool(pool0)
    dkv.set_page_table(pt0)
    m = attn_model(4, 2, 32, H.A_F16, n_layers=2)
    sl, ac = dev.upload(seq_len), dev.upload(acc)
    nl, fr, nf = dev.alloc(12), dev.alloc(3 * 8 * 4), dev.alloc(12)
    dev.fill_u32(fr, 0xFFFFFFFF, 24)
    a = H.RollbackArgs(C.pointer(m), C.pointer(dkv.desc), 3, 5, int(sl), int(ac), int(nl), int(fr), 8, int(nf), 1,
                       0x7E00)
    H.check(H.lib().opure_kv_rollback(dev.h, C.byref(a)))
    dev.sync()
    assert np.array_equal(dev.download(nl, np.int32, (3,)), want_len)
    assert np.array_equal(dev.download(nf, np.int32, (3,)), want_nf)
    assert np.array_equal(dev.download(fr, np.int32, (3, 8)), want_freed)
    assert np.array_equal(dkv.get_page_table(), kv.page_table)
    assert np.array_equal(dkv.get_pool(), kv.pool)


# ---------------------------------------------------------------------------
@pytest.mark.parametrize("wfmt", [H.W_I8PC, H.W_I4G128], ids=["i8pc", "i4g128"])
def test_device_quantisers_match_oracle(dev, wfmt):
    """The device quantisers that build every synthetic model (opure_quantize_*)
    produce the oracle quantisers' bits (oracle.quant_i8pc / quant_i4g128):
    same int8 / packed uint4 codes, same fp16 / bf16 scales and zero points."""
    rng = np.random.default_rng(17 + wfmt)
    out, inn = 96, 4096
    w = (rng.standard_normal((out, inn)) * 0.02).astype(np.float32)
    w[3] = 0.0                                      # an all-zero row (scale from the 1e-8 floor)
    w[5, :128] = 0.01                               # a constant group
    w[7] *= 40.0                                    # a wide row
    wb = dev.upload(w)
    want = O.quant_i8pc(w) if wfmt == H.W_I8PC else O.quant_i4g128(w)
    if wfmt == H.W_I8PC:
        q, s = dev.alloc(out * inn), dev.alloc(out * 2)
        H.check(H.lib().opure_quantize_i8pc(dev.h, int(wb), out, inn, int(q), int(s)))
        dev.sync()
        assert np.array_equal(dev.download(q, np.int8, (out, inn)), want["w"])
        assert np.array_equal(dev.download(s, np.uint16, (out,)), want["scale"])
    else:
        G = inn // 128
        q, s, z = dev.alloc(out * inn // 2), dev.alloc(out * G * 2), dev.alloc(out * G * 2)
        H.check(H.lib().opure_quantize_i4g128(dev.h, int(wb), out, inn, int(q), int(s), int(z)))
        dev.sync()
        assert np.array_equal(dev.download(q, np.uint8, (out, inn // 2)), want["w"])
        assert np.array_equal(dev.download(s, np.uint16, (out, G)), want["scale"])
        assert np.array_equal(dev.download(z, np.uint16, (out, G)), want["zero"])


# ---------------------------------------------------------------------------
def test_bw_measure_copies_and_reports(dev):
    """opure_bw_measure: a copy leaves dst equal to src, both modes report a
    positive rate below the published 8 TB/s ceiling of a read, and bad
    arguments are refused before any launch."""
    n = 64 << 20
    src, dst = dev.alloc(n), dev.alloc(n)
    H.check(H.lib().opure_synth_normal_f32(dev.h, int(src), n // 4, 5, 0, 1.0, 0.0))
    dev.fill_u32(dst, 0, n // 4)
    read = dev.bw_measure(H.BW_READ, src, None, n, 3)
    copy = dev.bw_measure(H.BW_COPY, src, dst, n, 2)
    assert 0.0 < read and 0.0 < copy
    a = dev.download(src, np.uint32, (n // 4,))
    b = dev.download(dst, np.uint32, (n // 4,))
    assert np.array_equal(a, b)
    g = C.c_double()
    assert H.lib().opure_bw_measure(dev.h, H.BW_COPY, int(src), None, n, 1, C.byref(g)) == H.E_INVALID
    assert H.lib().opure_bw_measure(dev.h, H.BW_READ, int(src), None, n - 8, 1, C.byref(g)) == H.E_INVALID
