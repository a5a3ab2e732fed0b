"""Verify steps on models loaded from disk (config.json + safetensors through
opure_model_load) against the CPU oracle.

- a model written from an oracle host model and loaded from its directory
  gives the same logits, bit for bit, as the same weights uploaded directly,
  and logits within the path's bar of the oracle's (1e-4 fp32, 2e-2 16-bit);
- a float model loaded as int8 / int4 (quantised on the device at load time)
  equals the oracle run on the oracle's own quantisation of the same weights;
- the engine created from directories (opure_engine_initialize) emits the
  same ids as the engine over directly uploaded models.
"""
import ctypes as C

import numpy as np
import pytest

import opure_engine as E
import opure_hip as H
import oracle as O
import st_write as W
from gpu_util import VerifyRunner, device_kv, device_model, say
from test_gpu_verify import random_cache, small_model

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = H.Dev(0)
    yield d
    d.close()


class Loaded:
    """A loaded model in the shape VerifyRunner takes (desc + cfg)."""

    def __init__(self, dev, d, opts=None):
        self.lm = E.LoadedModel(dev, d, opts)
        self.desc = self.lm.desc
        self.cfg = {"vocab": self.desc.vocab}


def step_logits(dev, dm, m, kv, tokens, seq_len):
    B, R = tokens.shape
    dkv = device_kv(dev, m, kv)
    run = VerifyRunner(dev, dm, dkv, B, R, max_ctx=320)
    run.step(tokens, seq_len, accept=H.ACCEPT_GREEDY)
    return run.get_logits(), run.get_accept()


FMTS = [(O.W_F32, O.A_F32, 1e-4), (O.W_I8PC, O.A_F16, 2e-2), (O.W_I4G128, O.A_BF16, 2e-2)]
FMT_IDS = ["f32", "i8-f16", "i4-bf16"]


@pytest.mark.parametrize("fmt", FMTS, ids=FMT_IDS)
@pytest.mark.parametrize("tied", [True, False], ids=["tied", "untied"])
def test_loaded_model_verify_step(dev, tmp_path, fmt, tied):
    wfmt, afmt, tol = fmt
    say("loaded model", FMT_IDS[FMTS.index(fmt)], "tied" if tied else "untied")
    m = small_model(wfmt, afmt, tied=tied)
    d = W.write_model_dir(str(tmp_path / "m"), m, shards=2 if tied else 1)
    lm = Loaded(dev, d)
    c = lm.desc
    assert (c.wfmt, c.afmt, c.rope_max_pos) == (wfmt, afmt, m.cfg["max_pos"])
    assert np.float32(c.attn_scale) == np.float32(m.cfg["attn_scale"])
    half = m.cfg["head_dim"] // 2
    assert np.array_equal(dev.download(c.rope_cos, np.float32, (c.rope_max_pos, half)), m.rope_cos)
    assert np.array_equal(dev.download(c.rope_sin, np.float32, (c.rope_max_pos, half)), m.rope_sin)

    B, R = 2, 5
    kv = random_cache(m, B, 320, 48, seed=7)
    seq_len = np.array([251, 96], np.int32)
    tokens = np.random.default_rng(3).integers(0, m.cfg["vocab"], size=(B, R)).astype(np.int32)
    got, (out, acc) = step_logits(dev, lm, m, kv, tokens, seq_len)
    ref, (rout, racc) = step_logits(dev, device_model(dev, m), m, kv, tokens, seq_len)
    assert np.array_equal(got, ref), "a loaded model differs from the same weights uploaded directly"
    assert np.array_equal(out, rout) and np.array_equal(acc, racc)

    kv_o = O.HostKV(m, n_pages=kv.n_pages, batch=B, max_pages_per_seq=kv.max_pages)
    kv_o.pool[...] = kv.pool
    kv_o.page_table[...] = kv.page_table
    want = O.verify_forward(m, kv_o, tokens, seq_len)
    err = np.abs(got - want).max()
    say("max_abs logits vs oracle", err)
    assert err <= tol
    w_out, w_acc = O.accept_greedy(got, tokens[:, 1:])
    assert np.array_equal(out, w_out) and np.array_equal(acc, w_acc)
    lm.lm.close()


def test_head_dim_96_through_the_vector_attention(dev, tmp_path):
    """A head size the reference refuses (96): loaded, and verified against
    the oracle through the attention's vector path."""
    m = small_model(O.W_I8PC, O.A_F16, hidden=384, heads=(4, 2), hd=96, attn_scale=96 ** -0.5)
    d = W.write_model_dir(str(tmp_path / "m"), m)
    lm = Loaded(dev, d)
    assert lm.desc.head_dim == 96
    B, R = 2, 5
    kv = random_cache(m, B, 320, 48, seed=7)
    seq_len = np.array([251, 96], np.int32)
    tokens = np.random.default_rng(3).integers(0, m.cfg["vocab"], size=(B, R)).astype(np.int32)
    got, _ = step_logits(dev, lm, m, kv, tokens, seq_len)
    kv_o = O.HostKV(m, n_pages=kv.n_pages, batch=B, max_pages_per_seq=kv.max_pages)
    kv_o.pool[...] = kv.pool
    kv_o.page_table[...] = kv.page_table
    err = np.abs(got - O.verify_forward(m, kv_o, tokens, seq_len)).max()
    say("max_abs logits vs oracle (hd 96)", err)
    assert err <= 2e-2
    lm.lm.close()


@pytest.mark.parametrize("wfmt,afmt", [(O.W_I8PC, O.A_F16), (O.W_I4G128, O.A_BF16)], ids=["to-i8", "to-i4"])
def test_float_model_quantised_on_load(dev, tmp_path, wfmt, afmt):
    f = small_model(O.W_F32, O.A_F32, tied=False, seed=9)
    d = W.write_model_dir(str(tmp_path / "m"), f)
    lm = Loaded(dev, d, E.load_options(wfmt=wfmt, afmt=afmt))
    assert (lm.desc.wfmt, lm.desc.afmt) == (wfmt, afmt)
    q = O.quant_i8pc if wfmt == O.W_I8PC else O.quant_i4g128
    cfg = dict(f.cfg, wfmt=wfmt, afmt=afmt)
    w = {"embed": q(f.embed["w"]), "lm_head": q(f.lm_head["w"]), "final_norm": f.final_norm,
         "rope_cos": f.rope_cos, "rope_sin": f.rope_sin,
         "layers": [dict(attn_norm=L["attn_norm"], mlp_norm=L["mlp_norm"],
                         **{k: q(L[k]["w"]) for k in ("qkv", "o", "gate_up", "down")}) for L in f.layers]}
    m = O.HostModel.from_arrays(cfg, w)
    B, R = 2, 5
    kv = random_cache(m, B, 320, 48, seed=7)
    seq_len = np.array([251, 96], np.int32)
    tokens = np.random.default_rng(3).integers(0, m.cfg["vocab"], size=(B, R)).astype(np.int32)
    got, _ = step_logits(dev, lm, m, kv, tokens, seq_len)
    ref, _ = step_logits(dev, device_model(dev, m), m, kv, tokens, seq_len)
    assert np.array_equal(got, ref), "device quantisation at load differs from the oracle's quantisers"
    kv_o = O.HostKV(m, n_pages=kv.n_pages, batch=B, max_pages_per_seq=kv.max_pages)
    kv_o.pool[...] = kv.pool
    kv_o.page_table[...] = kv.page_table
    err = np.abs(got - O.verify_forward(m, kv_o, tokens, seq_len)).max()
    say("max_abs logits vs oracle", err)
    assert err <= 2e-2
    lm.lm.close()


def test_engine_from_directories(dev, tmp_path):
    """opure_engine_initialize over a target and a draft directory emits the
    ids of the engine over the same weights uploaded directly, greedy and
    speculative."""
    tgt = small_model(O.W_I8PC, O.A_F16, n_layers=4, seed=11, max_pos=256)
    drf = small_model(O.W_I8PC, O.A_F16, n_layers=1, seed=12, max_pos=256)
    td = W.write_model_dir(str(tmp_path / "target"), tgt)
    dd = W.write_model_dir(str(tmp_path / "draft"), drf)
    prompt = np.random.default_rng(5).integers(0, 1024, 24).astype(np.int32)
    a = E.Engine.from_dirs(dev, td, dd, max_positions=256, draft_tokens=4)
    ga, _ = a.generate(prompt, 40)
    sa, ha, _ = a.generate_speculative(prompt, 40)
    dt, dd_ = device_model(dev, tgt), device_model(dev, drf)
    b = E.Engine(dev, dt.desc, dd_.desc, max_positions=256, draft_tokens=4)
    gb, _ = b.generate(prompt, 40)
    sb, hb, _ = b.generate_speculative(prompt, 40)
    say("greedy", ga[:10].tolist(), "accepted", ha.tolist())
    assert np.array_equal(ga, gb) and np.array_equal(sa, sb) and np.array_equal(ha, hb)
    assert np.array_equal(sa, ga)
    a.close()
    b.close()


@pytest.mark.parametrize("pairs", ["adjacent", "half"])
def test_forward_logits_from_directory(dev, tmp_path, pairs):
    """The engine's ForwardLogits (opure_engine_forward_logits) on a model
    loaded from its directory by the engine itself (Initialize(modelDir, ...)):
    the last position's logits of a 12-token prompt against the numpy forward
    of the stored weights, fp32 (1e-4).  "half": the directory holds a
    rotate-half checkpoint and is loaded with rope_pairs = HALF, so the
    kernels' adjacent-pair RoPE on the permuted rows must give the
    rotate-half forward of the rows as stored."""
    import npref
    m = small_model(O.W_F32, O.A_F32, n_layers=2, seed=21, max_pos=256)
    d = W.write_model_dir(str(tmp_path / pairs), m)
    lo = E.load_options(attn_scale=float(m.cfg["attn_scale"]),
                        rope_pairs=E.ROPE_PAIRS_HALF if pairs == "half" else E.ROPE_PAIRS_ADJACENT)
    eng = E.Engine.from_dirs(dev, d, None, load=lo, max_positions=64, draft_tokens=4)
    n = 12
    tokens = np.random.default_rng(8).integers(0, m.cfg["vocab"], size=(1, n)).astype(np.int32)
    got, am = eng.forward_logits(tokens[0], m.cfg["vocab"])
    kv = O.HostKV(m, n_pages=4, batch=1, max_pages_per_seq=4)
    kv.page_table[0] = np.arange(4)
    want = npref.forward(m, np.zeros_like(kv.pool), kv.page_table, tokens, np.zeros(1, np.int32), rope_pairs=pairs)[0, -1]
    err = float(np.abs(got - want).max())
    say(pairs, "forward_logits max_abs vs numpy", err)
    assert err <= 1e-4 and am == int(np.argmax(got))
    eng.close()
