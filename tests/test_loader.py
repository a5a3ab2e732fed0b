"""The model-directory loader on the host (no GPU): safetensors files written
here from the oracle's host models are read back byte for byte, q/k/v and
gate/up come back fused exactly as the oracle's models hold them, and bad
files fail with an error that names the problem.

Cases the reference's own reader gets wrong are pinned here: packed 4-bit
tensors take half a byte per element (its ElementBytes(I4) = 1,
src/core/Opure_Streamer.cpp:104-117, rejects them), and its per-tensor
"scale" header key is honoured per tensor (it uploads every scale from one
loop variable's address, src/engine/Opure_Graph.cpp:521-527).
"""
import json
import os

import numpy as np
import pytest

import opure_engine as E
import opure_hip as H
import oracle as O
import st_write as W


def small(wfmt, afmt, tied=True, seed=5, n_layers=2):
    return O.HostModel(n_layers=n_layers, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1024,
                       wfmt=wfmt, afmt=afmt, attn_scale=0.125, theta=10000.0, max_pos=512, tied=tied, seed=seed,
                       norm_jitter=0.1)


FMTS = [(O.W_F32, O.A_F32), (O.W_I8PC, O.A_F16), (O.W_I4G128, O.A_BF16)]
FMT_IDS = ["f32", "i8", "i4"]


def as_bytes(a):
    return None if a is None else np.ascontiguousarray(a).view(np.uint8).ravel()


def expect_linear(got: dict, lin: dict, wfmt: int):
    assert got["wfmt"] == wfmt and got["out"] == lin["out"] and got["in"] == lin["in"]
    assert np.array_equal(got["w"], as_bytes(lin["w"]))
    if wfmt == O.W_F32:
        assert got["scale"] is None and got["zero"] is None
    else:
        assert np.array_equal(got["scale"], as_bytes(lin["scale"]))
    if wfmt == O.W_I4G128:
        assert np.array_equal(got["zero"], as_bytes(lin["zero"]))


def expect_model(f: E.ModelFiles, m: O.HostModel):
    c = m.cfg
    wf = c["wfmt"]
    expect_linear(f.read(E.ROLE_EMBED), m.embed, wf)
    expect_linear(f.read(E.ROLE_LM_HEAD), m.lm_head, wf)
    fn = f.read(E.ROLE_FINAL_NORM)
    assert fn["out"] == c["hidden"] and fn["in"] == 1 and np.array_equal(fn["w"], as_bytes(m.final_norm))
    for i, L in enumerate(m.layers):
        for role, key in ((E.ROLE_QKV, "qkv"), (E.ROLE_O, "o"), (E.ROLE_GATE_UP, "gate_up"), (E.ROLE_DOWN, "down")):
            expect_linear(f.read(role, i), L[key], wf)
        assert np.array_equal(f.read(E.ROLE_ATTN_NORM, i)["w"], as_bytes(L["attn_norm"]))
        assert np.array_equal(f.read(E.ROLE_MLP_NORM, i)["w"], as_bytes(L["mlp_norm"]))


@pytest.mark.parametrize("fmt", FMTS, ids=FMT_IDS)
@pytest.mark.parametrize("tied", [True, False], ids=["tied", "untied"])
def test_round_trip(tmp_path, fmt, tied):
    m = small(*fmt, tied=tied)
    d = W.write_model_dir(str(tmp_path / "m"), m)
    f = E.ModelFiles(d)
    i = f.info()
    c = m.cfg
    assert (i.n_layers, i.hidden, i.n_heads, i.n_kv_heads, i.head_dim, i.ffn, i.vocab) == \
        (c["n_layers"], c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["ffn"], c["vocab"])
    assert i.stored_wfmt == fmt[0] and i.wfmt == fmt[0] and i.afmt == fmt[1]
    assert i.tied == int(tied) and i.rope_max_pos == c["max_pos"] and i.rope_theta == 10000.0
    assert np.float32(i.rms_eps) == np.float32(c["rms_eps"])
    assert np.float32(i.attn_scale) == np.float32(0.125)      # default 1/sqrt(64)
    assert i.file_bytes == os.path.getsize(os.path.join(d, "model.safetensors"))
    expect_model(f, m)
    f.close()


def test_safetensors_entries_read_back(tmp_path):
    """Every entry: dtype, shape, absolute offset and bytes as written; packed
    4-bit entries are half a byte per element."""
    m = small(O.W_I4G128, O.A_BF16, tied=False)
    t = W.model_tensors(m, int4_dtype="U4")
    p = str(tmp_path / "a.safetensors")
    W.write_safetensors(p, t, {"format": "pt"})
    st = E.SafeTensors(p)
    got = st.tensors()
    assert [g["name"] for g in got] == [e[0] for e in t]
    with open(p, "rb") as fh:
        hlen = int.from_bytes(fh.read(8), "little")
    off = 8 + hlen
    for g, (name, dtype, shape, raw, _) in zip(got, t):
        assert g["dtype"] == dtype and g["shape"] == tuple(shape) and g["offset"] == off
        assert g["bytes"] == len(raw) and g["data"].tobytes() == bytes(raw)
        if dtype == "U4":
            assert g["bytes"] * 2 == int(np.prod(shape))
        off += len(raw)
    q = st.find("model.layers.1.self_attn.k_proj.weight")
    assert q["shape"] == (m.cfg["n_kv_heads"] * 64, 256) and q["dtype"] == "U4"
    with pytest.raises(H.OpureError) as e:
        st.find("model.layers.9.self_attn.k_proj.weight")
    assert e.value.code == H.E_INVALID and "not found" in str(e.value)
    st.close()


@pytest.mark.parametrize("int4_dtype", ["U8", "U4"])
def test_int4_packed_forms(tmp_path, int4_dtype):
    m = small(O.W_I4G128, O.A_BF16)
    d = W.write_model_dir(str(tmp_path / "m"), m, int4_dtype=int4_dtype)
    expect_model(E.ModelFiles(d), m)


def test_sharded_index(tmp_path):
    m = small(O.W_I8PC, O.A_F16, tied=False)
    d = W.write_model_dir(str(tmp_path / "m"), m, shards=3)
    f = E.ModelFiles(d)
    assert f.info().n_tensors == len(W.model_tensors(m))
    expect_model(f, m)


@pytest.mark.parametrize("dtype", ["BF16", "F16"])
def test_float16_weights_widen_exactly(tmp_path, dtype):
    """BF16 / F16 weights and norms are widened to fp32 exactly."""
    m = small(O.W_F32, O.A_F32)
    d = W.write_model_dir(str(tmp_path / "m"), m, float_dtype=dtype, norm_dtype=dtype)
    f = E.ModelFiles(d)

    def rt(a):
        a = np.asarray(a, np.float32)
        if dtype == "F16":
            return a.astype(np.float16).astype(np.float32)
        return O.bf16_bits_to_f32(O.np_f32_to_bf16_bits(a).reshape(a.shape))
    got = f.read(E.ROLE_QKV, 1)
    assert np.array_equal(got["w"].view(np.float32).reshape(got["out"], got["in"]), rt(m.layers[1]["qkv"]["w"]))
    got = f.read(E.ROLE_ATTN_NORM, 0)
    assert np.array_equal(got["w"].view(np.float32), rt(m.layers[0]["attn_norm"]))


def test_signed_int4_reads_as_unsigned_with_zero_8(tmp_path):
    """I4 (signed nibbles v) is stored as U4 nibbles v + 8 with zero point 8:
    s * ((v + 8) - 8) = s * v."""
    m = small(O.W_I4G128, O.A_BF16)
    t = W.model_tensors(m, int4_dtype="U4")
    out = []
    for name, dtype, shape, raw, extra in t:
        if name.endswith(".weight_zero"):
            continue
        if dtype == "U4":
            raw = (np.frombuffer(raw, np.uint8) ^ 0x88).tobytes()   # u - 8 in two's complement nibbles
            dtype = "I4"
        out.append((name, dtype, shape, raw, extra))
    d = tmp_path / "m"
    d.mkdir()
    W.write_safetensors(str(d / "model.safetensors"), out)
    (d / "config.json").write_text(json.dumps(W.config_of(m)))
    got = E.ModelFiles(str(d)).read(E.ROLE_O, 0)
    lin = m.layers[0]["o"]
    assert np.array_equal(got["w"], as_bytes(lin["w"]))
    assert np.array_equal(got["scale"], as_bytes(lin["scale"]))
    assert (got["zero"].view(np.uint16) == O.np_f32_to_bf16_bits(np.float32(8.0))).all()
    # the signed reading: v = nibble - 16 when the sign bit is set (Opure_Streamer.cpp:403-426)
    b = np.frombuffer(out[[e[0] for e in out].index("model.layers.0.self_attn.o_proj.weight")][3], np.uint8)
    hi = (b >> 4).astype(np.int32)
    v = np.where(hi >= 8, hi - 16, hi)
    assert np.array_equal(v + 8, (lin["w"].ravel() >> 4).astype(np.int32))


def test_reference_header_scale_form(tmp_path):
    """The reference's files: quantised tensors with a per-tensor "scale" key
    and no scale tensors.  int8 reads as per-channel with fp16(scale) on every
    row; U4 as group-128 with bf16(scale) and zero 0."""
    m = small(O.W_I8PC, O.A_F16)
    t = [e for e in W.model_tensors(m) if not e[0].endswith(".weight_scale")]
    scales = {}
    out = []
    for k, (name, dtype, shape, raw, extra) in enumerate(t):
        if dtype == "I8":
            scales[name] = 1e-3 * (1 + k)
            extra = {"scale": scales[name]}
        out.append((name, dtype, shape, raw, extra))
    d = tmp_path / "m"
    d.mkdir()
    W.write_safetensors(str(d / "model.safetensors"), out)
    (d / "config.json").write_text(json.dumps(W.config_of(m)))
    f = E.ModelFiles(str(d))
    got = f.read(E.ROLE_QKV, 1)
    p = "model.layers.1.self_attn."
    want = np.concatenate([np.full(256, scales[p + "q_proj.weight"]), np.full(128, scales[p + "k_proj.weight"]),
                           np.full(128, scales[p + "v_proj.weight"])]).astype(np.float32)
    assert np.array_equal(got["scale"].view(np.uint16), W.f32_to_f16_bits(want))
    assert np.array_equal(got["w"], as_bytes(m.layers[1]["qkv"]["w"]))
    assert E.SafeTensors(str(d / "model.safetensors")).find(p + "k_proj.weight")["scale"] == scales[p + "k_proj.weight"]

    m4 = small(O.W_I4G128, O.A_BF16)
    t = [e for e in W.model_tensors(m4, int4_dtype="U4") if not e[0].endswith((".weight_scale", ".weight_zero"))]
    t = [(n, dt, sh, raw, {"scale": 0.0123} if dt == "U4" else None) for n, dt, sh, raw, _ in t]
    d4 = tmp_path / "m4"
    d4.mkdir()
    W.write_safetensors(str(d4 / "model.safetensors"), t)
    (d4 / "config.json").write_text(json.dumps(W.config_of(m4)))
    got = E.ModelFiles(str(d4)).read(E.ROLE_DOWN, 0)
    assert (got["scale"].view(np.uint16) == O.np_f32_to_bf16_bits(np.float32(0.0123))).all()
    assert (got["zero"].view(np.uint16) == 0).all()


def test_quantise_on_load_option(tmp_path):
    m = small(O.W_F32, O.A_F32)
    d = W.write_model_dir(str(tmp_path / "m"), m)
    i = E.ModelFiles(d, E.load_options(wfmt=H.W_I4G128, attn_scale=1.0)).info()
    assert i.stored_wfmt == H.W_F32 and i.wfmt == H.W_I4G128 and i.afmt == H.A_BF16 and i.attn_scale == 1.0
    # a quantised file cannot be loaded as another quantised format
    d8 = W.write_model_dir(str(tmp_path / "m8"), small(O.W_I8PC, O.A_F16))
    with pytest.raises(H.OpureError) as e:
        E.ModelFiles(d8, E.load_options(wfmt=H.W_I4G128))
    assert e.value.code == H.E_UNSUPPORTED


# ---- malformed files ---------------------------------------------------------
def _err(d, opts=None):
    with pytest.raises(H.OpureError) as e:
        E.ModelFiles(str(d), opts)
    return e.value


def _dir_with(tmp_path, m, tensors=None, cfg=None, patch=None):
    d = tmp_path / "bad"
    d.mkdir(exist_ok=True)
    W.write_safetensors(str(d / "model.safetensors"), tensors if tensors is not None else W.model_tensors(m),
                        header_patch=patch)
    (d / "config.json").write_text(json.dumps(cfg if cfg is not None else W.config_of(m)))
    return d


def test_int4_sized_one_byte_per_element_is_rejected(tmp_path):
    """A U4 entry whose span was computed at one byte per element (the
    reference's ElementBytes(I4)) does not match its shape."""
    m = small(O.W_I4G128, O.A_BF16)
    t = W.model_tensors(m, int4_dtype="U4")
    t = [(n, dt, sh, raw + bytes(len(raw)) if n == "model.layers.0.mlp.up_proj.weight" else raw, x)
         for n, dt, sh, raw, x in t]
    e = _err(_dir_with(tmp_path, m, t))
    assert e.code == H.E_INVALID and "up_proj.weight" in str(e) and "imply" in str(e)


def test_bad_files_name_the_problem(tmp_path):
    m = small(O.W_I8PC, O.A_F16)
    base = W.model_tensors(m)
    # a tensor missing
    e = _err(_dir_with(tmp_path, m, [x for x in base if x[0] != "model.layers.1.mlp.down_proj.weight"]))
    assert "model.layers.1.mlp.down_proj.weight" in str(e) and "not found" in str(e)
    # a wrong shape
    bad = [(n, dt, (sh[0] // 2, sh[1] * 2) if n == "model.layers.0.self_attn.k_proj.weight" else sh, r, x)
           for n, dt, sh, r, x in base]
    e = _err(_dir_with(tmp_path, m, bad))
    assert "k_proj.weight" in str(e) and "[128, 256]" in str(e)
    # a scale of the wrong length
    bad = [(n, dt, (sh[0] // 2,), r[:len(r) // 2], x) if n == "model.layers.0.self_attn.o_proj.weight_scale"
           else (n, dt, sh, r, x) for n, dt, sh, r, x in base]
    e = _err(_dir_with(tmp_path, m, bad))
    assert "o_proj.weight_scale" in str(e)
    # no scale at all
    e = _err(_dir_with(tmp_path, m, [x for x in base if x[0] != "model.layers.0.mlp.up_proj.weight_scale"]))
    assert "up_proj.weight" in str(e) and "scale" in str(e)
    # data_offsets past the payload
    def past(h):
        h["model.norm.weight"]["data_offsets"][1] += 4096
    e = _err(_dir_with(tmp_path, m, base, patch=past))
    assert "model.norm.weight" in str(e)
    # offsets out of order
    def rev(h):
        a = h["model.embed_tokens.weight"]["data_offsets"]
        h["model.embed_tokens.weight"]["data_offsets"] = [a[1], a[0]]
    e = _err(_dir_with(tmp_path, m, base, patch=rev))
    assert "embed_tokens" in str(e)
    # unknown dtype
    def f8(h):
        h["model.norm.weight"]["dtype"] = "F8_E4M3"
    assert _err(_dir_with(tmp_path, m, base, patch=f8)).code == H.E_UNSUPPORTED


@pytest.mark.parametrize("over,code,words", [
    ({"rope_scaling": {"rope_type": "llama3", "factor": 8.0}}, H.E_UNSUPPORTED, "rope_scaling"),
    ({"hidden_act": "gelu"}, H.E_UNSUPPORTED, "gelu"),
    ({"head_dim": 72}, H.E_UNSUPPORTED, "head_dim"),
    ({"head_dim": 320}, H.E_UNSUPPORTED, "head_dim"),
    ({"attention_bias": True}, H.E_UNSUPPORTED, "bias"),
    ({"num_key_value_heads": 3}, H.E_INVALID, "num_key_value_heads"),
    ({"rms_norm_eps": None}, H.E_INVALID, "rms_norm_eps"),
    ({"hidden_size": -1}, H.E_INVALID, "hidden_size"),
], ids=["rope_scaling", "act", "head_dim", "head_dim_big", "bias", "gqa", "eps", "negative"])
def test_config_refusals(tmp_path, over, code, words):
    m = small(O.W_I8PC, O.A_F16)
    cfg = W.config_of(m, **over)
    if over.get("rms_norm_eps", 1) is None:
        del cfg["rms_norm_eps"]
    e = _err(_dir_with(tmp_path, m, cfg=cfg))
    assert e.code == code and words in str(e)


def test_truncated_and_garbled_files(tmp_path):
    m = small(O.W_F32, O.A_F32, n_layers=1)
    d = _dir_with(tmp_path, m)
    p = d / "model.safetensors"
    raw = p.read_bytes()
    p.write_bytes(raw[:5])
    assert "shorter" in str(_err(d))
    p.write_bytes((len(raw) * 2).to_bytes(8, "little") + raw[8:])
    assert "header length" in str(_err(d))
    hlen = int.from_bytes(raw[:8], "little")
    p.write_bytes(raw[:8] + raw[8:8 + hlen].replace(b'"dtype":', b'"dtype";', 1) + raw[8 + hlen:])
    assert "json" in str(_err(d))
    (d / "config.json").write_text("{\"vocab_size\": 12,")
    p.write_bytes(raw)
    assert "json" in str(_err(d))
    os.remove(d / "config.json")
    assert "config.json" in str(_err(d))


# ---- RoPE pairing of the stored q / k rows -------------------------------------
def test_rope_pairs_half_matches_a_rotate_half_forward(tmp_path):
    """A checkpoint trained with rotate-half RoPE (HF Llama's pairs (p, p + hd/2)),
    loaded with rope_pairs = HALF: the loader permutes each head's q / k rows
    (new 2p = old p, new 2p+1 = old p + hd/2, scales and zero points with them),
    and the oracle's adjacent-pair forward on the loaded weights equals an
    independent numpy forward that applies rotate-half RoPE to the weights as
    stored.  Loaded as ADJACENT (the reference's reading) the same file gives
    a different forward, so the option is what makes it right."""
    import npref
    m = small(O.W_F32, O.A_F32, n_layers=2, seed=12)
    d = W.write_model_dir(str(tmp_path / "hf"), m)
    f = E.ModelFiles(d, E.load_options(attn_scale=0.125, rope_pairs=E.ROPE_PAIRS_HALF))
    c = m.cfg
    nh, nkv, hd = c["n_heads"], c["n_kv_heads"], c["head_dim"]
    layers = []
    for i, L in enumerate(m.layers):
        got = f.read(E.ROLE_QKV, i)
        q = got["w"].view(np.float32).reshape(got["out"], got["in"])
        src = L["qkv"]["w"]
        perm = np.arange(got["out"])
        for h0, n in ((0, nh), (nh * hd, nkv)):
            for hh in range(n):
                b = h0 + hh * hd
                perm[b:b + hd:2] = b + np.arange(hd // 2)
                perm[b + 1:b + hd:2] = b + hd // 2 + np.arange(hd // 2)
        assert np.array_equal(q, src[perm])                     # q and k permuted per head, v as stored
        layers.append(dict(L, qkv=dict(L["qkv"], w=np.ascontiguousarray(q))))
    loaded = O.HostModel.from_arrays(c, dict(embed=m.embed, lm_head=m.lm_head, final_norm=m.final_norm,
                                             rope_cos=m.rope_cos, rope_sin=m.rope_sin, layers=layers))
    R = 8
    tokens = np.random.default_rng(3).integers(0, c["vocab"], size=(1, R)).astype(np.int32)
    seq = np.zeros(1, np.int32)
    kv = O.HostKV(loaded, n_pages=4, batch=1, max_pages_per_seq=4)
    kv.page_table[0] = np.arange(4)
    got = O.verify_forward(loaded, kv, tokens, seq)
    pool = np.zeros_like(kv.pool)
    want = npref.forward(m, pool, kv.page_table, tokens, seq, rope_pairs="half")
    assert np.abs(got - want).max() <= 1e-4
    kv2 = O.HostKV(m, n_pages=4, batch=1, max_pages_per_seq=4)
    kv2.page_table[0] = np.arange(4)
    assert np.abs(O.verify_forward(m, kv2, tokens, seq) - want).max() > 1e-2
    f.close()


def test_rope_pairs_half_moves_scales_with_rows(tmp_path):
    """int8 and int4 files: the permuted q / k rows keep their own scales (and
    int4 zero points)."""
    for wfmt, afmt in ((O.W_I8PC, O.A_F16), (O.W_I4G128, O.A_BF16)):
        m = small(wfmt, afmt, n_layers=1, seed=13)
        d = W.write_model_dir(str(tmp_path / f"m{wfmt}"), m)
        plain = E.ModelFiles(d).read(E.ROLE_QKV, 0)
        half = E.ModelFiles(d, E.load_options(rope_pairs=E.ROPE_PAIRS_HALF)).read(E.ROLE_QKV, 0)
        out, hd = plain["out"], m.cfg["head_dim"]
        qk = (m.cfg["n_heads"] + m.cfg["n_kv_heads"]) * hd
        perm = np.arange(out)
        for b in range(0, qk, hd):
            perm[b:b + hd:2] = b + np.arange(hd // 2)
            perm[b + 1:b + hd:2] = b + hd // 2 + np.arange(hd // 2)
        for key in ("w", "scale", "zero"):
            if plain[key] is None:
                continue
            a, b = plain[key].reshape(out, -1), half[key].reshape(out, -1)
            assert np.array_equal(b, a[perm]), key
    with pytest.raises(H.OpureError) as e:
        E.ModelFiles(d, E.load_options(rope_pairs=2))
    assert e.value.code == H.E_INVALID and "rope_pairs" in str(e.value)


# ---- untrusted headers, shard names and scales ----------------------------------
def test_hostile_headers_are_refused(tmp_path):
    """Shapes whose element count overflows 64 bits, dimensions that are not
    integers below 2^53, and headers nested past 64 levels fail with an error
    (the reader never wraps a size or recurses without bound)."""
    m = small(O.W_F32, O.A_F32, n_layers=1)
    name = "model.layers.0.mlp.down_proj.weight"

    def patched(fn):
        d = _dir_with(tmp_path, m, patch=fn)
        return _err(d)

    def huge(h):
        h[name]["shape"] = [2 ** 32, 2 ** 32]
        h[name]["data_offsets"] = [0, 0]
    e = patched(huge)
    assert e.code == H.E_INVALID and "overflows" in str(e)

    def big_dim(h):
        h[name]["shape"] = [2 ** 60, 1]
    assert "bad shape" in str(patched(big_dim))

    def frac_dim(h):
        h[name]["shape"] = [256.5, 512]
    assert "bad shape" in str(patched(frac_dim))

    def frac_off(h):
        a, b = h[name]["data_offsets"]
        h[name]["data_offsets"] = [a + 0.5, b + 0.5]
    assert "data_offsets" in str(patched(frac_off))

    def deep(h):
        v = 1
        for _ in range(200):
            v = [v]
        h["__metadata__"] = {"nest": v}
    e = patched(deep)
    assert e.code == H.E_INVALID and "nesting" in str(e)


def test_shard_names_stay_inside_the_directory(tmp_path):
    m = small(O.W_I8PC, O.A_F16, tied=False)
    d = W.write_model_dir(str(tmp_path / "m"), m, shards=2)
    idx = os.path.join(d, "model.safetensors.index.json")
    doc = json.load(open(idx))
    first = next(iter(doc["weight_map"]))
    outside = tmp_path / "elsewhere.safetensors"
    outside.write_bytes(open(os.path.join(d, doc["weight_map"][first]), "rb").read())
    for bad in ("../elsewhere.safetensors", str(outside)):
        doc["weight_map"][first] = bad
        json.dump(doc, open(idx, "w"))
        e = _err(d)
        assert e.code == H.E_INVALID and "outside the model directory" in str(e)
    # a link inside the directory that points out of it
    os.symlink(str(outside), os.path.join(d, "link.safetensors"))
    doc["weight_map"][first] = "link.safetensors"
    json.dump(doc, open(idx, "w"))
    assert "resolves outside" in str(_err(d))


def test_scales_outside_the_kernel_range_are_refused(tmp_path):
    """A finite nonzero scale that rounds to 0 or to infinity in the fp16 (int8)
    or bf16 (int4) the kernels read would zero or blow up its linear: refused."""
    m = small(O.W_I8PC, O.A_F16, n_layers=1)
    t = W.model_tensors(m)
    sname = "model.layers.0.self_attn.o_proj.weight_scale"
    for val in (1e-9, 1e6):
        bad = [(n, "F32", sh, np.full(sh, val, np.float32).tobytes(), x) if n == sname else (n, dt, sh, r, x)
               for n, dt, sh, r, x in t]
        f = E.ModelFiles(str(_dir_with(tmp_path, m, bad)))
        with pytest.raises(H.OpureError) as e:
            f.read(E.ROLE_O, 0)
        assert e.value.code == H.E_UNSUPPORTED and "fp16 range" in str(e.value)
        f.close()
    m4 = small(O.W_I4G128, O.A_BF16, n_layers=1)
    t4 = [e for e in W.model_tensors(m4, int4_dtype="U4") if not e[0].endswith((".weight_scale", ".weight_zero"))]
    t4 = [(n, dt, sh, raw, {"scale": 1e-45} if dt == "U4" else None) for n, dt, sh, raw, _ in t4]
    f = E.ModelFiles(str(_dir_with(tmp_path, m4, t4)))
    with pytest.raises(H.OpureError) as e:
        f.read(E.ROLE_DOWN, 0)
    assert e.value.code == H.E_UNSUPPORTED and "bf16 range" in str(e.value)
