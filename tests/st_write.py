"""Writes model directories (config.json + safetensors) for the loader tests,
from the oracle's host models.

The safetensors layout follows the format's published description: an 8-byte
little-endian header length, a JSON header of {name: {dtype, shape,
data_offsets}} (offsets relative to the payload), padded with spaces to a
multiple of 8, then the payload.  Tensor names are the Hugging Face Llama
ones; q/k/v and gate/up are written as separate tensors (the loader fuses
them).
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np

import oracle as O

FLOAT_NP = {"F32": np.float32}


def write_safetensors(path: str, tensors: list, metadata: dict | None = None, header_patch=None) -> None:
    """tensors: [(name, dtype, shape, raw bytes, extra header keys or None)].
    header_patch(header_dict) may edit the header before it is written (to
    build malformed files)."""
    header, off, blobs = {}, 0, []
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, dtype, shape, raw, extra in tensors:
        raw = bytes(raw)
        e = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        if extra:
            e.update(extra)
        header[name] = e
        blobs.append(raw)
        off += len(raw)
    if header_patch:
        header_patch(header)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _float_tensor(a: np.ndarray, dtype: str) -> bytes:
    a = np.ascontiguousarray(a, np.float32)
    if dtype == "F32":
        return a.tobytes()
    if dtype == "F16":
        return f32_to_f16_bits(a).tobytes()
    return O.np_f32_to_bf16_bits(a).tobytes()


def linear_tensors(base: str, lin: dict, wfmt: int, rows: slice, *, float_dtype="F32", int4_dtype="U8") -> list:
    """Tensors of rows `rows` of a row-major host linear in its stored form."""
    inn = lin["in"]
    w = lin["w"][rows]
    n = w.shape[0]
    if wfmt == O.W_F32:
        return [(base + ".weight", float_dtype, (n, inn), _float_tensor(w, float_dtype), None)]
    if wfmt == O.W_I8PC:
        return [(base + ".weight", "I8", (n, inn), np.ascontiguousarray(w, np.int8).tobytes(), None),
                (base + ".weight_scale", "F16", (n,), np.ascontiguousarray(lin["scale"][rows], np.uint16).tobytes(),
                 None)]
    shape = (n, inn // 2) if int4_dtype == "U8" else (n, inn)
    g = inn // 128
    return [(base + ".weight", int4_dtype, shape, np.ascontiguousarray(w, np.uint8).tobytes(), None),
            (base + ".weight_scale", "BF16", (n, g), np.ascontiguousarray(lin["scale"][rows], np.uint16).tobytes(), None),
            (base + ".weight_zero", "BF16", (n, g), np.ascontiguousarray(lin["zero"][rows], np.uint16).tobytes(), None)]


def config_of(m: O.HostModel, **over) -> dict:
    c = m.cfg
    cfg = {"architectures": ["LlamaForCausalLM"], "model_type": "llama", "hidden_act": "silu",
           "vocab_size": c["vocab"], "hidden_size": c["hidden"], "intermediate_size": c["ffn"],
           "num_hidden_layers": c["n_layers"], "num_attention_heads": c["n_heads"],
           "num_key_value_heads": c["n_kv_heads"], "head_dim": c["head_dim"],
           "max_position_embeddings": c["max_pos"], "rms_norm_eps": c["rms_eps"], "rope_theta": c.get("theta", 1e4),
           "tie_word_embeddings": bool(c["tied"]), "torch_dtype": "float32"}
    if c["wfmt"] != O.W_F32:
        cfg["quantization_config"] = {
            "quant_method": "opure",
            "weight_format": "int8_per_channel" if c["wfmt"] == O.W_I8PC else "int4_g128",
            "activation_dtype": {O.A_F16: "float16", O.A_BF16: "bfloat16", O.A_F32: "float32"}[c["afmt"]]}
    cfg.update(over)
    return cfg


def model_tensors(m: O.HostModel, *, float_dtype="F32", int4_dtype="U8", norm_dtype="F32") -> list:
    c = m.cfg
    wf = c["wfmt"]
    nh, nkv, hd, ff = c["n_heads"], c["n_kv_heads"], c["head_dim"], c["ffn"]
    kw = dict(float_dtype=float_dtype, int4_dtype=int4_dtype)
    all_rows = slice(None)
    t = linear_tensors("model.embed_tokens", m.embed, wf, all_rows, **kw)
    for i, L in enumerate(m.layers):
        p = f"model.layers.{i}."
        t.append((p + "input_layernorm.weight", norm_dtype, (c["hidden"],), _float_tensor(L["attn_norm"], norm_dtype),
                  None))
        t.append((p + "post_attention_layernorm.weight", norm_dtype, (c["hidden"],),
                  _float_tensor(L["mlp_norm"], norm_dtype), None))
        q, k = nh * hd, nkv * hd
        t += linear_tensors(p + "self_attn.q_proj", L["qkv"], wf, slice(0, q), **kw)
        t += linear_tensors(p + "self_attn.k_proj", L["qkv"], wf, slice(q, q + k), **kw)
        t += linear_tensors(p + "self_attn.v_proj", L["qkv"], wf, slice(q + k, q + 2 * k), **kw)
        t += linear_tensors(p + "self_attn.o_proj", L["o"], wf, all_rows, **kw)
        t += linear_tensors(p + "mlp.gate_proj", L["gate_up"], wf, slice(0, ff), **kw)
        t += linear_tensors(p + "mlp.up_proj", L["gate_up"], wf, slice(ff, 2 * ff), **kw)
        t += linear_tensors(p + "mlp.down_proj", L["down"], wf, all_rows, **kw)
    t.append(("model.norm.weight", norm_dtype, (c["hidden"],), _float_tensor(m.final_norm, norm_dtype), None))
    if not c["tied"]:
        t += linear_tensors("lm_head", m.lm_head, wf, all_rows, **kw)
    return t


def write_model_dir(d: str, m: O.HostModel, *, config_over: dict | None = None, shards: int = 1,
                    **tensor_kw) -> str:
    """config.json and model.safetensors (shards > 1: model-0000i-of-0000n
    files plus model.safetensors.index.json) for host model m."""
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(config_of(m, **(config_over or {})), f, indent=2)
    t = model_tensors(m, **tensor_kw)
    if shards == 1:
        write_safetensors(os.path.join(d, "model.safetensors"), t, {"format": "pt"})
        return d
    per = (len(t) + shards - 1) // shards
    wmap = {}
    for s in range(shards):
        name = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        part = t[s * per:(s + 1) * per]
        write_safetensors(os.path.join(d, name), part, {"format": "pt"})
        wmap.update({e[0]: name for e in part})
    with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wmap}, f)
    return d
