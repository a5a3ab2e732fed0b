"""Seeded synthetic models built on the device through the C-ABI.

Every linear is drawn N(0, 0.02) from Philox (seed, tensor id) by
opure_synth_normal_f32 and quantised on the device (per-channel int8 with fp16
scales, or group-128 uint4 with bf16 scale/zero), so a full 1B or 8B-shaped
model never needs a host copy.  Norm gains are 1 (the HF initialisation).
`download()` returns the same host layout the CPU oracle consumes.

Configurations (the workloads the verify path is measured on):
  c1  SmolLM-135M shape, fp32, 30 layers (+ a 2-layer draft), K=4
  c3  Llama-3.2-1B shape, int8 per-channel / fp16, K=5, 2048-token context
  c4  Llama-3-8B shape, int4 group-128 / bf16, K=7, 8192-token context
  c5  c3's weights, batch of sequences with ragged contexts, K=6
"""
from __future__ import annotations

import ctypes as C

import numpy as np

import opure_hip as H

CONFIGS = {
    "c1": dict(n_layers=30, hidden=576, n_heads=9, n_kv_heads=3, head_dim=64, ffn=1536, vocab=49152,
               wfmt=H.W_F32, afmt=H.A_F32, rms_eps=1e-5, attn_scale=1.0, theta=10000.0, tied=True,
               K=4, ctx=32, batch=1),
    "c3": dict(n_layers=16, hidden=2048, n_heads=32, n_kv_heads=8, head_dim=64, ffn=8192, vocab=128256,
               wfmt=H.W_I8PC, afmt=H.A_F16, rms_eps=1e-5, attn_scale=64 ** -0.5, theta=500000.0, tied=True,
               K=5, ctx=2048, batch=1),
    "c4": dict(n_layers=32, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
               wfmt=H.W_I4G128, afmt=H.A_BF16, rms_eps=1e-5, attn_scale=128 ** -0.5, theta=500000.0, tied=False,
               K=7, ctx=8192, batch=1),
}


def linear_bytes(wfmt: int, out: int, inn: int) -> int:
    if wfmt == H.W_F32:
        return out * inn * 4
    if wfmt == H.W_I8PC:
        return out * inn + out * 2
    return out * inn // 2 + 2 * out * (inn // 128) * 2


def verify_bytes(cfg: dict, rows: int, ctx: int) -> dict:
    """Algorithmic HBM bytes of one verify step of `rows` rows (all sequences
    together) over `ctx` cached tokens per sequence: every weight once (the LM
    head reads its whole table, the embedding gather only `rows` rows when
    untied), the K/V of every cached position once per layer plus the rows'
    own K/V written, and the fp32 logits written once."""
    h, nh, nkv, hd, ff, V, L = (cfg[k] for k in ("hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab",
                                                   "n_layers"))
    w = cfg["wfmt"]
    layer = (linear_bytes(w, (nh + 2 * nkv) * hd, h) + linear_bytes(w, h, nh * hd) +
             linear_bytes(w, 2 * ff, h) + linear_bytes(w, h, ff) + 2 * h * 4)
    head = linear_bytes(w, V, h)
    gather = 0 if cfg["tied"] else rows * linear_bytes(w, 1, h)
    weights = L * layer + head + gather + h * 4
    eb = 4 if cfg["afmt"] == H.A_F32 else 2
    kv = L * 2 * nkv * hd * eb * (ctx + rows)
    logits = rows * V * 4
    return dict(weights=weights, kv=kv, logits=logits, total=weights + kv + logits)


class SynthModel:
    def __init__(self, dev: H.Dev, cfg: dict, seed: int = 1234, max_pos: int = 4096):
        self.dev, self.cfg, self.seed = dev, dict(cfg), seed
        c = self.cfg
        h, nh, nkv, hd, ff, V = c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["ffn"], c["vocab"]
        self.shapes = {"qkv": ((nh + 2 * nkv) * hd, h), "o": (h, nh * hd), "gate_up": (2 * ff, h), "down": (h, ff)}
        biggest = max([V * h] + [a * b for a, b in self.shapes.values()])
        self._tmp = dev.alloc(biggest * 4) if c["wfmt"] != H.W_F32 else None
        self.embed = self._linear(V, h, 0)
        self.lm_head = self.embed if c["tied"] else self._linear(V, h, 1)
        self.layers = []
        for L in range(c["n_layers"]):
            d = {"attn_norm": self._ones(h), "mlp_norm": self._ones(h)}
            for j, name in enumerate(("qkv", "o", "gate_up", "down")):
                d[name] = self._linear(*self.shapes[name], 2 + 4 * L + j,
                                       H.LAYOUT_TILED_SWIGLU if name == "gate_up" else H.LAYOUT_TILED)
            self.layers.append(d)
        self.final_norm = self._ones(h)
        cos, sin = H.rope_table(c["theta"], hd, max_pos, H.ROPE_GPU)
        self.rope_cos, self.rope_sin = dev.upload(cos), dev.upload(sin)
        self.max_pos = max_pos
        if self._tmp is not None:
            self._tmp.free()
            self._tmp = None
        dev.sync()
        self._desc()

    def _ones(self, n):
        b = self.dev.alloc(n * 4)
        self.dev.fill_u32(b, 0x3F800000, n)
        return b

    def _linear(self, out, inn, tid, layout=H.LAYOUT_TILED):
        """Seeded weights, quantised on the device in the row-major interchange
        layout (kept for downloads), plus the tiled copy the kernels read."""
        dev, w = self.dev, self.cfg["wfmt"]
        L = H.lib()
        if w == H.W_F32:
            wb = dev.alloc(out * inn * 4)
            H.check(L.opure_synth_normal_f32(dev.h, int(wb), out * inn, self.seed, tid, 0.02, 0.0))
            d = {"w": wb, "scale": None, "zero": None, "out": out, "in": inn}
        else:
            H.check(L.opure_synth_normal_f32(dev.h, int(self._tmp), out * inn, self.seed, tid, 0.02, 0.0))
            if w == H.W_I8PC:
                q, s = dev.alloc(out * inn), dev.alloc(out * 2)
                H.check(L.opure_quantize_i8pc(dev.h, int(self._tmp), out, inn, int(q), int(s)))
                d = {"w": q, "scale": s, "zero": None, "out": out, "in": inn}
            else:
                q, s, z = dev.alloc(out * inn // 2), dev.alloc(out * (inn // 128) * 2), dev.alloc(out * (inn // 128) * 2)
                H.check(L.opure_quantize_i4g128(dev.h, int(self._tmp), out, inn, int(q), int(s), int(z)))
                d = {"w": q, "scale": s, "zero": z, "out": out, "in": inn}
        d["tiled"], d["tiled_bufs"] = dev.tile(w, self._rowmajor(d), layout)
        return d

    @staticmethod
    def _rowmajor(d):
        return H.Linear(int(d["w"]), int(d["scale"]) if d["scale"] else None, int(d["zero"]) if d["zero"] else None,
                        d["out"], d["in"], H.LAYOUT_ROWMAJOR)

    @staticmethod
    def _lin(d):
        return d["tiled"]

    def _desc(self):
        c = self.cfg
        n = c["n_layers"]
        self._layers = (H.LayerWeights * n)()
        for i, d in enumerate(self.layers):
            self._layers[i] = H.LayerWeights(int(d["attn_norm"]), int(d["mlp_norm"]), self._lin(d["qkv"]),
                                             self._lin(d["o"]), self._lin(d["gate_up"]), self._lin(d["down"]))
        self.desc = H.Model(n, c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["ffn"], c["vocab"],
                            c["rms_eps"], c["attn_scale"], c["wfmt"], c["afmt"], int(self.rope_cos),
                            int(self.rope_sin), self.max_pos, self._lin(self.embed), self._lin(self.lm_head),
                            int(self.final_norm), C.cast(self._layers, C.POINTER(H.LayerWeights)))

    # ---- host copies for the CPU oracle ------------------------------------
    def _dl_linear(self, d):
        w = self.cfg["wfmt"]
        out, inn = d["out"], d["in"]
        r = {"out": out, "in": inn, "scale": None, "zero": None}
        if w == H.W_F32:
            r["w"] = self.dev.download(d["w"], np.float32, (out, inn))
        elif w == H.W_I8PC:
            r["w"] = self.dev.download(d["w"], np.int8, (out, inn))
            r["scale"] = self.dev.download(d["scale"], np.uint16, (out,))
        else:
            r["w"] = self.dev.download(d["w"], np.uint8, (out, inn // 2))
            r["scale"] = self.dev.download(d["scale"], np.uint16, (out, inn // 128))
            r["zero"] = self.dev.download(d["zero"], np.uint16, (out, inn // 128))
        return r

    def download(self) -> dict:
        c = self.cfg
        h = c["hidden"]
        emb = self._dl_linear(self.embed)
        out = {"embed": emb, "lm_head": emb if c["tied"] else self._dl_linear(self.lm_head),
               "final_norm": self.dev.download(self.final_norm, np.float32, (h,)),
               "rope_cos": self.dev.download(self.rope_cos, np.float32, (self.max_pos, c["head_dim"] // 2)),
               "rope_sin": self.dev.download(self.rope_sin, np.float32, (self.max_pos, c["head_dim"] // 2)),
               "layers": []}
        for d in self.layers:
            out["layers"].append({"attn_norm": self.dev.download(d["attn_norm"], np.float32, (h,)),
                                  "mlp_norm": self.dev.download(d["mlp_norm"], np.float32, (h,)),
                                  **{k: self._dl_linear(d[k]) for k in ("qkv", "o", "gate_up", "down")}})
        return out


def stage_bytes(cfg, stage, M, ctx):
    """Algorithmic HBM bytes of one launch of a verify-step stage for M rows
    over a ctx-token cache: the weights once, activations in and out once."""
    h, nh, nkv, hd, ff, V = (cfg[k] for k in ("hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab"))
    w = cfg["wfmt"]
    eb = 4 if cfg["afmt"] == H.A_F32 else 2
    qkv_out = (nh + 2 * nkv) * hd
    if stage == "embed":
        return M * linear_bytes(w, 1, h) + M * h * 4
    if stage == "qkv":      # fp32 residual + gain in, q out, K/V rows appended
        return linear_bytes(w, qkv_out, h) + M * h * 4 + h * 4 + M * qkv_out * eb
    if stage == "attention":
        return 2 * nkv * hd * eb * (ctx + M) + 2 * M * nh * hd * eb
    if stage == "o_proj":   # attention output in, residual read and written
        return linear_bytes(w, h, nh * hd) + M * nh * hd * eb + 2 * M * h * 4
    if stage == "gate_up":  # residual + gain in, SwiGLU output out
        return linear_bytes(w, 2 * ff, h) + M * h * 4 + h * 4 + M * ff * eb
    if stage == "down":
        return linear_bytes(w, h, ff) + M * ff * eb + 2 * M * h * 4
    if stage == "lm_head":  # fp32 logits out
        return linear_bytes(w, V, h) + M * h * 4 + h * 4 + M * V * 4
    return 0
