"""ctypes binding for the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product path.

The structures mirror oracle/opure_oracle.h.  `HostModel` holds a model's host
arrays (numpy) and builds the orc_model descriptor over them; the same arrays
are what a test uploads to the device, so both sides see identical inputs.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# OPURE_ORACLE_LIB: another build of the same sources (the sanitizer test's)
LIB_PATH = os.environ.get("OPURE_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

W_F32, W_I8PC, W_I4G128 = 0, 1, 2
A_F32, A_F16, A_BF16 = 0, 1, 2
ROPE_GPU, ROPE_CPUREF = 0, 1


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class OrcLinear(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scale", C.c_void_p), ("zero", C.c_void_p),
                ("out", C.c_uint32), ("in_", C.c_uint32)]


class OrcLayer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("mlp_norm", C.c_void_p), ("qkv", OrcLinear),
                ("o", OrcLinear), ("gate_up", OrcLinear), ("down", OrcLinear)]


class OrcModel(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("hidden", C.c_uint32), ("n_heads", C.c_uint32),
                ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("ffn", C.c_uint32),
                ("vocab", C.c_uint32), ("rms_eps", C.c_float), ("attn_scale", C.c_float),
                ("wfmt", C.c_uint32), ("afmt", C.c_uint32), ("rope_cos", C.c_void_p),
                ("rope_sin", C.c_void_p), ("rope_max_pos", C.c_uint32), ("embed", OrcLinear),
                ("lm_head", OrcLinear), ("final_norm", C.c_void_p), ("layers", C.POINTER(OrcLayer))]


class OrcKV(C.Structure):
    _fields_ = [("pool", C.c_void_p), ("n_pages", C.c_uint32), ("page_size", C.c_uint32),
                ("page_table", C.c_void_p), ("max_pages_per_seq", C.c_uint32)]


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _declare(L):
    vp, u32, u64, f32, i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float, C.c_int32
    L.orc_f16_to_f32.argtypes = [C.c_uint16]; L.orc_f16_to_f32.restype = f32
    L.orc_f32_to_f16.argtypes = [f32]; L.orc_f32_to_f16.restype = C.c_uint16
    L.orc_bf16_to_f32.argtypes = [C.c_uint16]; L.orc_bf16_to_f32.restype = f32
    L.orc_f32_to_bf16.argtypes = [f32]; L.orc_f32_to_bf16.restype = C.c_uint16
    L.orc_expf.argtypes = [f32]; L.orc_expf.restype = f32
    L.orc_philox4x32_10.argtypes = [vp, vp, vp]; L.orc_philox4x32_10.restype = None
    L.orc_philox_u32.argtypes = [u64, u32, u32, u32]; L.orc_philox_u32.restype = u32
    L.orc_xorshift_fill.argtypes = [u64, vp, u64, f32, f32]; L.orc_xorshift_fill.restype = None
    L.orc_xorshift_u32.argtypes = [u64, vp, u64]; L.orc_xorshift_u32.restype = None
    L.orc_set_threads.argtypes = [C.c_int]; L.orc_set_threads.restype = None
    L.orc_gemv.argtypes = [C.POINTER(OrcLinear), u32, vp, vp, u32]; L.orc_gemv.restype = None
    L.orc_rmsnorm_rows.argtypes = [vp, vp, vp, u32, u32, f32, u32]; L.orc_rmsnorm_rows.restype = None
    L.orc_round_act.argtypes = [vp, u64, u32]; L.orc_round_act.restype = None
    L.orc_rope_table.argtypes = [C.c_double, u32, u32, u32, vp, vp]; L.orc_rope_table.restype = None
    L.orc_rope_rows.argtypes = [vp, u32, u32, vp, vp, u32]; L.orc_rope_rows.restype = None
    L.orc_swiglu.argtypes = [vp, vp, vp, u64]; L.orc_swiglu.restype = None
    L.orc_attention_paged.argtypes = [C.POINTER(OrcModel), C.POINTER(OrcKV), u32, u32, u32, u32, vp, vp]
    L.orc_attention_paged.restype = None
    L.orc_verify_forward.argtypes = [C.POINTER(OrcModel), C.POINTER(OrcKV), u32, u32, vp, vp, vp]
    L.orc_verify_forward.restype = C.c_int
    L.orc_verify_forward_traced.argtypes = [C.POINTER(OrcModel), C.POINTER(OrcKV), u32, u32, vp, vp, vp, vp]
    L.orc_verify_forward_traced.restype = C.c_int
    L.orc_verify_embed.argtypes = [C.POINTER(OrcModel), u32, vp, vp]; L.orc_verify_embed.restype = C.c_int
    L.orc_verify_layers.argtypes = [C.POINTER(OrcModel), C.POINTER(OrcKV), u32, u32, vp, vp, u32, u32]
    L.orc_verify_layers.restype = C.c_int
    L.orc_verify_head.argtypes = [C.POINTER(OrcModel), u32, vp, vp]; L.orc_verify_head.restype = C.c_int
    L.orc_set_perturbation.argtypes = [C.c_int32, u32, u64]; L.orc_set_perturbation.restype = None
    L.orc_argmax_rows.argtypes = [vp, u32, u32, vp, vp]; L.orc_argmax_rows.restype = None
    L.orc_accept_greedy.argtypes = [vp, vp, u32, u32, u32, vp, vp]; L.orc_accept_greedy.restype = None
    L.orc_accept_rejection.argtypes = [vp, vp, vp, u32, u32, u32, f32, u64, vp, vp, vp, vp]
    L.orc_accept_rejection.restype = None
    L.orc_sample_rows.argtypes = [vp, u32, u32, f32, u64, vp, vp, u32, vp]; L.orc_sample_rows.restype = None
    L.orc_kv_rollback.argtypes = [C.POINTER(OrcKV), C.POINTER(OrcModel), u32, u32, vp, vp, vp, vp, vp,
                                  u32, vp, u32]
    L.orc_kv_rollback.restype = None
    del i32


# ---------------------------------------------------------------------------
#  scalar helpers
# ---------------------------------------------------------------------------
def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    L = lib()
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([L.orc_f32_to_f16(float(v)) for v in x], dtype=np.uint16)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    L = lib()
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([L.orc_f32_to_bf16(float(v)) for v in x], dtype=np.uint16)


def philox(ctr, key):
    c = np.asarray(ctr, dtype=np.uint32)
    k = np.asarray(key, dtype=np.uint32)
    o = np.zeros(4, dtype=np.uint32)
    lib().orc_philox4x32_10(_p(c), _p(k), _p(o))
    return o


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def rope_table(theta: float, head_dim: int, max_pos: int, mode: int = ROPE_GPU):
    cos = np.zeros((max_pos, head_dim // 2), dtype=np.float32)
    sin = np.zeros_like(cos)
    lib().orc_rope_table(float(theta), head_dim, max_pos, mode, _p(cos), _p(sin))
    return cos, sin


def linear(w, scale=None, zero=None, out=0, in_=0) -> OrcLinear:
    return OrcLinear(_p(w), _p(scale), _p(zero), out, in_)


def gemv(lin: dict, wfmt: int, x: np.ndarray) -> np.ndarray:
    """y[m, o] = sum_i W[o, i] x[m, i] for a linear dict {w, scale, zero, out, in}."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.shape[0]
    y = np.zeros((M, lin["out"]), dtype=np.float32)
    L = linear(lin["w"], lin.get("scale"), lin.get("zero"), lin["out"], lin["in"])
    lib().orc_gemv(C.byref(L), wfmt, _p(x), _p(y), M)
    return y


# ---------------------------------------------------------------------------
#  quantisers (test-data generation)
# ---------------------------------------------------------------------------
def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def np_f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def quant_i8pc(w: np.ndarray):
    """Symmetric per-output-row int8 with an fp16 scale: w ~= scale[o] * q[o, i]."""
    w = np.asarray(w, dtype=np.float32)
    amax = np.abs(w).max(axis=1)
    s16 = (np.maximum(amax, 1e-8) / 127.0).astype(np.float16)
    # a row too small for an fp16 scale (an all-zero row) gets the smallest
    # positive one, so its codes are 0 rather than 0/0
    s16[s16 == 0] = np.uint16(1).view(np.float16)
    s = s16.astype(np.float32)
    q = np.clip(np.rint(w / s[:, None]), -127, 127).astype(np.int8)
    return {"w": np.ascontiguousarray(q), "scale": s16.view(np.uint16).copy(), "zero": None,
            "out": w.shape[0], "in": w.shape[1]}


def quant_i4g128(w: np.ndarray):
    """Asymmetric group-128 uint4 along the input axis with bf16 scale and zero:
    w ~= scale[o, g] * (q[o, i] - zero[o, g]).  Element 2j is the high nibble."""
    w = np.asarray(w, dtype=np.float32)
    O, K = w.shape
    assert K % 128 == 0
    g = w.reshape(O, K // 128, 128)
    mn, mx = g.min(axis=2), g.max(axis=2)
    s_b = np_f32_to_bf16_bits(np.maximum(mx - mn, 1e-8) / 15.0)
    s = bf16_bits_to_f32(s_b)
    z_b = np_f32_to_bf16_bits(-mn / s)
    z = bf16_bits_to_f32(z_b)
    q = np.clip(np.rint(g / s[..., None] + z[..., None]), 0, 15).astype(np.uint8).reshape(O, K)
    packed = ((q[:, 0::2] << 4) | q[:, 1::2]).astype(np.uint8)
    return {"w": np.ascontiguousarray(packed), "scale": s_b.reshape(O, K // 128).copy(),
            "zero": z_b.reshape(O, K // 128).copy(), "out": O, "in": K}


def dequant(lin: dict, wfmt: int) -> np.ndarray:
    if wfmt == W_F32:
        return lin["w"].astype(np.float64)
    if wfmt == W_I8PC:
        return lin["w"].astype(np.float64) * f16_bits_to_f32(lin["scale"]).astype(np.float64)[:, None]
    O, K = lin["out"], lin["in"]
    p = lin["w"]
    q = np.empty((O, K), dtype=np.float64)
    q[:, 0::2] = p >> 4
    q[:, 1::2] = p & 15
    s = np.repeat(bf16_bits_to_f32(lin["scale"]).astype(np.float64), 128, axis=1)
    z = np.repeat(bf16_bits_to_f32(lin["zero"]).astype(np.float64), 128, axis=1)
    return s * (q - z)


def make_linear(rng: np.random.Generator, out: int, in_: int, wfmt: int, std: float = 0.02):
    w = rng.standard_normal((out, in_), dtype=np.float32) * np.float32(std)
    if wfmt == W_F32:
        return {"w": np.ascontiguousarray(w), "scale": None, "zero": None, "out": out, "in": in_}
    if wfmt == W_I8PC:
        return quant_i8pc(w)
    return quant_i4g128(w)


# ---------------------------------------------------------------------------
#  model + KV cache on the host
# ---------------------------------------------------------------------------
class HostModel:
    """Seeded synthetic model: linears ~ N(0, 0.02), norm gains = 1."""

    def __init__(self, *, n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab,
                 wfmt=W_F32, afmt=A_F32, rms_eps=1e-5, attn_scale=1.0, theta=10000.0,
                 rope_mode=ROPE_GPU, max_pos=4096, tied=True, seed=1234, norm_jitter=0.0):
        self.cfg = dict(n_layers=n_layers, hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv_heads,
                        head_dim=head_dim, ffn=ffn, vocab=vocab, wfmt=wfmt, afmt=afmt,
                        rms_eps=rms_eps, attn_scale=attn_scale, theta=theta, rope_mode=rope_mode,
                        max_pos=max_pos, tied=tied, seed=seed)
        rng = np.random.default_rng(seed)
        qkv_out = (n_heads + 2 * n_kv_heads) * head_dim
        self.embed = make_linear(rng, vocab, hidden, wfmt)
        self.lm_head = self.embed if tied else make_linear(rng, vocab, hidden, wfmt)

        def gain():
            g = np.ones(hidden, dtype=np.float32)
            if norm_jitter:
                g += (rng.standard_normal(hidden, dtype=np.float32) * np.float32(norm_jitter))
            return g

        self.final_norm = gain()
        self.layers = []
        for _ in range(n_layers):
            self.layers.append(dict(
                attn_norm=gain(), mlp_norm=gain(),
                qkv=make_linear(rng, qkv_out, hidden, wfmt),
                o=make_linear(rng, hidden, n_heads * head_dim, wfmt),
                gate_up=make_linear(rng, 2 * ffn, hidden, wfmt),
                down=make_linear(rng, hidden, ffn, wfmt)))
        self.rope_cos, self.rope_sin = rope_table(theta, head_dim, max_pos, rope_mode)
        self._build()

    @classmethod
    def from_arrays(cls, cfg: dict, w: dict) -> "HostModel":
        """Wraps host arrays (e.g. downloaded from the device) as an oracle model."""
        self = cls.__new__(cls)
        keys = ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab", "wfmt", "afmt",
                "rms_eps", "attn_scale")
        self.cfg = {k: cfg[k] for k in keys}
        self.cfg["max_pos"] = w["rope_cos"].shape[0]
        self.cfg["tied"] = w["lm_head"] is w["embed"]
        self.embed, self.lm_head, self.final_norm = w["embed"], w["lm_head"], w["final_norm"]
        self.layers, self.rope_cos, self.rope_sin = w["layers"], w["rope_cos"], w["rope_sin"]
        self._build()
        return self

    def _build(self):
        c = self.cfg

        def lin(d):
            return linear(d["w"], d.get("scale"), d.get("zero"), d["out"], d["in"])

        self._layers = (OrcLayer * c["n_layers"])()
        for i, Ld in enumerate(self.layers):
            self._layers[i] = OrcLayer(_p(Ld["attn_norm"]), _p(Ld["mlp_norm"]), lin(Ld["qkv"]),
                                       lin(Ld["o"]), lin(Ld["gate_up"]), lin(Ld["down"]))
        self.desc = OrcModel(c["n_layers"], c["hidden"], c["n_heads"], c["n_kv_heads"], c["head_dim"],
                             c["ffn"], c["vocab"], c["rms_eps"], c["attn_scale"], c["wfmt"], c["afmt"],
                             _p(self.rope_cos), _p(self.rope_sin), c["max_pos"], lin(self.embed),
                             lin(self.lm_head), _p(self.final_norm),
                             C.cast(self._layers, C.POINTER(OrcLayer)))


def act_np_dtype(afmt: int):
    return np.float32 if afmt == A_F32 else np.uint16


def kv_planes(pool):
    """Logical (K, V) views [layers][pages][kv_heads][page_size][head_dim] of a
    paged pool.  K planes are stored token-major, V planes channel-major
    ([head_dim][page_size]), so V is a transposed view; both are writable."""
    K = pool[:, :, 0]
    L, P, nkv, ps, hd = K.shape
    V = pool[:, :, 1].reshape(L, P, nkv, hd, ps).swapaxes(-1, -2)
    return K, V


class HostKV:
    """Paged cache [n_layers][n_pages][2][n_kv][page][hd] with per-sequence page tables."""

    def __init__(self, model: HostModel, n_pages: int, batch: int, max_pages_per_seq: int,
                 page_size: int = 16):
        c = model.cfg
        self.model = model
        self.page_size = page_size
        self.n_pages = n_pages
        self.batch = batch
        self.max_pages = max_pages_per_seq
        shape = (c["n_layers"], n_pages, 2, c["n_kv_heads"], page_size, c["head_dim"])
        self.pool = np.zeros(shape, dtype=act_np_dtype(c["afmt"]))
        self.page_table = np.full((batch, max_pages_per_seq), -1, dtype=np.int32)
        self._mk()

    def _mk(self):
        self.desc = OrcKV(_p(self.pool), self.n_pages, self.page_size, _p(self.page_table), self.max_pages)

    def fill_random(self, rng: np.random.Generator, std: float = 1.0):
        afmt = self.model.cfg["afmt"]
        v = rng.standard_normal(self.pool.shape, dtype=np.float32) * np.float32(std)
        if afmt == A_F32:
            self.pool[...] = v
        elif afmt == A_F16:
            self.pool[...] = v.astype(np.float16).view(np.uint16)
        else:
            self.pool[...] = np_f32_to_bf16_bits(v).reshape(self.pool.shape)


def verify_forward(model: HostModel, kv: HostKV, tokens: np.ndarray, seq_len: np.ndarray) -> np.ndarray:
    tokens = np.ascontiguousarray(tokens, dtype=np.int32)
    seq_len = np.ascontiguousarray(seq_len, dtype=np.int32)
    B, R = tokens.shape
    logits = np.zeros((B, R, model.cfg["vocab"]), dtype=np.float32)
    kv._mk()
    rc = lib().orc_verify_forward(C.byref(model.desc), C.byref(kv.desc), B, R, _p(tokens), _p(seq_len),
                                  _p(logits))
    if rc != 0:
        raise ValueError(f"orc_verify_forward failed: {rc}")
    return logits


STAGE_XN_ATTN, STAGE_Q, STAGE_ATT, STAGE_XN_MLP, STAGE_H = 0, 1, 2, 3, 4


def verify_embed(model: HostModel, tokens: np.ndarray) -> np.ndarray:
    """fp32 residual [B*R][hidden] of the embedding rows of `tokens`."""
    t = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
    x = np.zeros((t.size, model.cfg["hidden"]), dtype=np.float32)
    rc = lib().orc_verify_embed(C.byref(model.desc), t.size, _p(t), _p(x))
    if rc != 0:
        raise ValueError(f"orc_verify_embed failed: {rc}")
    return x


def verify_layers(model: HostModel, kv: HostKV, x: np.ndarray, seq_len, R: int, first: int, count: int) -> np.ndarray:
    """Applies layers [first, first+count) to a copy of residual x ([B*R][hidden]),
    appending the rows' K/V to the cache; returns the new residual."""
    seq_len = np.ascontiguousarray(seq_len, dtype=np.int32)
    x = np.array(x, dtype=np.float32, order="C", copy=True)
    kv._mk()
    rc = lib().orc_verify_layers(C.byref(model.desc), C.byref(kv.desc), seq_len.size, R, _p(seq_len), _p(x), first,
                                 count)
    if rc != 0:
        raise ValueError(f"orc_verify_layers failed: {rc}")
    return x


def verify_head(model: HostModel, x: np.ndarray) -> np.ndarray:
    """Final RMSNorm + LM head of residual rows x: logits [rows][vocab]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros((x.shape[0], model.cfg["vocab"]), dtype=np.float32)
    rc = lib().orc_verify_head(C.byref(model.desc), x.shape[0], _p(x), _p(out))
    if rc != 0:
        raise ValueError(f"orc_verify_head failed: {rc}")
    return out


def set_perturbation(layer: int = -1, stage: int = 0, index: int = 0) -> None:
    """One element of one rounded intermediate moved by one ulp (layer < 0: off)."""
    lib().orc_set_perturbation(int(layer), int(stage), int(index))


def verify_forward_traced(model: HostModel, kv: HostKV, tokens: np.ndarray, seq_len: np.ndarray):
    """Returns logits and layer 0's intermediates {q, att, x_attn, h, x_layer, xn_final}."""
    c = model.cfg
    tokens = np.ascontiguousarray(tokens, dtype=np.int32)
    seq_len = np.ascontiguousarray(seq_len, dtype=np.int32)
    B, R = tokens.shape
    MR = B * R
    qd, h, ff = c["n_heads"] * c["head_dim"], c["hidden"], c["ffn"]
    sizes = [("q", qd), ("att", qd), ("x_attn", h), ("h", ff), ("x_layer", h), ("xn_final", h)]
    trace = np.zeros(sum(MR * w for _, w in sizes), dtype=np.float32)
    logits = np.zeros((B, R, c["vocab"]), dtype=np.float32)
    kv._mk()
    rc = lib().orc_verify_forward_traced(C.byref(model.desc), C.byref(kv.desc), B, R, _p(tokens), _p(seq_len),
                                         _p(logits), _p(trace))
    if rc != 0:
        raise ValueError(f"orc_verify_forward_traced failed: {rc}")
    out, off = {}, 0
    for name, w in sizes:
        out[name] = trace[off:off + MR * w].reshape(MR, w)
        off += MR * w
    return logits, out


def accept_greedy(target_logits: np.ndarray, drafts: np.ndarray):
    t = np.ascontiguousarray(target_logits, dtype=np.float32)
    d = np.ascontiguousarray(drafts, dtype=np.int32)
    B, K1, V = t.shape
    out = np.zeros((B, K1), dtype=np.int32)
    acc = np.zeros(B, dtype=np.int32)
    lib().orc_accept_greedy(_p(t), _p(d), B, K1 - 1, V, _p(out), _p(acc))
    return out, acc


def accept_rejection(target_logits, draft_logits, drafts, temperature, seed, pos_base=None):
    t = np.ascontiguousarray(target_logits, dtype=np.float32)
    q = np.ascontiguousarray(draft_logits, dtype=np.float32)
    d = np.ascontiguousarray(drafts, dtype=np.int32)
    B, K1, V = t.shape
    pb = None if pos_base is None else np.ascontiguousarray(pos_base, dtype=np.uint32)
    out = np.zeros((B, K1), dtype=np.int32)
    acc = np.zeros(B, dtype=np.int32)
    dist = np.zeros((B, V), dtype=np.float32)
    lib().orc_accept_rejection(_p(t), _p(q), _p(d), B, K1 - 1, V, float(temperature), int(seed), _p(pb),
                               _p(out), _p(acc), _p(dist))
    return out, acc, dist


def sample_rows(logits, temperature, seed, pos, seq, stream):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    rows, V = lg.shape
    p = np.ascontiguousarray(pos, dtype=np.uint32)
    s = np.ascontiguousarray(seq, dtype=np.uint32)
    out = np.zeros(rows, dtype=np.int32)
    lib().orc_sample_rows(_p(lg), rows, V, float(temperature), int(seed), _p(p), _p(s), stream, _p(out))
    return out


def kv_rollback(kv: HostKV, model: HostModel, K: int, seq_len, accepted, poison_bits=0, freed_stride=8):
    seq_len = np.ascontiguousarray(seq_len, dtype=np.int32)
    accepted = np.ascontiguousarray(accepted, dtype=np.int32)
    B = seq_len.shape[0]
    new_len = np.zeros(B, dtype=np.int32)
    freed = np.full((B, freed_stride), -1, dtype=np.int32)
    n_freed = np.zeros(B, dtype=np.int32)
    kv._mk()
    lib().orc_kv_rollback(C.byref(kv.desc), C.byref(model.desc), B, K, _p(seq_len), _p(accepted),
                          _p(kv.page_table), _p(new_len), _p(freed), freed_stride, _p(n_freed), poison_bits)
    return new_len, freed, n_freed
