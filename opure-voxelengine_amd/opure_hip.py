"""ctypes binding of the libopure_hip C-ABI (include/opure_hip.h).

This is the Python face of the boundary used by the tests and bench.py; the
structures mirror the header field for field.  Every call checks the return
code and raises OpureError with opure_last_error(); a missing library raises
at import of the binding's first use (there is no fallback path).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libopure_hip.so")

OK, E_INVALID, E_NODEVICE, E_HIP, E_OOM, E_UNSUPPORTED, E_CAPACITY, E_DEVICE = 0, -1, -2, -3, -4, -5, -6, -7
MAX_ROWS, PAGE_SIZE = 16, 16
W_F32, W_I8PC, W_I4G128 = 0, 1, 2
A_F32, A_F16, A_BF16 = 0, 1, 2
ROPE_GPU, ROPE_CPUREF = 0, 1
EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU = 0, 1, 2
STAGES = ("embed", "qkv", "attention", "o_proj", "gate_up", "down", "lm_head", "accept")
ACCEPT_NONE, ACCEPT_GREEDY, ACCEPT_REJECTION = 0, 1, 2
BW_READ, BW_COPY = 0, 1
GEMV_MFMA, GEMV_VALU = 0, 1
REJ_ONE_LAUNCH, REJ_STAGED = 0, 1
GREEDY_IN_LM_HEAD, GREEDY_SEPARATE = 0, 1


class OpureError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"opure error {code}: {msg}")
        self.code = code


LAYOUT_ROWMAJOR, LAYOUT_TILED, LAYOUT_TILED_SWIGLU = 0, 1, 2


class Linear(C.Structure):
    _fields_ = [("w", C.c_void_p), ("scale", C.c_void_p), ("zero", C.c_void_p),
                ("out", C.c_uint32), ("in_", C.c_uint32), ("layout", C.c_uint32)]


class LayerWeights(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("mlp_norm", C.c_void_p), ("qkv", Linear), ("o", Linear),
                ("gate_up", Linear), ("down", Linear)]


class Model(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("hidden", C.c_uint32), ("n_heads", C.c_uint32),
                ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("ffn", C.c_uint32),
                ("vocab", C.c_uint32), ("rms_eps", C.c_float), ("attn_scale", C.c_float),
                ("wfmt", C.c_uint32), ("afmt", C.c_uint32), ("rope_cos", C.c_void_p),
                ("rope_sin", C.c_void_p), ("rope_max_pos", C.c_uint32), ("embed", Linear),
                ("lm_head", Linear), ("final_norm", C.c_void_p), ("layers", C.POINTER(LayerWeights))]


class KV(C.Structure):
    _fields_ = [("pool", C.c_void_p), ("n_pages", C.c_uint32), ("page_size", C.c_uint32),
                ("page_table", C.c_void_p), ("max_pages_per_seq", C.c_uint32)]


class GemvArgs(C.Structure):
    _fields_ = [("W", Linear), ("x", C.c_void_p), ("y", C.c_void_p), ("M", C.c_uint32),
                ("xfmt", C.c_uint32), ("yfmt", C.c_uint32), ("epilogue", C.c_uint32)]


class AttnArgs(C.Structure):
    _fields_ = [("model", C.POINTER(Model)), ("kv", C.POINTER(KV)), ("layer", C.c_uint32),
                ("batch", C.c_uint32), ("rows", C.c_uint32), ("seq_len", C.c_void_p),
                ("max_ctx", C.c_uint32), ("q", C.c_void_p), ("out", C.c_void_p)]


class AcceptArgs(C.Structure):
    _fields_ = [("batch", C.c_uint32), ("k", C.c_uint32), ("vocab", C.c_uint32),
                ("target_logits", C.c_void_p), ("draft_logits", C.c_void_p), ("drafts", C.c_void_p),
                ("drafts_stride", C.c_uint32), ("temperature", C.c_float), ("seed", C.c_uint64),
                ("pos_base", C.c_void_p), ("out_tokens", C.c_void_p), ("accepted", C.c_void_p),
                ("dist_out", C.c_void_p)]


class SampleArgs(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("vocab", C.c_uint32), ("logits", C.c_void_p),
                ("temperature", C.c_float), ("seed", C.c_uint64), ("pos", C.c_void_p), ("seq", C.c_void_p),
                ("stream", C.c_uint32), ("out", C.c_void_p)]


class RollbackArgs(C.Structure):
    _fields_ = [("model", C.POINTER(Model)), ("kv", C.POINTER(KV)), ("batch", C.c_uint32), ("k", C.c_uint32),
                ("seq_len", C.c_void_p), ("accepted", C.c_void_p), ("new_seq_len", C.c_void_p),
                ("freed", C.c_void_p), ("freed_stride", C.c_uint32), ("n_freed", C.c_void_p),
                ("poison", C.c_uint32), ("poison_bits", C.c_uint32)]


class VerifyArgs(C.Structure):
    _fields_ = [("model", C.POINTER(Model)), ("kv", C.POINTER(KV)), ("batch", C.c_uint32),
                ("rows", C.c_uint32), ("tokens", C.c_void_p), ("seq_len", C.c_void_p),
                ("max_ctx", C.c_uint32), ("logits", C.c_void_p), ("accept_mode", C.c_uint32),
                ("draft_logits", C.c_void_p), ("temperature", C.c_float), ("seed", C.c_uint64),
                ("pos_base", C.c_void_p), ("out_tokens", C.c_void_p), ("accepted", C.c_void_p),
                ("dist_out", C.c_void_p), ("rollback", C.c_uint32), ("new_seq_len", C.c_void_p),
                ("freed", C.c_void_p), ("freed_stride", C.c_uint32), ("n_freed", C.c_void_p),
                ("poison", C.c_uint32), ("poison_bits", C.c_uint32)]


class VerifyLayerArgs(C.Structure):
    _fields_ = [("model", C.POINTER(Model)), ("kv", C.POINTER(KV)), ("layer", C.c_uint32), ("batch", C.c_uint32),
                ("rows", C.c_uint32), ("seq_len", C.c_void_p), ("max_ctx", C.c_uint32), ("x", C.c_void_p)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OpureError(E_INVALID, f"{LIB_PATH} is not built (run opure-voxelengine_amd/build.py)")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    vp, u32, u64, f32, i = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float, C.c_int
    sig = {
        "opure_dev_create": ([i, C.POINTER(vp)], i), "opure_dev_destroy": ([vp], i),
        "opure_dev_name": ([vp], C.c_char_p), "opure_dev_hbm_bytes": ([vp], u64),
        "opure_last_error": ([], C.c_char_p),
        "opure_buf_alloc": ([vp, u64, C.POINTER(vp)], i), "opure_buf_free": ([vp, vp], i),
        "opure_buf_upload": ([vp, vp, u64, vp, u64], i), "opure_buf_upload_ranges": ([vp, vp, u32], i),
        "opure_buf_download": ([vp, vp, vp, u64, u64], i), "opure_buf_fill_u32": ([vp, vp, u32, u64], i),
        "opure_buf_copy": ([vp, vp, vp, u64], i),
        "opure_stream_begin": ([vp], i), "opure_stream_sync": ([vp], i),
        "opure_graph_begin": ([vp], i), "opure_graph_end": ([vp, C.POINTER(vp)], i),
        "opure_graph_launch": ([vp, vp], i), "opure_graph_destroy": ([vp], i),
        "opure_timer_begin": ([vp], i), "opure_timer_end": ([vp], i),
        "opure_timer_ms": ([vp, C.POINTER(f32)], i),
        "opure_bw_measure": ([vp, u32, vp, vp, u64, u32, C.POINTER(C.c_double)], i),
        "opure_rope_table": ([C.c_double, u32, u32, u32, vp, vp], i),
        "opure_gemv_batched_f32": ([vp, C.POINTER(GemvArgs)], i),
        "opure_gemv_batched_i8pc": ([vp, C.POINTER(GemvArgs)], i),
        "opure_gemv_batched_i4g128": ([vp, C.POINTER(GemvArgs)], i),
        "opure_attn_decode_paged": ([vp, C.POINTER(AttnArgs)], i),
        "opure_accept_greedy": ([vp, C.POINTER(AcceptArgs)], i),
        "opure_accept_rejection": ([vp, C.POINTER(AcceptArgs)], i),
        "opure_accept_rejection_noalloc": ([vp, C.POINTER(AcceptArgs)], i),
        "opure_sample_rows": ([vp, C.POINTER(SampleArgs)], i),
        "opure_philox_uniform": ([vp, u64, vp, vp, u32, u32, vp], i),
        "opure_kv_rollback": ([vp, C.POINTER(RollbackArgs)], i),
        "opure_verify_reserve": ([vp, C.POINTER(Model), u32, u32, u32], i),
        "opure_verify_step": ([vp, C.POINTER(VerifyArgs)], i),
        "opure_verify_layer": ([vp, C.POINTER(VerifyLayerArgs)], i),
        "opure_debug_workspace": ([vp, C.POINTER(vp), C.POINTER(u64)], i),
        "opure_debug_set_wait_limit": ([vp, u32], i),
        "opure_debug_set_gemv_engine": ([vp, u32], i),
        "opure_debug_set_rejection_launches": ([vp, u32], i),
        "opure_debug_set_greedy_acceptance": ([vp, u32], i),
        "opure_debug_exp_check": ([vp, C.POINTER(u64)], i),
        "opure_debug_verify_offsets": ([C.POINTER(Model), u32, u32, u32, C.POINTER(u64)], i),
        "opure_tiled_bytes": ([u32, u32, u32, C.POINTER(u64), C.POINTER(u64)], i),
        "opure_tile_linear": ([vp, u32, u32, C.POINTER(Linear), vp, vp, C.POINTER(Linear)], i),
        "opure_profile_enable": ([vp, C.c_int], i),
        "opure_profile_read": ([vp, C.POINTER(u32), C.POINTER(C.c_double)], i),
        "opure_synth_normal_f32": ([vp, vp, u64, u64, u32, f32, f32], i),
        "opure_quantize_i8pc": ([vp, vp, u32, u32, vp, vp], i),
        "opure_quantize_i4g128": ([vp, vp, u32, u32, vp, vp, vp], i),
        "opure_convert_f32": ([vp, vp, vp, u32, u64], i),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res


def check(rc: int) -> None:
    if rc != OK:
        raise OpureError(rc, lib().opure_last_error().decode(errors="replace"))


def rope_table(theta: float, head_dim: int, max_pos: int, mode: int = ROPE_GPU):
    cos = np.zeros((max_pos, head_dim // 2), dtype=np.float32)
    sin = np.zeros_like(cos)
    check(lib().opure_rope_table(float(theta), head_dim, max_pos, mode, cos.ctypes.data, sin.ctypes.data))
    return cos, sin


class Buf:
    """A device allocation owned by a Dev."""

    def __init__(self, dev: "Dev", nbytes: int):
        self.dev = dev
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib().opure_buf_alloc(dev.h, max(1, self.nbytes), C.byref(p)))
        self.ptr = p.value

    def free(self):
        if self.ptr:
            check(lib().opure_buf_free(self.dev.h, self.ptr))
            self.ptr = None

    def __int__(self):
        return self.ptr


class Dev:
    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        check(lib().opure_dev_create(ordinal, C.byref(h)))
        self.h = h.value
        self._bufs = []

    @property
    def name(self) -> str:
        return lib().opure_dev_name(self.h).decode()

    @property
    def hbm_bytes(self) -> int:
        return int(lib().opure_dev_hbm_bytes(self.h))

    def alloc(self, nbytes: int) -> Buf:
        b = Buf(self, nbytes)
        self._bufs.append(b)
        return b

    def upload(self, arr: np.ndarray) -> Buf:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes)
        check(lib().opure_buf_upload(self.h, b.ptr, 0, arr.ctypes.data, arr.nbytes))
        return b

    def write(self, buf, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        check(lib().opure_buf_upload(self.h, int(buf), offset, arr.ctypes.data, arr.nbytes))

    def download(self, buf, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        check(lib().opure_buf_download(self.h, out.ctypes.data, int(buf), offset, out.nbytes))
        return out

    def fill_u32(self, buf, value: int, count: int) -> None:
        check(lib().opure_buf_fill_u32(self.h, int(buf), value & 0xFFFFFFFF, count))

    def sync(self) -> None:
        check(lib().opure_stream_sync(self.h))

    def timer_begin(self):
        check(lib().opure_timer_begin(self.h))

    def timer_end(self):
        check(lib().opure_timer_end(self.h))

    def timer_ms(self) -> float:
        ms = C.c_float()
        check(lib().opure_timer_ms(self.h, C.byref(ms)))
        return float(ms.value)

    def bw_measure(self, mode: int, src, dst, nbytes: int, reps: int) -> float:
        """GB/s of `reps` read-only (BW_READ) or copy (BW_COPY) launches over nbytes."""
        g = C.c_double()
        check(lib().opure_bw_measure(self.h, mode, int(src), int(dst) if dst is not None else None, nbytes, reps,
                                     C.byref(g)))
        return float(g.value)

    def tile(self, wfmt: int, src: "Linear", layout: int = LAYOUT_TILED):
        """Tiled copy of a row-major device linear: (Linear, [buffers to keep alive])."""
        wb, sb = C.c_uint64(), C.c_uint64()
        check(lib().opure_tiled_bytes(wfmt, src.out, src.in_, C.byref(wb), C.byref(sb)))
        w = self.alloc(wb.value)
        s = self.alloc(sb.value) if sb.value else None
        dst = Linear()
        check(lib().opure_tile_linear(self.h, wfmt, layout, C.byref(src), int(w), int(s) if s else None, C.byref(dst)))
        return dst, [w, s]

    def profile(self, on: bool):
        check(lib().opure_profile_enable(self.h, 1 if on else 0))

    def profile_read(self) -> dict:
        """{stage: (launches, total ms)} since the last read."""
        n = len(STAGES)
        counts, ms = (C.c_uint32 * n)(), (C.c_double * n)()
        check(lib().opure_profile_read(self.h, counts, ms))
        return {STAGES[i]: (int(counts[i]), float(ms[i])) for i in range(n)}

    def graph_begin(self):
        check(lib().opure_graph_begin(self.h))

    def graph_end(self):
        g = C.c_void_p()
        check(lib().opure_graph_end(self.h, C.byref(g)))
        return g.value

    def graph_launch(self, g):
        check(lib().opure_graph_launch(self.h, g))

    def graph_destroy(self, g):
        check(lib().opure_graph_destroy(g))

    def on_close(self, fn) -> None:
        """Registers a callback run first by close() (objects that hold device
        resources and must be released before the device)."""
        self.__dict__.setdefault("_closers", []).append(fn)

    def close(self):
        for fn in reversed(self.__dict__.get("_closers", [])):
            fn()
        self.__dict__["_closers"] = []
        for b in self._bufs:
            if b.ptr:
                lib().opure_buf_free(self.h, b.ptr)
                b.ptr = None
        self._bufs = []
        if self.h:
            lib().opure_dev_destroy(self.h)
            self.h = None


def act_dtype(afmt: int):
    return np.float32 if afmt == A_F32 else np.uint16


class DeviceModel:
    """A model resident on the device, described by opure_model.

    `weights` is a dict with the host arrays of a model: embed, lm_head (may be
    the same dict as embed), final_norm, rope_cos, rope_sin and layers (each with
    attn_norm, mlp_norm, qkv, o, gate_up, down); every linear is a dict
    {w, scale, zero, out, in}.  Arrays are uploaded once; tied linears share
    their device buffers.
    """

    def __init__(self, dev: Dev, cfg: dict, weights: dict):
        self.dev = dev
        self.cfg = dict(cfg)
        self._cache = {}

        def up(a):
            if a is None:
                return None
            k = id(a)
            if k not in self._cache:
                self._cache[k] = (a, dev.upload(a))
            return self._cache[k][1]

        self._tiled = {}

        def lin(d, layout=LAYOUT_TILED):
            k = (id(d), layout)
            if k not in self._tiled:
                rm = Linear(int(up(d["w"])), int(up(d.get("scale"))) if d.get("scale") is not None else None,
                            int(up(d.get("zero"))) if d.get("zero") is not None else None, d["out"], d["in"],
                            LAYOUT_ROWMAJOR)
                self._tiled[k] = dev.tile(cfg["wfmt"], rm, layout)
            return self._tiled[k][0]

        n = cfg["n_layers"]
        self._layers = (LayerWeights * n)()
        for i, L in enumerate(weights["layers"]):
            self._layers[i] = LayerWeights(int(up(L["attn_norm"])), int(up(L["mlp_norm"])), lin(L["qkv"]),
                                           lin(L["o"]), lin(L["gate_up"], LAYOUT_TILED_SWIGLU), lin(L["down"]))
        self.rope_cos = up(weights["rope_cos"])
        self.rope_sin = up(weights["rope_sin"])
        self.desc = Model(n, cfg["hidden"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["ffn"],
                          cfg["vocab"], cfg["rms_eps"], cfg["attn_scale"], cfg["wfmt"], cfg["afmt"],
                          int(self.rope_cos), int(self.rope_sin), weights["rope_cos"].shape[0],
                          lin(weights["embed"]), lin(weights["lm_head"]), int(up(weights["final_norm"])),
                          C.cast(self._layers, C.POINTER(LayerWeights)))


class DeviceKV:
    """A paged KV pool plus page tables on the device."""

    def __init__(self, dev: Dev, cfg: dict, n_pages: int, batch: int, max_pages_per_seq: int):
        self.dev = dev
        eb = 4 if cfg["afmt"] == A_F32 else 2
        self.shape = (cfg["n_layers"], n_pages, 2, cfg["n_kv_heads"], PAGE_SIZE, cfg["head_dim"])
        self.pool = dev.alloc(int(np.prod(self.shape)) * eb)
        self.page_table = dev.alloc(batch * max_pages_per_seq * 4)
        self.n_pages, self.batch, self.max_pages = n_pages, batch, max_pages_per_seq
        self.afmt = cfg["afmt"]
        self.desc = KV(int(self.pool), n_pages, PAGE_SIZE, int(self.page_table), max_pages_per_seq)

    def set_pool(self, host_pool: np.ndarray):
        assert host_pool.shape == self.shape
        self.dev.write(self.pool, host_pool)

    def set_page_table(self, pt: np.ndarray):
        assert pt.shape == (self.batch, self.max_pages)
        self.dev.write(self.page_table, np.ascontiguousarray(pt, dtype=np.int32))

    def get_pool(self) -> np.ndarray:
        return self.dev.download(self.pool, act_dtype(self.afmt), self.shape)

    def get_page_table(self) -> np.ndarray:
        return self.dev.download(self.page_table, np.int32, (self.batch, self.max_pages))


def gemv(dev: Dev, wfmt: int, lin: Linear, x, y, M: int, xfmt: int, yfmt: int, epilogue: int) -> None:
    """One batched GEMV; a row-major `lin` is tiled first (into temporaries)."""
    keep = None
    if lin.layout == LAYOUT_ROWMAJOR and lin.w:
        lin, keep = dev.tile(wfmt, lin, LAYOUT_TILED_SWIGLU if epilogue == EPI_SWIGLU else LAYOUT_TILED)
    a = GemvArgs(lin, int(x), int(y), M, xfmt, yfmt, epilogue)
    fn = {W_F32: lib().opure_gemv_batched_f32, W_I8PC: lib().opure_gemv_batched_i8pc,
          W_I4G128: lib().opure_gemv_batched_i4g128}[wfmt]
    check(fn(dev.h, C.byref(a)))
    if keep is not None:
        dev.sync()
        for b in keep:
            if b is not None:
                b.free()
