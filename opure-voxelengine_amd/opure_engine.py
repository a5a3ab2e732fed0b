"""ctypes binding of include/opure_engine.h (libopure_engine.so): the native
C++20 generation engine (greedy and speculative) over the verify path."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

import opure_hip as H

# OPURE_ENGINE_LIB: another build of the engine sources (e.g. with sanitizers)
ENGINE_PATH = os.environ.get("OPURE_ENGINE_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                                                                 "libopure_engine.so")
_lib = None


class Options(C.Structure):
    _fields_ = [("max_positions", C.c_uint32), ("draft_tokens", C.c_uint32), ("use_graphs", C.c_uint32),
                ("stop_token", C.c_int32)]


class Stats(C.Structure):
    _fields_ = [("emitted", C.c_uint32), ("verify_steps", C.c_uint32), ("draft_steps", C.c_uint32),
                ("accepted_total", C.c_uint32), ("ms_prefill", C.c_double), ("ms_generate", C.c_double)]


class Metrics(C.Structure):
    _fields_ = [("generate_calls", C.c_uint64), ("verify_steps", C.c_uint64), ("drafts_proposed", C.c_uint64),
                ("drafts_accepted", C.c_uint64), ("tokens_emitted", C.c_uint64),
                ("speculative_acceptance", C.c_double)]


class LoadOptions(C.Structure):
    _fields_ = [("max_positions", C.c_uint32), ("wfmt", C.c_int32), ("afmt", C.c_int32), ("attn_scale", C.c_float),
                ("rope_pairs", C.c_uint32)]


class ModelInfo(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "ffn", "vocab",
                                          "max_position_embeddings")] + \
               [("rms_eps", C.c_float), ("attn_scale", C.c_float), ("rope_theta", C.c_double), ("tied", C.c_uint32),
                ("stored_wfmt", C.c_uint32), ("wfmt", C.c_uint32), ("afmt", C.c_uint32), ("rope_max_pos", C.c_uint32),
                ("n_tensors", C.c_uint32), ("file_bytes", C.c_uint64)]


class HostLinearC(C.Structure):
    _fields_ = [("wfmt", C.c_uint32), ("out", C.c_uint32), ("in_", C.c_uint32), ("w", C.c_void_p),
                ("scale", C.c_void_p), ("zero", C.c_void_p), ("w_bytes", C.c_uint64), ("scale_bytes", C.c_uint64),
                ("zero_bytes", C.c_uint64)]


class TensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_uint32), ("ndim", C.c_uint32), ("shape", C.c_int64 * 8),
                ("offset", C.c_uint64), ("bytes", C.c_uint64), ("data", C.c_void_p), ("has_scale", C.c_uint32),
                ("scale", C.c_double)]


ROPE_PAIRS_ADJACENT, ROPE_PAIRS_HALF = 0, 1
ROLE_EMBED, ROLE_LM_HEAD, ROLE_QKV, ROLE_O, ROLE_GATE_UP, ROLE_DOWN, ROLE_ATTN_NORM, ROLE_MLP_NORM, ROLE_FINAL_NORM = \
    range(9)
DTYPES = ("F32", "F16", "BF16", "U8", "I8", "U4", "I4")


def lib():
    global _lib
    if _lib is None:
        H.lib()                                   # libopure_hip first (the engine links it)
        if not os.path.exists(ENGINE_PATH):
            raise H.OpureError(H.E_INVALID, f"{ENGINE_PATH} is not built (run opure-voxelengine_amd/build.py)")
        L = C.CDLL(ENGINE_PATH)
        vp, u32, i = C.c_void_p, C.c_uint32, C.c_int
        L.opure_engine_last_error.argtypes, L.opure_engine_last_error.restype = [], C.c_char_p
        L.opure_engine_create.argtypes = [vp, C.POINTER(H.Model), C.POINTER(H.Model), C.POINTER(Options), C.POINTER(vp)]
        L.opure_engine_destroy.argtypes = [vp]
        L.opure_engine_generate.argtypes = [vp, vp, u32, u32, vp, C.POINTER(Stats)]
        L.opure_engine_generate_speculative.argtypes = [vp, vp, u32, u32, vp, vp, u32, C.POINTER(Stats)]
        L.opure_engine_get_metrics.argtypes = [vp, C.POINTER(Metrics)]
        L.opure_engine_reset_metrics.argtypes = [vp]
        L.opure_page_pool_create.argtypes = [u32, C.POINTER(vp)]
        L.opure_page_pool_destroy.argtypes = [vp]
        L.opure_page_pool_available.argtypes = [vp, C.POINTER(u32)]
        L.opure_page_pool_alloc.argtypes = [vp, u32, vp]
        L.opure_page_pool_release.argtypes = [vp, vp, u32]
        L.opure_page_pool_grow_seq.argtypes = [vp, vp, u32, u32, C.POINTER(u32)]
        L.opure_engine_verify_step.argtypes = [vp, vp, u32, u32, vp, C.POINTER(u32)]
        L.opure_engine_forward_logits.argtypes = [vp, vp, u32, vp, C.POINTER(u32)]
        L.opure_engine_rollback_kv.argtypes = [vp, u32, u32, u32, C.POINTER(u32)]
        L.opure_engine_pages.argtypes = [vp, i, C.POINTER(u32), C.POINTER(u32), vp, u32, C.POINTER(u32)]
        cp = C.c_char_p
        L.opure_engine_initialize.argtypes = [vp, cp, cp, C.POINTER(LoadOptions), C.POINTER(Options), C.POINTER(vp)]
        L.opure_model_files_open.argtypes = [cp, C.POINTER(LoadOptions), C.POINTER(vp)]
        L.opure_model_files_info.argtypes = [vp, C.POINTER(ModelInfo)]
        L.opure_model_files_read.argtypes = [vp, u32, u32, C.POINTER(HostLinearC)]
        L.opure_model_files_close.argtypes = [vp]
        L.opure_model_load.argtypes = [vp, cp, C.POINTER(LoadOptions), C.POINTER(vp)]
        L.opure_loaded_model_desc.argtypes = [vp, C.POINTER(C.POINTER(H.Model)), C.POINTER(C.c_uint64)]
        L.opure_model_unload.argtypes = [vp]
        L.opure_safetensors_open.argtypes = [cp, C.POINTER(vp)]
        L.opure_safetensors_count.argtypes = [vp, C.POINTER(u32)]
        L.opure_safetensors_tensor.argtypes = [vp, u32, C.POINTER(TensorInfo)]
        L.opure_safetensors_find.argtypes = [vp, cp, C.POINTER(TensorInfo)]
        L.opure_safetensors_close.argtypes = [vp]
        for f in ("opure_engine_initialize", "opure_model_files_open", "opure_model_files_info",
                  "opure_model_files_read", "opure_model_files_close", "opure_model_load", "opure_loaded_model_desc",
                  "opure_model_unload", "opure_safetensors_open", "opure_safetensors_count",
                  "opure_safetensors_tensor", "opure_safetensors_find", "opure_safetensors_close"):
            getattr(L, f).restype = i
        for f in ("opure_engine_create", "opure_engine_destroy", "opure_engine_generate",
                  "opure_engine_generate_speculative", "opure_engine_get_metrics", "opure_engine_reset_metrics",
                  "opure_page_pool_create", "opure_page_pool_destroy", "opure_page_pool_available",
                  "opure_page_pool_alloc", "opure_page_pool_release", "opure_page_pool_grow_seq",
                  "opure_engine_verify_step", "opure_engine_rollback_kv", "opure_engine_pages",
                  "opure_engine_forward_logits"):
            getattr(L, f).restype = i
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != H.OK:
        raise H.OpureError(rc, lib().opure_engine_last_error().decode(errors="replace"))


class Engine:
    """VoxelEngine on device `dev` for a target model (and optional draft);
    the model descriptors (opure_model ctypes structures) must stay alive."""

    def __init__(self, dev: H.Dev, target_desc, draft_desc=None, max_positions: int = 4096, draft_tokens: int = 4,
                 use_graphs: bool = True, stop_token: int = -1, _handle=None):
        self.dev, self._t, self._d = dev, target_desc, draft_desc
        if _handle is None:
            o = Options(max_positions, draft_tokens, 1 if use_graphs else 0, stop_token)
            h = C.c_void_p()
            check(lib().opure_engine_create(dev.h, C.byref(target_desc), C.byref(draft_desc) if draft_desc else None,
                                            C.byref(o), C.byref(h)))
            _handle = h.value
        self.h = _handle
        self.K = draft_tokens
        dev.on_close(self.close)             # the engine frees its buffers before the device goes

    @classmethod
    def from_dirs(cls, dev: H.Dev, target_dir: str, draft_dir: str | None = None, load: LoadOptions | None = None,
                  max_positions: int = 4096, draft_tokens: int = 4, use_graphs: bool = True,
                  stop_token: int = -1) -> "Engine":
        """opure_engine_initialize: the engine loads and owns both models."""
        o = Options(max_positions, draft_tokens, 1 if use_graphs else 0, stop_token)
        h = C.c_void_p()
        check(lib().opure_engine_initialize(dev.h, target_dir.encode(), draft_dir.encode() if draft_dir else None,
                                            C.byref(load) if load else None, C.byref(o), C.byref(h)))
        return cls(dev, None, None, max_positions, draft_tokens, use_graphs, stop_token, _handle=h.value)

    def generate(self, prompt, n_new: int):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_new, dtype=np.int32)
        st = Stats()
        check(lib().opure_engine_generate(self.h, p.ctypes.data, p.size, n_new, out.ctypes.data, C.byref(st)))
        return out, st

    def forward_logits(self, tokens, vocab: int):
        """(logits [vocab], argmax) of the last of `tokens` prefilled into a fresh cache."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros(vocab, dtype=np.float32)
        am = C.c_uint32()
        check(lib().opure_engine_forward_logits(self.h, t.ctypes.data, t.size, out.ctypes.data, C.byref(am)))
        return out, int(am.value)

    def verify_step(self, tokens, seq_len: int):
        """(accepted, emitted ids): one verify step of the target on these rows."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros(t.size, dtype=np.int32)
        acc = C.c_uint32()
        check(lib().opure_engine_verify_step(self.h, t.ctypes.data, t.size, seq_len, out.ctypes.data, C.byref(acc)))
        return int(acc.value), out[:acc.value + 1].tolist()

    def rollback_kv(self, seq_len: int, accepted: int, k: int) -> int:
        n = C.c_uint32()
        check(lib().opure_engine_rollback_kv(self.h, seq_len, accepted, k, C.byref(n)))
        return int(n.value)

    def pages(self, draft: bool = False):
        """(pages in the pool, pages free, the sequence's page-table row)."""
        tot, av, n = C.c_uint32(), C.c_uint32(), C.c_uint32()
        check(lib().opure_engine_pages(self.h, 1 if draft else 0, C.byref(tot), C.byref(av), None, 0, C.byref(n)))
        row = np.zeros(n.value, dtype=np.int32)
        check(lib().opure_engine_pages(self.h, 1 if draft else 0, C.byref(tot), C.byref(av), row.ctypes.data, n.value,
                                       C.byref(n)))
        return int(tot.value), int(av.value), row

    def generate_speculative(self, prompt, n_new: int):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_new, dtype=np.int32)
        hist = np.zeros(n_new + 1, dtype=np.uint32)
        st = Stats()
        check(lib().opure_engine_generate_speculative(self.h, p.ctypes.data, p.size, n_new, out.ctypes.data,
                                                      hist.ctypes.data, hist.size, C.byref(st)))
        return out, hist[:st.verify_steps].copy(), st

    def close(self):
        if self.h:
            lib().opure_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def metrics(self) -> Metrics:
        m = Metrics()
        check(lib().opure_engine_get_metrics(self.h, C.byref(m)))
        return m

    def reset_metrics(self) -> None:
        check(lib().opure_engine_reset_metrics(self.h))


class PagePool:
    """opure_page_pool: the free list of a paged KV pool's pages (host only)."""

    def __init__(self, n_pages: int):
        h = C.c_void_p()
        check(lib().opure_page_pool_create(n_pages, C.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            lib().opure_page_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def available(self) -> int:
        n = C.c_uint32()
        check(lib().opure_page_pool_available(self.h, C.byref(n)))
        return n.value

    def alloc(self, n: int) -> np.ndarray:
        ids = np.full(max(n, 1), -1, dtype=np.int32)
        check(lib().opure_page_pool_alloc(self.h, n, ids.ctypes.data))
        return ids[:n]

    def release(self, ids) -> None:
        a = np.ascontiguousarray(ids, dtype=np.int32).ravel()
        check(lib().opure_page_pool_release(self.h, a.ctypes.data if a.size else None, a.size))

    def grow_seq(self, row: np.ndarray, tokens: int) -> int:
        """Fills the -1 entries of row[:ceil(tokens/16)] in place; returns the pages taken."""
        assert row.dtype == np.int32 and row.flags.c_contiguous
        added = C.c_uint32()
        check(lib().opure_page_pool_grow_seq(self.h, row.ctypes.data, row.size, tokens, C.byref(added)))
        return added.value


def load_options(max_positions: int = 0, wfmt: int = -1, afmt: int = -1, attn_scale: float = 0.0,
                 rope_pairs: int = ROPE_PAIRS_ADJACENT) -> LoadOptions:
    return LoadOptions(max_positions, wfmt, afmt, attn_scale, rope_pairs)


class ModelFiles:
    """opure_model_files: config.json + the mapped safetensors of a model
    directory, read on the host."""

    def __init__(self, model_dir: str, opts: LoadOptions | None = None):
        h = C.c_void_p()
        check(lib().opure_model_files_open(str(model_dir).encode(), C.byref(opts) if opts else None, C.byref(h)))
        self.h = h.value

    def info(self) -> ModelInfo:
        i = ModelInfo()
        check(lib().opure_model_files_info(self.h, C.byref(i)))
        return i

    def read(self, role: int, layer: int = 0) -> dict:
        """The role's row-major interchange arrays, copied out: {"wfmt", "out",
        "in", "w", "scale", "zero"} as uint8 byte arrays (None when absent)."""
        r = HostLinearC()
        check(lib().opure_model_files_read(self.h, role, layer, C.byref(r)))

        def grab(p, n):
            return np.ctypeslib.as_array((C.c_uint8 * n).from_address(p)).copy() if p and n else None
        return {"wfmt": r.wfmt, "out": r.out, "in": r.in_, "w": grab(r.w, r.w_bytes),
                "scale": grab(r.scale, r.scale_bytes), "zero": grab(r.zero, r.zero_bytes)}

    def close(self) -> None:
        if self.h:
            lib().opure_model_files_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class LoadedModel:
    """opure_loaded_model: a model directory on the device; `desc` is its
    opure_model, valid until close()."""

    def __init__(self, dev: H.Dev, model_dir: str, opts: LoadOptions | None = None):
        h = C.c_void_p()
        check(lib().opure_model_load(dev.h, str(model_dir).encode(), C.byref(opts) if opts else None, C.byref(h)))
        self.h = h.value
        p, nb = C.POINTER(H.Model)(), C.c_uint64()
        check(lib().opure_loaded_model_desc(self.h, C.byref(p), C.byref(nb)))
        self.desc, self.device_bytes = p.contents, nb.value
        dev.on_close(self.close)

    def close(self) -> None:
        if self.h:
            lib().opure_model_unload(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class SafeTensors:
    """opure_safetensors: a read-only mapped .safetensors file."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(lib().opure_safetensors_open(str(path).encode(), C.byref(h)))
        self.h = h.value

    @staticmethod
    def _info(t: TensorInfo) -> dict:
        shape = tuple(t.shape[i] for i in range(t.ndim))
        data = np.ctypeslib.as_array((C.c_uint8 * t.bytes).from_address(t.data)).copy() if t.bytes else \
            np.zeros(0, np.uint8)
        return {"name": t.name.decode(), "dtype": DTYPES[t.dtype], "shape": shape, "offset": t.offset,
                "bytes": t.bytes, "data": data, "scale": t.scale if t.has_scale else None}

    def tensors(self) -> list:
        n = C.c_uint32()
        check(lib().opure_safetensors_count(self.h, C.byref(n)))
        out = []
        for i in range(n.value):
            t = TensorInfo()
            check(lib().opure_safetensors_tensor(self.h, i, C.byref(t)))
            out.append(self._info(t))
        return out

    def find(self, name: str) -> dict:
        t = TensorInfo()
        check(lib().opure_safetensors_find(self.h, name.encode(), C.byref(t)))
        return self._info(t)

    def close(self) -> None:
        if self.h:
            lib().opure_safetensors_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
