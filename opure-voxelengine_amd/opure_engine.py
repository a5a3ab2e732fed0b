"""ctypes binding of include/opure_engine.h (libopure_engine.so): the native
C++20 generation engine (greedy and speculative) over the verify path."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

import opure_hip as H

ENGINE_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libopure_engine.so")
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
        L.opure_engine_rollback_kv.argtypes = [vp, u32, u32, u32, C.POINTER(u32)]
        L.opure_engine_pages.argtypes = [vp, i, C.POINTER(u32), C.POINTER(u32), vp, u32, C.POINTER(u32)]
        for f in ("opure_engine_create", "opure_engine_destroy", "opure_engine_generate",
                  "opure_engine_generate_speculative", "opure_engine_get_metrics", "opure_engine_reset_metrics",
                  "opure_page_pool_create", "opure_page_pool_destroy", "opure_page_pool_available",
                  "opure_page_pool_alloc", "opure_page_pool_release", "opure_page_pool_grow_seq",
                  "opure_engine_verify_step", "opure_engine_rollback_kv", "opure_engine_pages"):
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
                 use_graphs: bool = True, stop_token: int = -1):
        self.dev, self._t, self._d = dev, target_desc, draft_desc
        o = Options(max_positions, draft_tokens, 1 if use_graphs else 0, stop_token)
        h = C.c_void_p()
        check(lib().opure_engine_create(dev.h, C.byref(target_desc), C.byref(draft_desc) if draft_desc else None,
                                        C.byref(o), C.byref(h)))
        self.h = h.value
        self.K = draft_tokens
        dev.on_close(self.close)             # the engine frees its buffers before the device goes

    def generate(self, prompt, n_new: int):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_new, dtype=np.int32)
        st = Stats()
        check(lib().opure_engine_generate(self.h, p.ctypes.data, p.size, n_new, out.ctypes.data, C.byref(st)))
        return out, st

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
