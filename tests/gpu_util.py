"""Helpers shared by the GPU tests: move oracle-side host models and caches to
the device through the C-ABI, and run verify steps."""
import ctypes as C
import sys

import numpy as np

import opure_hip as H
import oracle as O


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def host_weights(m: O.HostModel) -> dict:
    return dict(embed=m.embed, lm_head=m.lm_head, final_norm=m.final_norm, rope_cos=m.rope_cos,
                rope_sin=m.rope_sin, layers=m.layers)


def device_model(dev: H.Dev, m: O.HostModel) -> H.DeviceModel:
    return H.DeviceModel(dev, m.cfg, host_weights(m))


def device_kv(dev: H.Dev, m: O.HostModel, kv: O.HostKV) -> H.DeviceKV:
    d = H.DeviceKV(dev, m.cfg, kv.n_pages, kv.batch, kv.max_pages)
    d.set_pool(kv.pool)
    d.set_page_table(kv.page_table)
    return d


class VerifyRunner:
    """Owns device buffers for verify steps of one shape."""

    def __init__(self, dev, dm: H.DeviceModel, dkv: H.DeviceKV, B: int, R: int, max_ctx: int):
        self.dev, self.dm, self.dkv, self.B, self.R, self.max_ctx = dev, dm, dkv, B, R, max_ctx
        V = dm.cfg["vocab"]
        self.tokens = dev.alloc(B * R * 4)
        self.seq_len = dev.alloc(B * 4)
        self.new_len = dev.alloc(B * 4)
        self.logits = dev.alloc(B * R * V * 4)
        self.out_tokens = dev.alloc(B * R * 4)
        self.accepted = dev.alloc(B * 4)
        self.dist = dev.alloc(B * V * 4)
        self.draft_logits = dev.alloc(B * max(1, R - 1) * V * 4)
        self.freed = dev.alloc(B * 8 * 4)
        self.n_freed = dev.alloc(B * 4)
        H.check(H.lib().opure_verify_reserve(dev.h, C.byref(dm.desc), B, R, max_ctx))

    def args(self, accept=H.ACCEPT_NONE, rollback=False, temperature=1.0, seed=0, poison=False, poison_bits=0,
             free_pages=False):
        a = H.VerifyArgs()
        a.model = C.pointer(self.dm.desc)
        a.kv = C.pointer(self.dkv.desc)
        a.batch, a.rows = self.B, self.R
        a.tokens, a.seq_len, a.max_ctx = int(self.tokens), int(self.seq_len), self.max_ctx
        a.logits = int(self.logits)
        a.accept_mode = accept
        a.draft_logits = int(self.draft_logits)
        a.temperature = temperature
        a.seed = seed
        a.pos_base = None
        a.out_tokens, a.accepted, a.dist_out = int(self.out_tokens), int(self.accepted), int(self.dist)
        a.rollback = 1 if rollback else 0
        a.new_seq_len = int(self.new_len)
        a.freed = int(self.freed) if free_pages else None
        a.freed_stride = 8
        a.n_freed = int(self.n_freed)
        a.poison = 1 if poison else 0
        a.poison_bits = poison_bits
        self._keep = a
        return a

    def step(self, tokens, seq_len, **kw):
        self.dev.write(self.tokens, np.ascontiguousarray(tokens, dtype=np.int32))
        self.dev.write(self.seq_len, np.ascontiguousarray(seq_len, dtype=np.int32))
        a = self.args(**kw)
        H.check(H.lib().opure_verify_step(self.dev.h, C.byref(a)))
        self.dev.sync()

    def get_logits(self):
        return self.dev.download(self.logits, np.float32, (self.B, self.R, self.dm.cfg["vocab"]))

    def get_accept(self):
        return (self.dev.download(self.out_tokens, np.int32, (self.B, self.R)),
                self.dev.download(self.accepted, np.int32, (self.B,)))


def top2_gap(logits: np.ndarray) -> np.ndarray:
    s = np.sort(logits.astype(np.float64), axis=-1)
    return s[..., -1] - s[..., -2]
