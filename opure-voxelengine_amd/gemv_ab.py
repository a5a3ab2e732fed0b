"""GEMV engine comparison on the 1B verify step's linears: the matrix-core
kernels (the product path) against the vector-ALU kernel
(opure_debug_set_gemv_engine), int8 per-channel weights and fp16 X, at 1 row
(a draft step) and 6 rows (a K=5 verify step).

    python opure-voxelengine_amd/gemv_ab.py [--reps 20]
    rocprofv3 --kernel-trace --output-format csv -d OUT -o ab -- python3 opure-voxelengine_amd/gemv_ab.py
    python opure-voxelengine_amd/gemv_ab.py --trace OUT/ab_kernel_trace.csv

The first form prints one JSON line per (linear, rows, engine) with the mean
time per launch from events around back-to-back launches (launch gaps
included).  Under rocprofv3 the same launches happen in the same order, and
--trace assigns the traced dispatches back to the cases and reports the
kernels' own mean duration and the HBM rate of the weight bytes.  Weights
rotate over copies totalling more than the 256 MB last-level cache, so every
launch streams its weights from HBM as the verify step does.
"""
from __future__ import annotations

import argparse
import csv
import ctypes as C
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import opure_hip as H  # noqa: E402

# name, out, in, epilogue (the 1B shapes: qkv, o_proj, gate/up, down, LM head)
SHAPES = [("qkv", 3072, 2048, H.EPI_STORE), ("o_proj", 2048, 2048, H.EPI_RESIDUAL),
          ("gate_up", 16384, 2048, H.EPI_SWIGLU), ("down", 2048, 8192, H.EPI_RESIDUAL),
          ("lm_head", 128256, 2048, H.EPI_STORE)]
ROWS = (1, 6)
ENGINES = (("mfma", H.GEMV_MFMA), ("valu", H.GEMV_VALU))
WARMUP = 3
POOL_BYTES = 640 << 20        # weight copies per shape: more than the last-level cache


def weight_bytes(out: int, inn: int) -> int:
    return out * inn + 2 * out


def cases(reps: int):
    for name, out, inn, epi in SHAPES:
        for M in ROWS:
            for eng, code in ENGINES:
                yield dict(linear=name, out=out, inn=inn, epi=epi, rows=M, engine=eng, code=code,
                           launches=WARMUP + reps)


def run(reps: int) -> None:
    dev = H.Dev(0)
    L = H.lib()
    tmp = dev.alloc(max(o * i for _, o, i, _ in SHAPES) * 4)
    for name, out, inn, epi in SHAPES:
        copies = max(1, POOL_BYTES // weight_bytes(out, inn))
        layout = H.LAYOUT_TILED_SWIGLU if epi == H.EPI_SWIGLU else H.LAYOUT_TILED
        tiled, keep = [], []
        for k in range(copies):
            H.check(L.opure_synth_normal_f32(dev.h, int(tmp), out * inn, 11, k, 0.02, 0.0))
            q, s = dev.alloc(out * inn), dev.alloc(out * 2)
            H.check(L.opure_quantize_i8pc(dev.h, int(tmp), out, inn, int(q), int(s)))
            t, kb = dev.tile(H.W_I8PC, H.Linear(int(q), int(s), None, out, inn, H.LAYOUT_ROWMAJOR), layout)
            dev.sync()
            q.free()
            s.free()
            tiled.append(t)
            keep += kb
        x = dev.alloc(8 * inn * 2)
        H.check(L.opure_synth_normal_f32(dev.h, int(tmp), 8 * inn, 12, 0, 1.0, 0.0))
        H.check(L.opure_convert_f32(dev.h, int(tmp), int(x), H.A_F16, 8 * inn))
        yout = out // 2 if epi == H.EPI_SWIGLU else out
        y = dev.alloc(8 * yout * 4)
        dev.fill_u32(y, 0, 8 * yout)
        yfmt = H.A_F16 if epi == H.EPI_SWIGLU else H.A_F32
        for c in cases(reps):
            if c["linear"] != name:
                continue
            H.check(L.opure_debug_set_gemv_engine(dev.h, c["code"]))
            args = [H.GemvArgs(t, int(x), int(y), c["rows"], H.A_F16, yfmt, epi) for t in tiled]
            for i in range(WARMUP):
                H.check(L.opure_gemv_batched_i8pc(dev.h, C.byref(args[i % copies])))
            dev.sync()
            dev.timer_begin()
            for i in range(reps):
                H.check(L.opure_gemv_batched_i8pc(dev.h, C.byref(args[(WARMUP + i) % copies])))
            dev.timer_end()
            us = dev.timer_ms() * 1e3 / reps
            dev.sync()
            print(json.dumps(dict(linear=name, shape=f"{out}x{inn}", rows=c["rows"], engine=c["engine"],
                                  us_per_launch_with_gaps=round(us, 2))), flush=True)
        H.check(L.opure_debug_set_gemv_engine(dev.h, H.GEMV_MFMA))
        for b in keep + [x, y]:
            if b is not None:
                b.free()
    dev.close()


def trace(path: str, reps: int) -> None:
    """Assigns the traced GEMV dispatches to the cases, in launch order."""
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            k = r.get("Kernel_Name", "")
            if "k_gemv" in k:
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), k))
    rows.sort()
    i = 0
    print("| linear | shape | rows | engine | kernel | mean us | weight GB/s | frac of 8 TB/s |")
    print("|---|---|---:|---|---|---:|---:|---:|")
    for c in cases(reps):
        seg = rows[i:i + c["launches"]][WARMUP:]
        i += c["launches"]
        if not seg:
            break
        us = sum(e - s for s, e, _ in seg) / len(seg) / 1e3
        gbs = weight_bytes(c["out"], c["inn"]) / (us * 1e-6) / 1e9
        kern = seg[0][2].split("(")[0].replace("opure_gemv::", "")
        print(f"| {c['linear']} | {c['out']}x{c['inn']} | {c['rows']} | {c['engine']} | `{kern}` | {us:.2f} | "
              f"{gbs:.0f} | {gbs / 8000:.3f} |")


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--trace", default=None)
    a = ap.parse_args()
    if a.trace:
        trace(a.trace, a.reps)
    else:
        run(a.reps)
