"""GEMV engine comparison: the matrix-core kernels (the product path) against
the vector-ALU kernel (opure_debug_set_gemv_engine) on the linears of three
verify-step shapes:

    1b-int8     Llama-3.2-1B linears, int8 per-channel weights, fp16 X, at 1 row
                (a draft step) and 6 rows (a K=5 verify step)
    smollm-f32  SmolLM-135M linears, fp32 weights and X, at 1 row (a greedy or
                draft step) and 5 rows (a K=4 verify step)
    8b-int4     Llama-3-8B linears, uint4 group-128 weights, bf16 X, at 1 row
                and 8 rows (a K=7 verify step)

    python opure-voxelengine_amd/gemv_ab.py [--set 1b-int8] [--reps 20]
    rocprofv3 --kernel-trace --output-format csv -d OUT -o ab -- python3 opure-voxelengine_amd/gemv_ab.py --set S
    python opure-voxelengine_amd/gemv_ab.py --set S --trace OUT/ab_kernel_trace.csv

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

# per set: weight format, activation format, rows, [(name, out, in, epilogue)]
SETS = {
    "1b-int8": (H.W_I8PC, H.A_F16, (1, 6),
                [("qkv", 3072, 2048, H.EPI_STORE), ("o_proj", 2048, 2048, H.EPI_RESIDUAL),
                 ("gate_up", 16384, 2048, H.EPI_SWIGLU), ("down", 2048, 8192, H.EPI_RESIDUAL),
                 ("lm_head", 128256, 2048, H.EPI_STORE)]),
    "smollm-f32": (H.W_F32, H.A_F32, (1, 5),
                   [("qkv", 960, 576, H.EPI_STORE), ("o_proj", 576, 576, H.EPI_RESIDUAL),
                    ("gate_up", 3072, 576, H.EPI_SWIGLU), ("down", 576, 1536, H.EPI_RESIDUAL),
                    ("lm_head", 49152, 576, H.EPI_STORE)]),
    "8b-int4": (H.W_I4G128, H.A_BF16, (1, 8),
                [("qkv", 6144, 4096, H.EPI_STORE), ("o_proj", 4096, 4096, H.EPI_RESIDUAL),
                 ("gate_up", 28672, 4096, H.EPI_SWIGLU), ("down", 4096, 14336, H.EPI_RESIDUAL),
                 ("lm_head", 128256, 4096, H.EPI_STORE)]),
}
ENGINES = (("mfma", H.GEMV_MFMA), ("valu", H.GEMV_VALU))
WARMUP = 3
POOL_BYTES = 640 << 20        # weight copies per shape: more than the last-level cache
GEMV_FN = {H.W_F32: "opure_gemv_batched_f32", H.W_I8PC: "opure_gemv_batched_i8pc",
           H.W_I4G128: "opure_gemv_batched_i4g128"}


def weight_bytes(wfmt: int, out: int, inn: int) -> int:
    if wfmt == H.W_F32:
        return out * inn * 4
    if wfmt == H.W_I8PC:
        return out * inn + 2 * out
    return out * inn // 2 + 4 * out * (inn // 128)


def cases(name: str, reps: int):
    wfmt, afmt, rows, shapes = SETS[name]
    for lin, out, inn, epi in shapes:
        for M in rows:
            for eng, code in ENGINES:
                yield dict(linear=lin, out=out, inn=inn, epi=epi, rows=M, engine=eng, code=code,
                           launches=WARMUP + reps, wfmt=wfmt, afmt=afmt)


def make_copies(dev, L, tmp, wfmt, out, inn, layout, copies):
    tiled, keep = [], []
    for k in range(copies):
        H.check(L.opure_synth_normal_f32(dev.h, int(tmp), out * inn, 11, k, 0.02, 0.0))
        if wfmt == H.W_F32:
            w = dev.alloc(out * inn * 4)
            H.check(L.opure_buf_copy(dev.h, int(w), int(tmp), out * inn * 4))
            src, tmps = H.Linear(int(w), None, None, out, inn, H.LAYOUT_ROWMAJOR), [w]
        elif wfmt == H.W_I8PC:
            q, s = dev.alloc(out * inn), dev.alloc(out * 2)
            H.check(L.opure_quantize_i8pc(dev.h, int(tmp), out, inn, int(q), int(s)))
            src, tmps = H.Linear(int(q), int(s), None, out, inn, H.LAYOUT_ROWMAJOR), [q, s]
        else:
            G = inn // 128
            q, s, z = dev.alloc(out * inn // 2), dev.alloc(out * G * 2), dev.alloc(out * G * 2)
            H.check(L.opure_quantize_i4g128(dev.h, int(tmp), out, inn, int(q), int(s), int(z)))
            src, tmps = H.Linear(int(q), int(s), int(z), out, inn, H.LAYOUT_ROWMAJOR), [q, s, z]
        t, kb = dev.tile(wfmt, src, layout)
        dev.sync()
        for b in tmps:
            b.free()
        tiled.append(t)
        keep += kb
    return tiled, keep


def run(name: str, reps: int) -> None:
    wfmt, afmt, rows, shapes = SETS[name]
    dev = H.Dev(0)
    L = H.lib()
    gemv = getattr(L, GEMV_FN[wfmt])
    eb = 4 if afmt == H.A_F32 else 2
    tmp = dev.alloc(max(o * i for _, o, i, _ in shapes) * 4)
    for lin, out, inn, epi in shapes:
        copies = max(1, POOL_BYTES // weight_bytes(wfmt, out, inn))
        layout = H.LAYOUT_TILED_SWIGLU if epi == H.EPI_SWIGLU else H.LAYOUT_TILED
        tiled, keep = make_copies(dev, L, tmp, wfmt, out, inn, layout, copies)
        x = dev.alloc(8 * inn * eb)
        H.check(L.opure_synth_normal_f32(dev.h, int(tmp), 8 * inn, 12, 0, 1.0, 0.0))
        H.check(L.opure_convert_f32(dev.h, int(tmp), int(x), afmt, 8 * inn))
        yout = out // 2 if epi == H.EPI_SWIGLU else out
        y = dev.alloc(8 * yout * 4)
        dev.fill_u32(y, 0, 8 * yout)
        yfmt = afmt if epi == H.EPI_SWIGLU else H.A_F32
        for c in cases(name, reps):
            if c["linear"] != lin:
                continue
            H.check(L.opure_debug_set_gemv_engine(dev.h, c["code"]))
            args = [H.GemvArgs(t, int(x), int(y), c["rows"], afmt, yfmt, epi) for t in tiled]
            for i in range(WARMUP):
                H.check(gemv(dev.h, C.byref(args[i % copies])))
            dev.sync()
            dev.timer_begin()
            for i in range(reps):
                H.check(gemv(dev.h, C.byref(args[(WARMUP + i) % copies])))
            dev.timer_end()
            us = dev.timer_ms() * 1e3 / reps
            dev.sync()
            print(json.dumps(dict(set=name, linear=lin, shape=f"{out}x{inn}", rows=c["rows"], engine=c["engine"],
                                  us_per_launch_with_gaps=round(us, 2))), flush=True)
        H.check(L.opure_debug_set_gemv_engine(dev.h, H.GEMV_MFMA))
        for b in keep + [x, y]:
            if b is not None:
                b.free()
    dev.close()


def trace(name: str, path: str, reps: int) -> None:
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
    for c in cases(name, reps):
        seg = rows[i:i + c["launches"]][WARMUP:]
        i += c["launches"]
        if not seg:
            break
        us = sum(e - s for s, e, _ in seg) / len(seg) / 1e3
        gbs = weight_bytes(c["wfmt"], c["out"], c["inn"]) / (us * 1e-6) / 1e9
        kern = seg[0][2].split("(")[0].replace("opure_gemv::", "")
        print(f"| {c['linear']} | {c['out']}x{c['inn']} | {c['rows']} | {c['engine']} | `{kern}` | {us:.2f} | "
              f"{gbs:.0f} | {gbs / 8000:.3f} |")


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--set", default="1b-int8", choices=sorted(SETS))
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--trace", default=None)
    a = ap.parse_args()
    if a.trace:
        trace(a.set, a.trace, a.reps)
    else:
        run(a.set, a.reps)
