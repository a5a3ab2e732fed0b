"""Times the thin GEMM (the GEMV over more than 16 rows, k_gemm_wide +
k_wide_reduce) on the 1B int8 shapes of a 32-sequence x 7-row batch.

    python3 opure-voxelengine_amd/wide_bench.py [--rows 224 ...] [--lib PATH]

Each shape is tiled once; 20 calls are captured in a hipGraph, replayed once
to warm up and once timed with stream events, so the figure is device time
per call (kernel + split reduction) without the Python launch cost.  Weights
are seeded random int8 with fp16 scales, X seeded N(0,1) in fp16.
"""
import argparse
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import opure_hip as H  # noqa: E402

# name, out, in, epilogue, output format: the 1B layer's GEMVs and its LM head
SHAPES = [("gate_up", 16384, 2048, H.EPI_SWIGLU, H.A_F16), ("qkv", 3072, 2048, H.EPI_STORE, H.A_F16),
          ("o_proj", 2048, 2048, H.EPI_RESIDUAL, H.A_F32), ("down", 2048, 8192, H.EPI_RESIDUAL, H.A_F32),
          ("lm_head", 128256, 2048, H.EPI_STORE, H.A_F32)]
PEAK_F16 = 2.5e15        # MI355X dense fp16 MFMA, FLOP/s


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--rows", type=int, nargs="+", default=[224])
    ap.add_argument("--lib", default=None, help="another build of libopure_hip.so")
    ap.add_argument("--calls", type=int, default=20)
    args = ap.parse_args()
    if args.lib:
        H.LIB_PATH = os.path.abspath(args.lib)
    dev = H.Dev(0)
    rng = np.random.default_rng(0)
    print("| shape | rows | us per call | TFLOP/s | frac of dense fp16 | weight GB/s |")
    print("|---|---:|---:|---:|---:|---:|")
    for name, out, inn, epi, yfmt in SHAPES:
        w = dev.upload(rng.integers(-127, 128, size=(out, inn), dtype=np.int8))
        s = dev.upload((rng.random(out) * 0.02).astype(np.float16))
        src = H.Linear(int(w), int(s), None, out, inn, H.LAYOUT_ROWMAJOR)
        lin, keep = dev.tile(H.W_I8PC, src, H.LAYOUT_TILED_SWIGLU if epi == H.EPI_SWIGLU else H.LAYOUT_TILED)
        for M in args.rows:
            x = dev.upload(rng.standard_normal((M, inn)).astype(np.float16))
            yo = out // 2 if epi == H.EPI_SWIGLU else out
            y = dev.alloc(M * yo * (4 if yfmt == H.A_F32 else 2))
            if yfmt == H.A_F32:
                dev.write(y, np.zeros((M, yo), np.float32))
            H.gemv(dev, H.W_I8PC, lin, x, y, M, H.A_F16, yfmt, epi)   # sizes the split workspace
            dev.sync()
            dev.graph_begin()
            for _ in range(args.calls):
                H.gemv(dev, H.W_I8PC, lin, x, y, M, H.A_F16, yfmt, epi)
            g = dev.graph_end()
            dev.graph_launch(g)
            dev.sync()
            dev.timer_begin()
            dev.graph_launch(g)
            dev.timer_end()
            dev.sync()
            dev.graph_destroy(g)
            us = dev.timer_ms() * 1e3 / args.calls
            flop = 2.0 * out * inn * M
            print(f"| {name} {out}x{inn} | {M} | {us:.2f} | {flop / us / 1e6:.1f} | {flop / (us * 1e-6) / PEAK_F16:.3f} | "
                  f"{out * inn / us / 1e3:.0f} |", flush=True)
            x.free()
            y.free()
        for b in keep:
            if b:
                b.free()
        w.free()
        s.free()
    dev.close()


if __name__ == "__main__":
    main()
