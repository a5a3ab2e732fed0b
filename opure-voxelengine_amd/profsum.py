"""Summarise a rocprofv3 kernel trace by verify step.

    python opure-voxelengine_amd/profsum.py <..._kernel_trace.csv> [--rows R]
    python opure-voxelengine_amd/profsum.py <..._counter_collection.csv> --pmc KERNEL... [--last N]

A verify step starts at its k_embed dispatch, whose grid holds one 256-thread
workgroup per scored row.  Only steps scoring `--rows` rows are kept (the
benchmark's timed steps, not the prefill or single-row draft steps), and every
kernel of those steps is reported per step: launches, mean and median
duration, and the share of the summed kernel time.

Each dispatch is also given its stage of the step: the GEMV launches of a
layer come in the order qkv, o_proj, gate_up, down, and the one after the last
layer is the LM head (a rows pass before a GEMV and a K-split reduction after
it belong to that GEMV); attention kernels are the attention stage, the
acceptance and rollback kernels the accept stage.  With `--config` (and
`--ctx`), the stage table adds each stage's algorithmic bytes per launch
(synth.stage_bytes), its GB/s from the mean kernel time and the fraction of
the 8 TB/s HBM peak -- the figures bench.py's roofline reports.  Prints
markdown.
"""
from __future__ import annotations

import argparse
import collections
import csv
import re
import statistics


def short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "").replace("opure_hip::", "").replace("void ", "")
    name = re.sub(r"\((KParams|AttnParams|GreedyParams|RollbackParams)\)$", "", name)
    return name.split("(")[0] if "(" in name and "<" not in name.split("(")[0][-1:] else name


GEMV_MAIN = ("k_gemv", "k_gemm_wide")
GEMV_ORDER = ("qkv", "o_proj", "gate_up", "down")


def stage_of_step(seg):
    """The stage of every dispatch of one step (see the module docstring)."""
    names = [r["Kernel_Name"] for r in seg]
    mains = [i for i, n in enumerate(names) if any(k in n for k in GEMV_MAIN)]
    n_layers = (len(mains) - 1) // 4
    out = []
    gi = -1
    for i, n in enumerate(names):
        if "k_embed" in n:
            out.append("embed")
        elif "k_attn" in n:
            out.append("attention")
        elif any(k in n for k in ("accept", "k_rej_", "rollback", "argmax")):
            out.append("accept")
        else:
            if i in mains:
                gi = mains.index(i)
            elif "rmsnorm_rows" in n:
                gi = next((mains.index(j) for j in mains if j > i), gi)
            out.append("lm_head" if gi >= 4 * n_layers else GEMV_ORDER[gi % 4] if gi >= 0 else "other")
    return out


def steps_of(rows, want_rows):
    starts = [i for i, r in enumerate(rows) if "k_embed" in r["Kernel_Name"]]
    out = []
    for si, i0 in enumerate(starts):
        i1 = starts[si + 1] if si + 1 < len(starts) else len(rows)
        wg = int(rows[i0]["Grid_Size_X"]) // max(1, int(rows[i0]["Workgroup_Size_X"]))
        if wg != want_rows:
            continue
        seg = rows[i0:i1]
        # a step ends at its acceptance kernel (later dispatches belong to the harness)
        end = max((j for j, r in enumerate(seg) if "accept" in r["Kernel_Name"] or "rollback" in r["Kernel_Name"]),
                  default=len(seg) - 1)
        out.append(seg[:end + 1])
    return out


def pmc(path, kernels, last):
    """Median per-dispatch value of each counter over the last `last`
    dispatches of each kernel whose name contains one of `kernels`
    (rocprofv3 --pmc ... --output-format csv: *_counter_collection.csv)."""
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    names, durs = {}, {}
    for r in csv.DictReader(open(path)):
        d = int(r["Dispatch_Id"])
        per[d][r["Counter_Name"]] += float(r["Counter_Value"])
        names[d] = r["Kernel_Name"]
        durs[d] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    for k in kernels:
        ds = sorted(d for d in per if k in names[d])[-last:]
        if not ds:
            print(f"{k}: no dispatch")
            continue
        for cn in sorted(per[ds[0]]):
            v = statistics.median(per[d][cn] for d in ds)
            print(f"{k:32s} {cn:12s} median {v:12.1f} KiB over {len(ds)} dispatches, "
                  f"median duration {statistics.median(durs[d] for d in ds):.2f} us")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--rows", type=int, default=6)
    ap.add_argument("--pmc", nargs="+", metavar="KERNEL", help="counter summary of these kernels instead")
    ap.add_argument("--last", type=int, default=64, help="with --pmc: the last N dispatches of each kernel")
    ap.add_argument("--config", help="workload (synth.CONFIGS key): adds bytes, GB/s and HBM fraction per stage")
    ap.add_argument("--ctx", type=int, help="cached tokens per sequence for the attention bytes (default: the config's)")
    a = ap.parse_args()
    if a.pmc:
        return pmc(a.trace, a.pmc, a.last)
    rows = [r for r in csv.DictReader(open(a.trace)) if r.get("Kind", "KERNEL_DISPATCH") == "KERNEL_DISPATCH"]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    steps = steps_of(rows, a.rows)
    if not steps:
        raise SystemExit(f"no verify step with {a.rows} rows in {a.trace}")
    per = collections.defaultdict(list)
    per_stage = collections.defaultdict(list)          # (stage, kernel) -> durations
    stage_step = collections.defaultdict(float)        # stage -> summed kernel time over all steps
    spans = []
    for seg in steps:
        spans.append((int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])) / 1e3)
        for r, st in zip(seg, stage_of_step(seg)):
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            per[short(r["Kernel_Name"])].append(d)
            per_stage[(st, short(r["Kernel_Name"]))].append(d)
            stage_step[st] += d
    n = len(steps)
    total = sum(sum(v) for v in per.values()) / n
    print(f"{n} verify steps of {a.rows} rows; first-to-last dispatch span per step: "
          f"median {statistics.median(spans):.1f} us; summed kernel time per step {total:.1f} us\n")
    print("| kernel | launches/step | mean us | median us | us/step | share |")
    print("|---|---:|---:|---:|---:|---:|")
    for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{k}` | {len(v) / n:.0f} | {statistics.mean(v):.2f} | {statistics.median(v):.2f} | "
              f"{sum(v) / n:.1f} | {100 * sum(v) / n / total:.1f}% |")
    cfg = None
    if a.config:
        import synth
        cfg = synth.CONFIGS[a.config]
    ctx = a.ctx if a.ctx is not None else (cfg["ctx"] if cfg else 0)
    print("\nBy stage and kernel:\n")
    print("| stage | kernel | launches/step | mean us | median us | us/step |")
    print("|---|---|---:|---:|---:|---:|")
    order = ("embed", "qkv", "attention", "o_proj", "gate_up", "down", "lm_head", "accept", "other")
    for (st, k), v in sorted(per_stage.items(), key=lambda kv: (order.index(kv[0][0]), -sum(kv[1]))):
        print(f"| {st} | `{k}` | {len(v) / n:.0f} | {statistics.mean(v):.2f} | {statistics.median(v):.2f} | "
              f"{sum(v) / n:.1f} |")
    cfg = None
    if a.config:
        import synth
        cfg = synth.CONFIGS[a.config]
    ctx = a.ctx if a.ctx is not None else (cfg["ctx"] if cfg else 0)
    n_layers = (sum(1 for (st, _k), v in per_stage.items() if st == "qkv" for _ in v) // n) or 1
    print("\nBy stage (an instance is one layer's, or the step's, launches of that stage"
          + (f"; algorithmic bytes for {a.rows} rows over {ctx} cached tokens, synth.stage_bytes" if cfg else "")
          + "):\n")
    print("| stage | instances/step | kernel us/instance | us/step |"
          + (" bytes/instance | GB/s | frac of 8 TB/s |" if cfg else ""))
    print("|---|---:|---:|---:|" + ("---:|---:|---:|" if cfg else ""))
    for st in order:
        if st not in stage_step:
            continue
        inst = n_layers if st in GEMV_ORDER + ("attention",) else 1
        us = stage_step[st] / n / inst
        line = f"| {st} | {inst} | {us:.2f} | {stage_step[st] / n:.1f} |"
        if cfg:
            by = synth.stage_bytes(cfg, st, a.rows, ctx) if st not in ("accept", "other") else 0
            line += f" {by} | {by / us / 1e3:.0f} | {by / us / 1e3 / 8000:.3f} |" if by else " | | |"
        print(line)

if __name__ == "__main__":
    main()
