"""Summarise a rocprofv3 kernel trace by verify step.

    python opure-voxelengine_amd/profsum.py <..._kernel_trace.csv> [--rows R]
    python opure-voxelengine_amd/profsum.py <..._counter_collection.csv> --pmc KERNEL... [--last N]

A verify step starts at its k_embed dispatch, whose grid holds one 256-thread
workgroup per scored row.  Only steps scoring `--rows` rows are kept (the
benchmark's timed steps, not the prefill or single-row draft steps), and every
kernel of those steps is reported per step: launches, mean and median
duration, and the share of the summed kernel time.  Prints markdown.
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
    a = ap.parse_args()
    if a.pmc:
        return pmc(a.trace, a.pmc, a.last)
    rows = [r for r in csv.DictReader(open(a.trace)) if r.get("Kind", "KERNEL_DISPATCH") == "KERNEL_DISPATCH"]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    steps = steps_of(rows, a.rows)
    if not steps:
        raise SystemExit(f"no verify step with {a.rows} rows in {a.trace}")
    per = collections.defaultdict(list)
    spans = []
    for seg in steps:
        spans.append((int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])) / 1e3)
        for r in seg:
            per[short(r["Kernel_Name"])].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    n = len(steps)
    total = sum(sum(v) for v in per.values()) / n
    print(f"{n} verify steps of {a.rows} rows; first-to-last dispatch span per step: "
          f"median {statistics.median(spans):.1f} us; summed kernel time per step {total:.1f} us\n")
    print("| kernel | launches/step | mean us | median us | us/step | share |")
    print("|---|---:|---:|---:|---:|---:|")
    for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{k}` | {len(v) / n:.0f} | {statistics.mean(v):.2f} | {statistics.median(v):.2f} | "
              f"{sum(v) / n:.1f} | {100 * sum(v) / n / total:.1f}% |")


if __name__ == "__main__":
    main()
