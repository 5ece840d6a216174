"""Kernel-trace timeline of a serving loop (test infrastructure): from a
rocprofv3 --kernel-trace --output-format csv directory, the kernels of the
first continuous-batching loop in it (from its first stage-in kernel up to
the next admission or fill kernel), their busy time against the window,
per-kernel totals, and the idle gaps between consecutive kernels by kernel
pair -- the device time lost between the loop's launches.

    python3 tests/native/kernel_gaps.py <rocprofv3 output directory>
"""
from __future__ import annotations

import collections
import csv
import glob
import sys

ADMISSION = ("TableScatter", "PrefillSynthetic", "FinishPageUpload", "TableReserve", "fillBuffer")


def short(name: str) -> str:
    name = name.replace("void ", "").replace("(anonymous namespace)::", "")
    return name.split("(")[0].split("<")[0].replace("dsdk::", "")


def loop_window(kernels):
    """The kernels from the first StageInKernel to the next admission."""
    names = [k[2] for k in kernels]
    first = next(i for i, n in enumerate(names) if "StageIn" in n)
    last = next((i for i in range(first, len(names)) if any(a in names[i] for a in ADMISSION)),
                len(names))
    return kernels[first:last]


def summarize(kernels):
    span = kernels[-1][1] - kernels[0][0]
    busy = sum(e - s for s, e, _ in kernels)
    lines = [f"kernels {len(kernels)} window {span / 1e6:.3f} ms busy {busy / 1e6:.3f} ms "
             f"({busy / span:.2f})"]
    tot = collections.defaultdict(lambda: [0, 0])
    for s, e, n in kernels:
        tot[short(n)][0] += 1
        tot[short(n)][1] += e - s
    for n, (c, t) in sorted(tot.items(), key=lambda x: -x[1][1]):
        lines.append(f"  {n:28s} n={c:5d} total {t / 1e6:8.3f} ms avg {t / c / 1e3:8.2f} us")
    gaps = collections.defaultdict(list)
    for (_, e0, n0), (s1, _, n1) in zip(kernels, kernels[1:]):
        gaps[(short(n0), short(n1))].append(s1 - e0)
    lines.append("idle gaps between consecutive kernels (us): pair, count, mean, p50, p90, sum")
    for (a, b), g in sorted(gaps.items(), key=lambda x: -sum(x[1])):
        g = sorted(g)
        lines.append(f"  {a:26s} -> {b:26s} n={len(g):5d} mean {sum(g) / len(g) / 1e3:7.2f} "
                     f"p50 {g[len(g) // 2] / 1e3:7.2f} p90 {g[int(len(g) * 0.9)] / 1e3:7.2f} "
                     f"sum {sum(g) / 1e6:.3f} ms")
    return lines


def main(directory: str) -> int:
    paths = glob.glob(directory + "/**/*kernel_trace.csv", recursive=True)
    if not paths:
        print("no kernel trace under", directory)
        return 1
    rows = list(csv.DictReader(open(paths[0])))
    kernels = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"])
                     for r in rows)
    print("\n".join(summarize(loop_window(kernels))))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1]))
