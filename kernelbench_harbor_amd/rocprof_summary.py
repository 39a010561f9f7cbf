"""Summarises a ``rocprofv3 --kernel-trace -f csv`` trace per (kernel, grid, workgroup size), or
a ``rocprofv3 --pmc`` counter collection per op call.

    python -m kernelbench_harbor_amd.rocprof_summary <prefix>_kernel_trace.csv [--match SUBSTR]
        [--by-next SUBSTR]
    python -m kernelbench_harbor_amd.rocprof_summary <prefix>_counter_collection.csv \
        --match kbh:: --pmc-calls N

Launches of one kernel symbol with different grids (for example the W4A16 kernel at several
M) are reported separately, so the average duration of one configuration can be compared with
the HIP-event figure bench.py reports for it.
"""
from __future__ import annotations

import argparse
import csv
import statistics


def summarize(path: str, match: str | None = None, by_next: str | None = None) -> list[dict]:
    """Rows per (kernel, grid, workgroup size). With `by_next`, a launch is also keyed by the
    grid of the next launch (in dispatch order) whose name contains `by_next`: the split-K GEMM
    of one call is followed by its own reduce kernel, whose grid (one thread per 4 outputs)
    tells the calls' M apart when the GEMM grids coincide (W4A16 M=1024 and M=2048 both run
    256 workgroups)."""
    with open(path, newline="") as f:
        rows = [r for r in csv.DictReader(f) if not match or match in r["Kernel_Name"]]
    rows.sort(key=lambda r: (int(r["Start_Timestamp"]), int(r.get("Dispatch_Id") or 0)))
    groups: dict[tuple, list[float]] = {}
    for i, r in enumerate(rows):
        nxt = 0
        if by_next and by_next not in r["Kernel_Name"]:
            for q in rows[i + 1:]:
                if by_next in q["Kernel_Name"]:
                    nxt = int(q["Grid_Size_X"])
                    break
        key = (r["Kernel_Name"], int(r["Grid_Size_X"]), int(r.get("Grid_Size_Y") or 1),
               int(r["Workgroup_Size_X"]), nxt)
        dur_us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        groups.setdefault(key, []).append(dur_us)
    out = []
    for (name, gx, gy, wg, nxt), ds in groups.items():
        ds.sort()
        out.append({"kernel": name, "grid_threads": (gx, gy), "workgroup": wg, "calls": len(ds),
                    "next_grid": nxt, "avg_us": statistics.fmean(ds),
                    "median_us": ds[len(ds) // 2], "min_us": ds[0], "max_us": ds[-1]})
    return out


def counter_totals(path: str, match: str | None = None) -> dict[str, dict]:
    """Sums each counter of a ``rocprofv3 --pmc ... -f csv`` run over the dispatches of kernels
    whose name contains `match`: {counter: {"total": sum, "dispatches": n}}."""
    out: dict[str, dict] = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if match and match not in r["Kernel_Name"]:
                continue
            d = out.setdefault(r["Counter_Name"], {"total": 0.0, "dispatches": 0})
            d["total"] += float(r["Counter_Value"])
            d["dispatches"] += 1
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--match", default=None)
    ap.add_argument("--by-next", default=None, metavar="SUBSTR",
                    help="also split each kernel's rows by the grid of the next launch whose "
                         "name contains SUBSTR (e.g. wide_reduce: tells M=1024 and M=2048 apart)")
    ap.add_argument("--pmc-calls", type=int, default=0,
                    help="the file is a --pmc counter collection: print each counter's sum over "
                         "the matching dispatches divided by this many op calls")
    a = ap.parse_args()
    if a.pmc_calls:
        for name, d in counter_totals(a.trace, a.match).items():
            print(f"{name} {d['total'] / a.pmc_calls:.1f} per call ({d['dispatches']} dispatches)")
        return
    rows = summarize(a.trace, a.match, a.by_next)
    nx = bool(a.by_next)
    print("| kernel | grid (threads x,y) | wg |" + (" next grid |" if nx else "") +
          " calls | avg us | median us | min us | max us |")
    print("|---|---|---|" + ("---|" if nx else "") + "---|---|---|---|---|")
    for r in rows:
        short = (r["kernel"].replace("(anonymous namespace)::", "").replace("void ", "")
                 .replace("kbh::", ""))
        # drop the argument list: the last top-level "(...)" (template arguments may hold
        # parentheses, as in "float __vector(4)")
        depth, cut = 0, len(short)
        for i, ch in enumerate(short):
            depth += ch == "<"
            depth -= ch == ">"
            if ch == "(" and depth == 0:
                cut = i
                break
        short = short[:cut].rstrip()
        nxt = (f"{r['next_grid'] or ''} | " if nx else "")
        print(f"| `{short}` | {r['grid_threads'][0]}x{r['grid_threads'][1]} | {r['workgroup']} | "
              f"{nxt}{r['calls']} | {r['avg_us']:.2f} | {r['median_us']:.2f} | "
              f"{r['min_us']:.2f} | {r['max_us']:.2f} |")


if __name__ == "__main__":
    main()
