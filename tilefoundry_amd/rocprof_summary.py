"""Reduce rocprofv3 CSV output to the small summaries kept under profiles/.

    python -m tilefoundry_amd.rocprof_summary stats <dir>   # *kernel_stats.csv -> stats_summary.json
    python -m tilefoundry_amd.rocprof_summary pmc <dir>     # *counter_collection.csv -> pmc_summary.json
    python -m tilefoundry_amd.rocprof_summary traffic <fetch_dir> <write_dir> <kernel substring>
    python -m tilefoundry_amd.rocprof_summary table <dir> [rows] [regex]  # stats_summary.json -> markdown

``stats`` keeps per-kernel call counts and durations and deletes the raw kernel
trace (it can exceed what a run may copy back). ``pmc`` averages each counter
per kernel over its dispatches. ``traffic`` turns FETCH_SIZE / WRITE_SIZE
(KiB per dispatch) into bytes per launch of one kernel, each scaled by what the
same counter reads for ``copy_stream`` -- a copy of known size issued through
the same 16-byte load / store path -- and prints the JSON bench.py reads from
profiles/roofline_traffic.json.
"""
from __future__ import annotations

import csv
import glob
import json
import os
import re
import sys
from collections import defaultdict


def stats(d: str) -> None:
    f = glob.glob(os.path.join(d, "*kernel_stats.csv"))[0]
    out = []
    for r in csv.DictReader(open(f)):
        out.append({"name": r["Name"][:160], "calls": int(r["Calls"]),
                    "avg_us": float(r["AverageNs"]) / 1e3, "min_us": float(r["MinNs"]) / 1e3,
                    "max_us": float(r["MaxNs"]) / 1e3,
                    "total_ms": float(r["TotalDurationNs"]) / 1e6, "pct": float(r["Percentage"])})
    json.dump(out, open(os.path.join(d, "stats_summary.json"), "w"), indent=1)
    for p in glob.glob(os.path.join(d, "*kernel_trace.csv")):
        os.remove(p)


def pmc(d: str) -> None:
    f = glob.glob(os.path.join(d, "*counter_collection.csv"))[0]
    agg = defaultdict(list)
    for r in csv.DictReader(open(f)):
        agg[(r["Kernel_Name"][:120], r["Counter_Name"])].append(float(r["Counter_Value"]))
    out = [{"kernel": k[0], "counter": k[1], "dispatches": len(v), "avg": sum(v) / len(v),
            "min": min(v), "max": max(v)} for k, v in agg.items()]
    out.sort(key=lambda e: -e["avg"] * e["dispatches"])
    json.dump({"rows": out}, open(os.path.join(d, "pmc_summary.json"), "w"), indent=1)
    os.remove(f)


def _avg(d: str, counter: str, needle: str) -> float:
    rows = json.load(open(os.path.join(d, "pmc_summary.json")))["rows"]
    hits = [r for r in rows if r["counter"] == counter and needle in r["kernel"]]
    if not hits:
        raise SystemExit(f"no {counter} rows for kernels matching {needle!r} in {d}")
    return max(hits, key=lambda r: r["dispatches"])["avg"]


def traffic(fetch_dir: str, write_dir: str, needle: str, copy_bytes: int = 64 << 20) -> dict:
    kib = 1024.0
    f_k = _avg(fetch_dir, "FETCH_SIZE", needle)
    w_k = _avg(write_dir, "WRITE_SIZE", needle)
    f_c = _avg(fetch_dir, "FETCH_SIZE", "copy_stream_kernel")
    w_c = _avg(write_dir, "WRITE_SIZE", "copy_stream_kernel")
    ff, wf = copy_bytes / (f_c * kib), copy_bytes / (w_c * kib)
    return {"kernel": needle, "fetch_kib_per_dispatch": f_k, "write_kib_per_dispatch": w_k,
            "copy_bytes": copy_bytes, "copy_fetch_kib": f_c, "copy_write_kib": w_c,
            "fetch_factor": round(ff, 5), "write_factor": round(wf, 5),
            "traffic_bytes_per_launch": int(round(f_k * kib * ff + w_k * kib * wf))}


def table(d: str, rows: int = 16, match: str | None = None) -> str:
    """The busiest kernels of a ``stats`` summary (those whose name matches the
    regular expression ``match``, when given) as a markdown table."""
    data = json.load(open(os.path.join(d, "stats_summary.json")))
    if match:
        data = [r for r in data if re.search(match, r["name"])]
    lines = ["| kernel | calls | avg us | min us | max us | % time |", "|---|---:|---:|---:|---:|---:|"]
    for r in data[:rows]:
        name = r["name"].replace("|", "\\|")
        lines.append(f"| `{name[:110]}` | {r['calls']} | {r['avg_us']:.2f} | {r['min_us']:.2f} | "
                     f"{r['max_us']:.2f} | {r['pct']:.2f} |")
    return "\n".join(lines)


if __name__ == "__main__":
    mode = sys.argv[1]
    if mode == "stats":
        stats(sys.argv[2])
    elif mode == "pmc":
        pmc(sys.argv[2])
    elif mode == "table":
        print(table(sys.argv[2], int(sys.argv[3]) if len(sys.argv) > 3 else 16,
                    sys.argv[4] if len(sys.argv) > 4 else None))
    elif mode == "traffic":
        print(json.dumps(traffic(sys.argv[2], sys.argv[3], sys.argv[4]), indent=1))
    else:
        raise SystemExit(__doc__)
